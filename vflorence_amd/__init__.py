"""MI355X (gfx950) decode-step attention path for vflorence.

Submodules:
    hip_attn          -- torch wrappers of the C ABI (counterpart of vllm_cpu_attn)
    layers.attention  -- vflorence::self_attention / vflorence::cross_attention ops
    utils.context     -- per-step Context read by the ops
    engine            -- block manager, scheduler, runner harness
    models.bart       -- BART decoder callers of the ops
"""

__version__ = "0.1.0"
