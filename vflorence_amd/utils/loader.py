"""Model construction: checkpoint weights, or a synthetic checkpoint made on any device.

``load_model`` mirrors vflorence/utils/loader.py:24-50: a transformers BART
checkpoint is read in fp32 through transformers (missing, unexpected or mismatched
keys are an error), its q/k/v projections are concatenated into the fused ones, and
the model is moved to the engine's device and dtype.

``synthetic_state_dict`` is a checkpoint in transformers' naming whose every value is
a function of (seed, parameter name, element index) only -- a 32-bit integer hash
mapped to a uniform value -- computed with integer and float64 operations that round
identically on the CPU and the GPU.  The same weights therefore load into
transformers' BART on the host and into this model on the device, which is what the
token-parity tests need; ``state_dict_checksum`` proves two copies are identical.
"""

from __future__ import annotations

import zlib

import torch

_MASK32 = 0xFFFFFFFF


def _mulmod32(x: torch.Tensor, c: int) -> torch.Tensor:
    """``x * c mod 2^32`` for int64 ``x`` in [0, 2^32), in 16-bit halves of ``c`` so no
    intermediate leaves the int64 range."""
    lo = x * (c & 0xFFFF)
    hi = ((x * (c >> 16)) & 0xFFFF) << 16
    return (lo + hi) & _MASK32


def _mix32(x: torch.Tensor) -> torch.Tensor:
    """murmur3's 32-bit finaliser on int64 tensors holding values in [0, 2^32)."""
    x = x ^ (x >> 16)
    x = _mulmod32(x, 0x85EBCA6B)
    x = x ^ (x >> 13)
    x = _mulmod32(x, 0xC2B2AE35)
    return x ^ (x >> 16)


def _hashed_uniform(shape, key: int, seed: int, lo: float, hi: float, device, dtype):
    """Elements ``lo + (hi - lo) * u`` with ``u = mix32(index, key, seed) / 2^32``."""
    n = 1
    for s in shape:
        n *= s
    out = torch.empty(n, dtype=dtype, device=device)
    chunk = 1 << 24
    base = (key * 0x9E3779B1 + seed * 0x7F4A7C15) & _MASK32
    for start in range(0, n, chunk):
        idx = torch.arange(start, min(n, start + chunk), dtype=torch.int64, device=device)
        x = _mix32((_mulmod32(idx & _MASK32, 0x27D4EB2F) + base) & _MASK32)
        u = x.to(torch.float64) * (1.0 / 4294967296.0)
        out[start:start + idx.numel()] = (lo + (hi - lo) * u).to(dtype)
    return out.view(shape)


def _canonical(name: str, tied: bool) -> str:
    """The parameter whose values ``name`` takes: BART's encoder and decoder token
    embeddings are the shared embedding; the LM head is too when tied."""
    if name.endswith("embed_tokens.weight") or (tied and name == "lm_head.weight"):
        return "model.shared.weight"
    return name


def synthetic_state_dict(hf_config, seed: int = 0, device="cpu", std: float = 0.02,
                         dtype=torch.float32) -> dict:
    """A BART checkpoint (transformers' parameter names and shapes) of hashed values.

    Matrices and embeddings are uniform with standard deviation ``std``; biases and
    ``final_logits_bias`` uniform with ``std / 2``; LayerNorm weights in
    ``1 +- std`` (all non-zero, so a dropped bias or a mis-ordered fused projection
    changes the tokens).  The token embeddings of encoder and decoder share the
    shared embedding's values, and so does the LM head when the config ties it.
    """
    import transformers

    with torch.device("meta"):
        shapes = {k: tuple(v.shape) for k, v in
                  transformers.BartForConditionalGeneration(hf_config).state_dict().items()}
    tied = bool(getattr(hf_config, "tie_word_embeddings", True))
    half = std * 3**0.5  # half-width of a uniform with this std
    made: dict[str, torch.Tensor] = {}
    out = {}
    for name, shape in shapes.items():
        canon = _canonical(name, tied)
        if canon not in made:
            key = zlib.crc32(canon.encode())
            if "layer_norm" in canon or "layernorm" in canon:
                if canon.endswith(".weight"):
                    t = _hashed_uniform(shape, key, seed, 1 - std, 1 + std, device, dtype)
                else:
                    t = _hashed_uniform(shape, key, seed, -half / 2, half / 2, device, dtype)
            elif canon.endswith(".bias") or canon == "final_logits_bias":
                t = _hashed_uniform(shape, key, seed, -half / 2, half / 2, device, dtype)
            else:
                t = _hashed_uniform(shape, key, seed, -half, half, device, dtype)
            made[canon] = t
        out[name] = made[canon]
    return out


def state_dict_checksum(state_dict: dict) -> int:
    """Order-independent integer checksum of the exact bits of every tensor."""
    total = 0
    for name in sorted(state_dict):
        t = state_dict[name].detach().contiguous().view(-1)
        bits = t.view(torch.int32 if t.element_size() == 4 else torch.int16).to(torch.int64)
        weights = torch.arange(1, bits.numel() + 1, dtype=torch.int64, device=bits.device) % 65521
        total = (total * 1000003 + int((bits * (weights + 1)).sum().item())
                 + zlib.crc32(name.encode())) & ((1 << 62) - 1)
    return total


def load_model(config, state_dict: dict | None = None):
    """The engine's BART on ``config.device`` in ``config.dtype``, eval mode.

    ``state_dict`` (transformers naming, any device) overrides reading
    ``config.model``; an in-memory config without one gets ``synthetic_state_dict``.
    """
    from transformers import PretrainedConfig

    from ..layers.bart import BartForConditionalGeneration, fuse_projections

    hf = config.hf_config
    if hf.model_type != "bart":
        raise ValueError(f"unsupported model_type: {hf.model_type!r}")
    if state_dict is None:
        if isinstance(config.model, PretrainedConfig):
            state_dict = synthetic_state_dict(hf, device=config.device)
        else:
            import transformers

            hf_model, info = transformers.BartForConditionalGeneration.from_pretrained(
                config.model, dtype=torch.float32, output_loading_info=True,
                local_files_only=True)
            errors = {k: info[k] for k in ("missing_keys", "unexpected_keys", "mismatched_keys",
                                           "error_msgs") if info.get(k)}
            if errors:
                raise RuntimeError(f"incompatible checkpoint: {errors}")
            state_dict = hf_model.state_dict()
    state_dict = dict(state_dict)
    with torch.device(config.device):
        model = BartForConditionalGeneration(hf).to(config.dtype)
    fuse_projections(model, state_dict)
    model.load_state_dict(state_dict, strict=True)
    repack_decode_weights(model)
    return model.eval()


def repack_decode_weights(model) -> None:
    """Refresh every decode-step projection's packed weight copy and the LM head's
    padded operands in place (after loading or updating weights; captured HIP graphs
    read the refreshed copies)."""
    from ..layers.bart import DecodeLinear

    for module in model.modules():
        if isinstance(module, DecodeLinear):
            module.repack()
    if hasattr(model, "repack_lm_head"):
        model.repack_lm_head()
