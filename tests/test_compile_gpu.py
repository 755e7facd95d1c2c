"""The decoder step under torch.compile, as the reference runs it
(vflorence/engine/model_runner.py:102-126: torch.compile(model, dynamic=True) with
the attention ops opaque):

* the compiled engine's tokens equal transformers' fixtures (fp32), greedy and beam
  search, at the small test shape and at BART-large shape;
* a compiled step writes the paged caches in place: no operation other than the
  self-attention op itself touches a cache-shaped tensor and no copy moves a cache's
  bytes (the reference's TORCH_COMPILE_FREEZING.md:416-428 check: Inductor adds no
  cache copies for the mutating op);
* one dynamic graph serves every multi-row batch size: after the first generate no
  further graph is compiled (tests/test_parity.py:41-56).
"""

import json
import os

import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "token_fixtures.json")


def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


def engine(cfg_kwargs, checksum, **kwargs):
    from transformers import BartConfig

    from vflorence_amd import LLM
    from vflorence_amd.utils.loader import state_dict_checksum, synthetic_state_dict

    cfg = BartConfig(**cfg_kwargs)
    sd = synthetic_state_dict(cfg, seed=0, device="cuda")
    assert state_dict_checksum(sd) == checksum
    return LLM(cfg, state_dict=sd, compile=True, **kwargs)


def graphs() -> int:
    return torch._dynamo.utils.counters["stats"]["unique_graphs"]


@pytest.fixture(scope="module")
def small_compiled():
    torch._dynamo.reset()
    fx = fixtures()["small"]
    return engine(fx["config"], fx["checksum"], max_num_seqs=24, dtype=torch.float32,
                  max_decoder_len=32, max_encoder_len=128)


@pytest.mark.parametrize("case", ["greedy", "greedy_rules", "beam4_early", "beam4_rules"])
def test_compiled_tokens_match_transformers_small(small_compiled, case):
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    c = fx["cases"][case]
    outs = small_compiled.generate([Request(p) for p in fx["prompts"]],
                                   SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]


def test_one_dynamic_graph_serves_every_batch_size(small_compiled):
    """After a first generate has compiled the step, batches of other sizes (rows
    padded to the buckets 2, 4, 8, 16, 24) compile nothing new."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    params = SamplingParams(**fx["cases"]["greedy"]["params"])
    small_compiled.generate([Request(p) for p in fx["prompts"][:3]], params)
    warm = graphs()
    assert warm > 0
    for n in (2, 5, 6):
        small_compiled.generate([Request(p) for p in fx["prompts"][:n]], params)
    beam = SamplingParams(**fx["cases"]["beam4_early"]["params"])
    small_compiled.generate([Request(p) for p in fx["prompts"]], beam)  # 24 rows
    assert graphs() == warm, "a batch size compiled a graph of its own"
    breaks = dict(torch._dynamo.utils.counters["graph_break"])
    print(f"[compile] {warm} graphs, graph breaks: {breaks}", flush=True)


def test_compiled_bart_large_fp32_tokens():
    """BART-large shapes (12 decoder layers, 16 heads x 64), fp32, 8 requests with
    prompts of 128..1024 tokens, 64 greedy tokens each, compiled decoder step."""
    from vflorence_amd import Request, SamplingParams

    torch._dynamo.reset()
    fx = fixtures()["bart_large"]
    c = fx["cases"]["greedy64"]
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=8, dtype=torch.float32,
                 max_decoder_len=64, max_encoder_len=1024)
    outs = llm.generate([Request(p) for p in fx["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_compiled_step_writes_the_caches_in_place(dtype):
    """Profile one compiled decode step (after the compiling one): the only operation
    that receives a cache-shaped tensor is the self-attention op, and no copy or clone
    of a cache runs -- Inductor re-inplaces the op's declared mutation."""
    from torch.profiler import ProfilerActivity, profile

    from vflorence_amd import Request, SamplingParams

    torch._dynamo.reset()
    fx = fixtures()["small"]
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=24, dtype=dtype,
                 max_decoder_len=32, max_encoder_len=128)
    params = SamplingParams(**{**fx["cases"]["greedy"]["params"], "max_tokens": 8,
                               "min_length": 9})
    for p in fx["prompts"]:
        llm.add_request(Request(p), params)
    with torch.inference_mode():
        llm.step()
        llm.step()  # compiled and warm
        cache = llm.runner.decoder_layers[0].self_attn.k_cache
        shape = list(cache.shape)
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA],
                     record_shapes=True) as prof:
            llm.step()
            torch.cuda.synchronize()
    touching = {e.name for e in prof.events() if shape in [list(s) for s in e.input_shapes]}
    assert "vflorence::self_attention" in touching, touching
    assert all(n.startswith("vflorence::") for n in touching), touching
    llm.abort()


def test_compiled_deferred_layer_norm_steps_equal_eager_steps():
    """bf16 at a width the decode-step kernels serve (d_model 256, ffn 1024): the decoder
    runs with deferred LayerNorms (linear_residual / linear_norm / layer_norm_apply), and
    the compiled step -- one graph, the custom ops opaque -- gives the eager step's tokens."""
    from transformers import BartConfig

    from vflorence_amd import LLM, Request, SamplingParams
    from vflorence_amd.utils.loader import synthetic_state_dict

    cfg = BartConfig(vocab_size=512, d_model=256, encoder_layers=1, decoder_layers=2,
                     encoder_attention_heads=4, decoder_attention_heads=4,
                     encoder_ffn_dim=1024, decoder_ffn_dim=1024, max_position_embeddings=256,
                     bos_token_id=0, pad_token_id=1, eos_token_id=2, decoder_start_token_id=2,
                     forced_eos_token_id=None, tie_word_embeddings=False)
    prompts = [[0] + [5 + (7 * i + 3 * r) % 500 for i in range(40 + 9 * r)] + [2]
               for r in range(6)]
    params = SamplingParams(max_tokens=12, num_beams=2, repetition_penalty=1.0,
                            eos_token_id=[2], length_penalty=1.0, no_repeat_ngram_size=0,
                            min_length=13, forced_bos_token_id=None, forced_eos_token_id=None,
                            suppress_tokens=[], begin_suppress_tokens=[], early_stopping=True)
    got = []
    for compiled in (False, True):
        torch._dynamo.reset()
        before = graphs()
        sd = synthetic_state_dict(cfg, seed=1, device="cuda")
        llm = LLM(cfg, state_dict=sd, compile=compiled, dtype=torch.bfloat16, max_num_seqs=16,
                  max_decoder_len=32, max_encoder_len=128)
        dec = llm.runner.model.model.decoder
        assert dec.deferred_norms
        got.append([o.completion_token_ids
                    for o in llm.generate([Request(p) for p in prompts], params)])
        if compiled:  # one graph for every step and batch size (counters are per process)
            assert graphs() - before == 1, graphs() - before
    assert got[0] == got[1]
    assert all(len(t) == 12 for t in got[0])
