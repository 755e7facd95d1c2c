"""The engine on the GPU: tokens equal transformers' (fp32, greedy and beam search),
the runner's step metadata and encoder paging follow the reference's formulas, and
every block and encoder page returns to its pool after a run or a failed step."""

import json
import math
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "token_fixtures.json")


def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


def engine(cfg_kwargs, checksum, eos_bias: float = 0.0, **kwargs):
    from transformers import BartConfig

    from vflorence_amd import LLM
    from vflorence_amd.utils.loader import state_dict_checksum, synthetic_state_dict

    cfg = BartConfig(**cfg_kwargs)
    sd = synthetic_state_dict(cfg, seed=0, device="cuda")
    if eos_bias:  # the fixture's reachable-EOS checkpoint (one fp32 add)
        flb = sd["final_logits_bias"].clone()
        flb[0, cfg.eos_token_id] += eos_bias
        sd["final_logits_bias"] = flb
    assert state_dict_checksum(sd) == checksum, "GPU-made weights differ from the fixture's"
    return LLM(cfg, state_dict=sd, **kwargs)


def assert_clean(llm):
    bm = llm.scheduler.block_manager
    assert llm.is_finished()
    assert bm.num_free_blocks == bm.num_blocks and not any(bm.ref_counts)
    assert llm.scheduler.num_pending_beams == 0 and not llm.scheduler.waiting
    runner = llm.runner
    assert not runner._cross_pages
    assert sorted(runner._cross_free) == list(range(llm.config.num_cross_blocks))
    assert runner._cross_staged is None


SMALL_CASES = ["greedy", "greedy_rules", "greedy_forced", "beam2", "beam4_early", "beam4_rules"]


@pytest.fixture(scope="module", params=[False, True], ids=["eager", "hipgraph"])
def small_engine(request):
    fx = fixtures()["small"]
    return engine(fx["config"], fx["checksum"], max_num_seqs=24, dtype=torch.float32,
                  max_decoder_len=32, max_encoder_len=128, cuda_graphs=request.param)


@pytest.mark.parametrize("case", SMALL_CASES)
def test_tokens_match_transformers_small_bart(small_engine, case):
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    c = fx["cases"][case]
    # every near-tie in the fixture is far above fp32 noise
    assert all(g is None or g > 1e-4 for g in c["min_gap"])
    outs = small_engine.generate([Request(p) for p in fx["prompts"]], SamplingParams(**c["params"]))
    got = [o.completion_token_ids for o in outs]
    assert got == c["tokens"]
    assert_clean(small_engine)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "hipgraph"])
def test_tokens_match_transformers_bart_large_fp32(graphs):
    """BART-large shapes (12+12 layers, 16 heads x 64, vocab 50265), fp32, 8 requests
    with encoder prompts of 128..1024 tokens, 64 greedy tokens each, batched."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["bart_large"]
    c = fx["cases"]["greedy64"]
    assert all(g > 1e-4 for g in c["min_gap"])
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=8, dtype=torch.float32,
                 max_decoder_len=64, max_encoder_len=1024, cuda_graphs=graphs)
    outs = llm.generate([Request(p) for p in fx["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]
    assert_clean(llm)


BEAM_CASES = {  # fixture, case, engine limits
    "bart_large_beam4": ("bart_large", "beam4", dict(max_num_seqs=32, max_decoder_len=24,
                                                      max_encoder_len=1024)),
    "bart_large_beam4_fused": ("bart_large", "beam4_fused",
                               dict(max_num_seqs=32, max_decoder_len=24, max_encoder_len=1024)),
    "florence2_base_beam3": ("florence2_base", "beam3",
                             dict(max_num_seqs=18, max_decoder_len=32, max_encoder_len=587)),
}


EOS_CASES = {  # reachable EOS: fixture, case, engine limits
    "bart_large_beam4_eos": ("bart_large_eos", "beam4_eos",
                             dict(max_num_seqs=32, max_decoder_len=24, max_encoder_len=1024)),
    "bart_large_beam4_eos_early": ("bart_large_eos", "beam4_eos_early",
                                   dict(max_num_seqs=32, max_decoder_len=24,
                                        max_encoder_len=1024)),
    "florence2_base_beam3_eos": ("florence2_base_eos", "beam3_eos",
                                 dict(max_num_seqs=18, max_decoder_len=32, max_encoder_len=587)),
    "florence2_base_beam3_eos_early": ("florence2_base_eos", "beam3_eos_early",
                                       dict(max_num_seqs=18, max_decoder_len=32,
                                            max_encoder_len=587)),
}


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "hipgraph"])
@pytest.mark.parametrize("name", list(EOS_CASES))
def test_beam_tokens_with_reachable_eos_match_transformers_fp32(name, graphs):
    """Beam search at the real model shapes with EOS reachable (an EOS logit bias and
    min_length 4, the reference's early-stopping check, tests/test_parity.py:88-122):
    hypotheses end at different steps, so the EOS rank gate, the length-normalised
    scores of finished hypotheses and both early-stopping rules decide the outputs.
    fp32, batched, against transformers' generate() one request at a time; token-exact.
    The fixture's outputs end at several lengths, and the two early-stopping rules give
    different outputs for some requests."""
    from vflorence_amd import Request, SamplingParams

    fixture, case, limits = EOS_CASES[name]
    fx = fixtures()[fixture]
    c = fx["cases"][case]
    assert all(g >= 1e-4 for g in c["min_gap"])  # no decisive step within fp32 rounding
    assert len({len(t) for t in c["tokens"]}) > 1  # hypotheses end at different steps
    llm = engine(fx["config"], fx["checksum"], eos_bias=fx["eos_bias"], dtype=torch.float32,
                 cuda_graphs=graphs, **limits)
    outs = llm.generate([Request(p) for p in c["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]
    assert_clean(llm)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "hipgraph"])
@pytest.mark.parametrize("name", list(BEAM_CASES))
def test_beam_tokens_match_transformers_fp32(name, graphs):
    """Beam search at the real model shapes, fp32, batched, against transformers'
    generate() one request at a time (tests/verify_parity.py:70-108,177 settings):
    BART-large with 4 beams (length penalty 2, no repeated 3-grams -- the torch rule
    path -- or without it -- the fused top-k kernel path), EOS suppressed, 24 tokens;
    Florence-2-base shapes with 3 beams, 587 encoder tokens, 32 tokens.  Token-exact."""
    from vflorence_amd import Request, SamplingParams

    fixture, case, limits = BEAM_CASES[name]
    fx = fixtures()[fixture]
    c = fx["cases"][case]
    assert all(g >= 1e-4 for g in c["min_gap"])  # no decisive step within fp32 rounding
    llm = engine(fx["config"], fx["checksum"], dtype=torch.float32, cuda_graphs=graphs,
                 **limits)
    outs = llm.generate([Request(p) for p in c["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]
    assert_clean(llm)


# Eight rounding steps of a bf16 logit in [4, 8): no decision with an fp32 margin this
# large may come out differently in bf16.
BF16_FLIP_MARGIN = 0.25


def first_difference(a, b):
    n = min(len(a), len(b))
    return next((i for i in range(n) if a[i] != b[i]), None if len(a) == len(b) else n)


@pytest.mark.parametrize("name", list(BEAM_CASES))
def test_beam_tokens_bf16_against_the_fp32_fixture(name):
    """The same beam cases in bf16 with HIP graphs against transformers' fp32 run: every
    request returns as many tokens (the reference's bf16 bar,
    tests/verify_parity.py:59-67), and where the tokens part, some decision up to the
    first differing position had an fp32 decisive margin below BF16_FLIP_MARGIN.  The
    whole decoder runs in bf16 here (weights, GEMMs, LayerNorms, attention), which moves
    candidate scores by a few rounding steps of the bf16 logits (2^-5 each in [4, 8));
    tests/test_attention_ab_gpu.py isolates the attention ops' share."""
    from vflorence_amd import Request, SamplingParams

    fixture, case, limits = BEAM_CASES[name]
    fx = fixtures()[fixture]
    c = fx["cases"][case]
    llm = engine(fx["config"], fx["checksum"], dtype=torch.bfloat16, cuda_graphs=True,
                 **limits)
    outs = llm.generate([Request(p) for p in c["prompts"]], SamplingParams(**c["params"]))
    got = [o.completion_token_ids for o in outs]
    report = []
    for r, (a, b) in enumerate(zip(got, c["tokens"])):
        assert len(a) == len(b), f"request {r}: {len(a)} tokens against {len(b)}"
        first = first_difference(a, b)
        if first is not None:
            # the diverging decision came at or before the first differing position
            smallest = min(g for g in c["gaps"][r][: first + 1] if g is not None)
            report.append(f"request {r}: first difference at step {first}, fp32 margin "
                          f"there {c['gaps'][r][first]:.2e}, smallest up to it {smallest:.2e}")
            assert smallest < BF16_FLIP_MARGIN, report[-1]
    same = sum(a == b for a, b in zip(got, c["tokens"]))
    print(f"[bf16 beam parity] {name}: {same}/{len(got)} requests token-identical to the "
          f"fp32 fixture; " + ("; ".join(report) if report else "no differences"), flush=True)
    assert_clean(llm)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_16bit_hip_graph_steps_equal_eager_steps(dtype):
    """bf16 / fp16 beam search: replayed decode steps give the same tokens as eager ones
    (every replay reads fresh metadata from the fixed buffers)."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    params = SamplingParams(**fx["cases"]["beam4_early"]["params"])
    got = []
    for graphs in (False, True):
        llm = engine(fx["config"], fx["checksum"], max_num_seqs=24, dtype=dtype,
                     max_decoder_len=32, max_encoder_len=128, cuda_graphs=graphs)
        outs = llm.generate([Request(p) for p in fx["prompts"]], params)
        assert all(1 <= len(o.completion_token_ids) <= params.max_tokens for o in outs)
        assert_clean(llm)
        # a second batch in a different composition reuses the captured sizes
        outs2 = llm.generate([Request(p) for p in fx["prompts"][::-1]], params)
        got.append(([o.completion_token_ids for o in outs], [o.completion_token_ids
                                                            for o in outs2]))
        assert_clean(llm)
    assert got[0] == got[1]


def test_prepare_and_encode_follow_the_reference_formulas(small_engine):
    """Slots, context lengths, tables and positions of one step
    (model_runner.py:294-305) read back from HBM against the formulas applied to the
    host core's rows, and the paged encoder K/V (:236-259).  Three requests join at
    different steps, so their rows hold different numbers of cached tokens."""
    from vflorence_amd import SamplingParams, hip_attn
    from vflorence_amd.engine.sequence import Sequence
    from vflorence_amd.utils.context import get_context, set_context

    llm = small_engine
    runner, sched = llm.runner, llm.scheduler
    params = SamplingParams(max_tokens=30).with_defaults(llm._sampling_params)
    fx = fixtures()["small"]
    joins = {0: 0, 5: 1, 17: 2}
    seqs = []
    with torch.inference_mode():
        for step in range(21):
            if step in joins:
                i = joins[step]
                seqs.append(Sequence(i, [2], fx["prompts"][i], params))
                sched.add(seqs[-1])
            batch = sched.schedule()
            if batch.fresh:
                runner._encode(batch.fresh)
            # tokens decided on the host: no decoder step needed to advance the rows
            sched.postprocess(batch, np.full(batch.num_rows, 10 + step, np.int64))
        batch = sched.schedule()
        rows = sched.running
        assert [r.num_cached_tokens for r in rows] == [21, 16, 4]
        ids, pos = runner._prepare(batch)
        ctx = get_context()
        # three rows padded to the 4-row bucket: the padding row feeds token 0 at
        # position 0, has an empty context and writes no slot
        assert pos.shape[0] == ids.shape[0] == ctx.context_lens.shape[0] == 4
        want_pos = [r.num_cached_tokens for r in rows]
        assert pos.tolist() == want_pos + [0]
        assert ids.tolist() == [r.token_ids[p] for r, p in zip(rows, want_pos)] + [0]
        assert ctx.context_lens.tolist() == [p + 1 for p in want_pos] + [0]
        assert ctx.slot_mapping.tolist() == [r.block_table[p // 16] * 16 + p % 16
                                             for r, p in zip(rows, want_pos)] + [-1]
        # 0-padded rows at the runner's fixed table width (the kernels read only
        # ceil(len / 16) entries of a row)
        width = ctx.block_tables.shape[1]
        assert width >= max(len(r.block_table) for r in rows)
        assert ctx.block_tables.tolist() == [r.block_table + [0] * (width - len(r.block_table))
                                             for r in rows] + [[0] * width]
        assert ctx.query_start_loc.tolist() == list(range(5))
        set_context()
        # encoder pages: request i's tokens at pages[t // 16] * 16 + t % 16 hold kv_proj;
        # bit for bit when the prompt ran eagerly on its own, within fp32 rounding when it
        # ran in a captured graph padded to a 256-token bucket (other GEMM row counts)
        layer = runner.decoder_layers[1]
        attn = layer.encoder_attn
        tol = 0 if runner._encoder_graphs is None else 1e-5
        for seq in seqs:
            pages, enc_len = runner._cross_pages[seq.request_id]
            assert enc_len == len(seq.encoder_token_ids) and len(pages) == math.ceil(enc_len / 16)
            hidden = runner.model.encode(torch.tensor([seq.encoder_token_ids], device="cuda"))
            k, v = attn.kv_proj(hidden)[0].chunk(2, dim=-1)
            t = torch.arange(enc_len)
            blk, off = pages[t // 16].long().cuda(), (t % 16).cuda()
            kc = attn.k_cache[blk, :, off, :]
            vc = hip_attn.v_cache_logical(attn.v_cache)[blk, :, off, :]
            torch.testing.assert_close(kc, k.view(enc_len, attn.num_heads, -1), rtol=tol,
                                       atol=tol)
            torch.testing.assert_close(vc, v.view(enc_len, attn.num_heads, -1), rtol=tol,
                                       atol=tol)
    llm.abort()
    assert_clean(llm)


def test_packed_encode_pages_every_prompt(small_engine):
    """Prompts of several lengths admitted in one step are encoded in one forward
    (equal lengths as one attention batch): every prompt's paged K/V equals its own
    encoder forward's kv_proj, and its pages come from the end of the free list group by
    group in first-seen length order (model_runner.py:169-177, 208-259)."""
    from vflorence_amd import SamplingParams, hip_attn
    from vflorence_amd.engine.sequence import Sequence

    llm = small_engine
    runner, sched = llm.runner, llm.scheduler
    params = SamplingParams(max_tokens=4).with_defaults(llm._sampling_params)
    p = fixtures()["small"]["prompts"]
    prompts = [p[1], p[3], p[0], p[1], p[5], p[3], p[4], p[1]]  # 17, 33, 5, 17, 100, ...
    free_before = list(runner._cross_free)
    with torch.inference_mode():
        seqs = [Sequence(i, [2], q, params) for i, q in enumerate(prompts)]
        for seq in seqs:
            sched.add(seq)
        batch = sched.schedule()
        assert len(batch.fresh) == len(prompts)
        runner._encode(batch.fresh)
        torch.cuda.synchronize()
        # pages: the groups (17 x3, 33 x2, 5, 100, 64) take the free list's tail in turn
        free, want_pages = list(free_before), {}
        for length in (17, 33, 5, 100, 64):
            group = [s for s in seqs if len(s.encoder_token_ids) == length]
            n = math.ceil(length / 16)
            taken = free[-n * len(group):]
            del free[-n * len(group):]
            for j, seq in enumerate(group):
                want_pages[seq.request_id] = taken[j * n: (j + 1) * n]
        assert runner._cross_free == free
        for seq in seqs:
            assert runner._cross_pages[seq.request_id][0].tolist() == want_pages[seq.request_id]
        assert_pages_hold_kv(runner, seqs)
    llm.abort()
    assert_clean(llm)


def assert_pages_hold_kv(runner, seqs):
    """Every prompt's encoder pages hold its own encoder forward's kv_proj (first and last
    decoder layer): the packed forward runs 100-300 tokens at once (padded to a bucket
    under HIP graphs) against one prompt at a time here, so the GEMMs' row counts and
    with them the fp32 rounding may differ."""
    from vflorence_amd import hip_attn

    for layer in (runner.decoder_layers[0], runner.decoder_layers[-1]):
        attn = layer.encoder_attn
        for seq in seqs:
            pages, enc_len = runner._cross_pages[seq.request_id]
            hidden = runner.model.encode(torch.tensor([seq.encoder_token_ids], device="cuda"))
            k, v = attn.kv_proj(hidden)[0].chunk(2, dim=-1)
            t = torch.arange(enc_len)
            blk, off = pages[t // 16].long().cuda(), (t % 16).cuda()
            kc = attn.k_cache[blk, :, off, :]
            vc = hip_attn.v_cache_logical(attn.v_cache)[blk, :, off, :]
            torch.testing.assert_close(kc, k.view(enc_len, attn.num_heads, -1), rtol=1e-5,
                                       atol=1e-5)
            torch.testing.assert_close(vc, v.view(enc_len, attn.num_heads, -1), rtol=1e-5,
                                       atol=1e-5)


def test_encoder_graphs_replay_with_new_prompts_and_fall_back_past_the_buckets(small_engine):
    """Under HIP graphs the packed encoder runs as captured graphs per token bucket with
    each layer's attention between them: two batches of different prompts in one bucket
    (the second replays the first's graphs, with eager work and synchronisations in
    between) and a batch past the largest bucket (eager) all page their own encoder
    outputs.  Without graphs the same batches run eagerly."""
    from vflorence_amd import SamplingParams
    from vflorence_amd.engine.encoder_graphs import token_bucket
    from vflorence_amd.engine.sequence import Sequence

    llm = small_engine
    runner, sched = llm.runner, llm.scheduler
    graphs = runner._encoder_graphs
    params = SamplingParams(max_tokens=4).with_defaults(llm._sampling_params)
    p = fixtures()["small"]["prompts"]  # 5, 17, 16, 33, 64 and 100 tokens
    batches = [[p[1], p[3], p[0], p[1], p[5]], [p[4], p[4], p[2], p[3]],
               [p[5], p[4], p[3], p[5]]]
    assert token_bucket(sum(map(len, batches[0])), 8192) == token_bucket(
        sum(map(len, batches[1])), 8192) == 256
    rid = 100
    try:
        with torch.inference_mode():
            for i, prompts in enumerate(batches):
                if graphs is not None and i == 2:
                    graphs.max_tokens = 200  # 297 tokens: past it, eagerly
                seqs = [Sequence(rid + j, [2], q, params) for j, q in enumerate(prompts)]
                rid += len(prompts)
                for seq in seqs:
                    sched.add(seq)
                batch = sched.schedule()
                runner._encode(batch.fresh)
                torch.cuda.synchronize()
                assert_pages_hold_kv(runner, seqs)
        if graphs is not None:
            assert 256 in graphs._buckets
            assert len(graphs._buckets[256].graphs) == len(runner.model.model.encoder.layers) + 1
    finally:
        if graphs is not None:
            graphs.max_tokens = 8192
    llm.abort()
    assert_clean(llm)
    # new pools: the captured steps and encoder graphs that wrote the old ones are dropped,
    # and the engine decodes the fixture's tokens again
    runner.allocate_kv_cache()
    assert not runner._graphs and (graphs is None or not graphs._buckets)
    fx = fixtures()["small"]
    c = fx["cases"]["greedy"]
    from vflorence_amd import Request

    outs = llm.generate([Request(q) for q in fx["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]
    assert_clean(llm)


def test_failed_step_releases_everything(small_engine):
    from vflorence_amd import Request, SamplingParams

    llm = small_engine
    runner = llm.runner
    fx = fixtures()["small"]
    calls = []
    original = runner._sample

    def failing(*args):
        calls.append(1)
        if len(calls) == 3:
            raise RuntimeError("decode failed")
        return original(*args)

    runner._sample = failing
    try:
        with pytest.raises(RuntimeError, match="decode failed"):
            llm.generate([Request(p) for p in fx["prompts"][:3]],
                         SamplingParams(max_tokens=8, num_beams=2))
    finally:
        del runner._sample
    assert_clean(llm)
    from vflorence_amd.utils.context import get_context

    assert get_context().cross_staged is None
    # and the engine still works
    outs = llm.generate([Request(fx["prompts"][0])], SamplingParams(max_tokens=4))
    assert len(outs[0].completion_token_ids) >= 1
    assert_clean(llm)


def test_rejected_request_returns_empty_and_others_run(small_engine):
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    too_long = Request(list(range(3, 3 + 200)))
    outs = small_engine.generate([Request(fx["prompts"][0]), too_long],
                                 SamplingParams(max_tokens=4))
    assert len(outs[0].completion_token_ids) >= 1 and outs[1].completion_token_ids == []
    assert_clean(small_engine)
    with pytest.raises(ValueError):
        small_engine.add_request(Request([5]), SamplingParams(max_tokens=33))
    np.testing.assert_equal(small_engine.is_finished(), True)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "hipgraph"])
def test_continuous_batching_keeps_each_requests_tokens(graphs):
    """Requests arrive at seeded Poisson times and leave when done, so the batch (and its
    cross-attention staging) changes from step to step; every completion still equals
    transformers' output for its prompt alone."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["small"]
    c = fx["cases"]["greedy"]
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=8, dtype=torch.float32,
                 max_decoder_len=32, max_encoder_len=128, cuda_graphs=graphs)
    rng = np.random.default_rng(0)
    arrive = np.cumsum(rng.poisson(1.5, size=30)).tolist()
    which = rng.integers(0, len(fx["prompts"]), size=30).tolist()
    params = SamplingParams(**c["params"])
    prompt_of, done, step = {}, {}, 0
    pending = list(zip(arrive, which))
    sizes = set()
    while pending or not llm.is_finished():
        while pending and pending[0][0] <= step:
            _, i = pending.pop(0)
            prompt_of[llm.add_request(Request(fx["prompts"][i]), params)] = i
        if not llm.is_finished():
            for rid, out in llm.step():
                done[rid] = out.completion_token_ids
            sizes.add(llm.scheduler.num_running)
        step += 1
    assert len(done) == 30 and len(sizes) > 3
    for rid, tokens in done.items():
        assert tokens == c["tokens"][prompt_of[rid]], rid
    if graphs:  # steps are padded to the row buckets 1, 2, 4, 8: one capture each at most
        assert len(llm.runner._graphs) <= 4
    assert_clean(llm)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "hipgraph"])
def test_tokens_match_transformers_florence2_base_shape_fp32(graphs):
    """Florence-2-base text-model shapes (6+6 layers, 12 heads x 64, vocab 51289), fp32,
    six requests reading 587 encoder tokens (577 visual + 10 prompt tokens in Florence-2),
    32 greedy tokens each, batched."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["florence2_base"]
    c = fx["cases"]["greedy32"]
    assert all(g > 1e-4 for g in c["min_gap"])
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=6, dtype=torch.float32,
                 max_decoder_len=32, max_encoder_len=587, cuda_graphs=graphs)
    outs = llm.generate([Request(p) for p in fx["prompts"]], SamplingParams(**c["params"]))
    assert [o.completion_token_ids for o in outs] == c["tokens"]
    assert_clean(llm)


def test_florence2_base_shape_3beam_bf16_hip_graph_equals_eager():
    """The Florence-2-base workload shape in bf16 with 3 beams: 18 rows in beam groups of
    three (padded to the 24-row bucket), cross-attention groups of three over 587 encoder
    tokens; graph replays give the tokens of eager steps."""
    from vflorence_amd import Request, SamplingParams

    fx = fixtures()["florence2_base"]
    params = SamplingParams(max_tokens=24, num_beams=3, eos_token_id=[2], length_penalty=1.0,
                            early_stopping=False, min_length=0, repetition_penalty=1.0,
                            no_repeat_ngram_size=0)
    got = []
    for graphs in (False, True):
        llm = engine(fx["config"], fx["checksum"], max_num_seqs=18, dtype=torch.bfloat16,
                     max_decoder_len=32, max_encoder_len=587, cuda_graphs=graphs)
        outs = llm.generate([Request(p) for p in fx["prompts"]], params)
        assert all(1 <= len(o.completion_token_ids) <= 24 for o in outs)
        got.append([o.completion_token_ids for o in outs])
        assert_clean(llm)
    assert got[0] == got[1]


def test_continuous_batching_stress_florence2_large_shape():
    """The continuous-batching stress workload's shape: Florence-2-large text decoder
    (12+12 layers, d_model 1024, 16 heads, vocab 51289), bf16, up to 512 running
    sequences, requests arriving as a seeded Poisson process with encoder lengths from a
    50/50 mix of 587 and U[64, 1024] and output lengths geometric (mean 96, cap 256).
    Active requests share one SamplingParams (the reference requires it,
    vflorence/engine/llm_engine.py:147), so each request is retired at its drawn length
    by cancelling it (``abort_request``: blocks and encoder pages released).  The batch
    changes size from step to step, the graphs stay within the row buckets, every row
    gets one token per step, and every block and page returns."""
    from transformers import BartConfig

    from vflorence_amd import LLM, Request, SamplingParams
    from vflorence_amd.engine.model_runner import row_buckets

    cfg = BartConfig(vocab_size=51289, max_position_embeddings=1024, forced_eos_token_id=None,
                     tie_word_embeddings=False)
    llm = LLM(cfg, max_num_seqs=512, dtype=torch.bfloat16, max_decoder_len=256,
              max_encoder_len=1024, cuda_graphs=True)
    rng = np.random.default_rng(5)
    n_req = 600
    arrive = np.cumsum(rng.poisson(0.4, size=n_req)).tolist()
    enc = np.where(rng.random(n_req) < 0.5, 587, rng.integers(64, 1025, size=n_req)).tolist()
    out_len = np.minimum(rng.geometric(1 / 96, size=n_req), 256).tolist()
    sp = SamplingParams(max_tokens=256, eos_token_id=[cfg.eos_token_id],
                        suppress_tokens=[cfg.eos_token_id])
    target, done, sizes, step = {}, {}, set(), 0
    pending = list(range(n_req))
    while pending or not llm.is_finished():
        while pending and arrive[pending[0]] <= step:
            i = pending.pop(0)
            ids = rng.integers(3, cfg.vocab_size, size=enc[i]).tolist()
            target[llm.add_request(Request(ids), sp)] = out_len[i]
        if not llm.is_finished():
            before = {r.request_id: len(r.token_ids) - 1 for r in llm.scheduler.running}
            sizes.add(len(before))
            for rid, out in llm.step():  # reached the 256-token cap: finished by the engine
                done[rid] = len(out.completion_token_ids)
            for row in llm.scheduler.running:
                generated = len(row.token_ids) - 1
                assert generated == before.get(row.request_id, 0) + 1
                if generated >= target[row.request_id]:
                    assert llm.abort_request(row.request_id)
                    done[row.request_id] = generated
        step += 1
    assert done == target
    assert max(sizes) <= 512 and len(sizes) > 50
    assert len(llm.runner._graphs) <= len(row_buckets(512))
    assert_clean(llm)


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_beam_step_uploads_the_group_plan_of_its_tables(dtype):
    """A beam-search step's beam groups run from the group plan the runner builds on the
    host: the plan in HBM (its used part) equals build_group_plan over the step's
    uploaded tables, lengths and group starts with the step's copy-on-write pairs folded
    in, and the self-attention metadata points at it."""
    from vflorence_amd import Request, SamplingParams, hip_attn
    from vflorence_amd.utils.context import get_context, set_context

    fx = fixtures()["small"]
    llm = engine(fx["config"], fx["checksum"], max_num_seqs=24, dtype=dtype,
                 max_decoder_len=32, max_encoder_len=128)
    params = SamplingParams(**{**fx["cases"]["beam4_early"]["params"], "max_tokens": 20,
                               "min_length": 21})
    for p in fx["prompts"][:5]:
        llm.add_request(Request(p), params)
    runner, sched = llm.runner, llm.scheduler
    with torch.inference_mode():
        for _ in range(19):  # forks and copy-on-write have made tables diverge
            llm.step()
        batch = sched.schedule()
        if batch.fresh:
            runner._encode(batch.fresh)
        runner._prepare(batch)
        torch.cuda.synchronize()
        ctx = get_context()
        sm = ctx.self_metadata
        assert sm.group_plan is not None and runner._step_grouped
        buf = runner._buffers
        padded = ctx.context_lens.shape[0]
        gs = ctx.self_metadata.group_start.cpu()
        groups = int(np.searchsorted(gs.numpy(), padded))
        want = hip_attn.build_group_plan(
            ctx.block_tables.cpu(), ctx.context_lens.cpu(), gs[: groups + 1], num_slots=buf.rows,
            max_group_size=hip_attn.MAX_GROUP_SIZE, num_blocks=runner.config.num_blocks)
        # the step's copy-on-write pairs ride in the plan (bf16/fp16: the fused launch
        # copies them)
        pairs = batch.num_pairs
        src = buf.d["copy_src"][:pairs].cpu().numpy()
        dst = buf.d["copy_dst"][:pairs].cpu().numpy()
        assert pairs > 0
        assert hip_attn.fold_plan_copies(want, src, dst, num_blocks=runner.config.num_blocks)
        used = 4 + groups * want.stride
        got = sm.group_plan.words[:used].cpu()
        # compare header and the entries each slot holds (the rest of a slot is unused)
        assert int(got[0]) == groups == int(want.words[0])
        shared = copies = 0
        for s in range(groups):
            a = got[4 + s * want.stride:]
            b = want.words[4 + s * want.stride:]
            n = int(b[2])
            assert torch.equal(a[:4 + 2 * n], b[:4 + 2 * n]), s  # header, entries
            shared += sum(bin(int(b[5 + 2 * e]) & 0xFF).count("1") > 1 for e in range(n))
            copies += sum(int(b[5 + 2 * e]) < 0 for e in range(n))  # flagged fork blocks
        assert shared > 0  # beams share prefix blocks
        assert copies == pairs  # every pair rides in the plan
        set_context()
    llm.abort()
