"""Seeded random sweeps of the attention entry points against the oracle.

Each case draws its dtype, head size, head count, row count, ragged context lengths
(zeros included), workgroup waves, row groups sharing one table (cross-attention
beams) and dispatch order (none, longest first, balanced), so combinations that the
targeted tests do not enumerate are still compared with the float64 oracle under the
same bars (1e-5 relative in fp32, 2e-2 absolute in bf16 / fp16).
"""

import random

import pytest
import torch

from test_kernels_gpu import DEV, check, grouped_case, hip, make_case

pytestmark = pytest.mark.gpu

CASES = 100


def draw(seed: int):
    r = random.Random(seed)
    dtype = r.choice([torch.bfloat16, torch.float16, torch.float32])
    head_dim = r.choice([64, 64, 128])
    H = r.randint(1, 16)
    waves = r.choice([0, 1, 2, 4, 8])
    grouped = r.random() < 0.5
    order = r.choice(["none", "longest", "balanced"])
    return r, dtype, head_dim, H, waves, grouped, order


def run(q, kc, vc, lens, table, scale, waves, starts, gmax, order):
    hip_attn = hip()
    firsts = lens.tolist() if starts is None else [lens[i].item() for i in starts[:-1]]
    perm = {"none": None, "longest": hip_attn.longest_first(firsts),
            "balanced": hip_attn.balanced_order(firsts, hip_attn.resident_run(DEV, q.shape[1]))}
    meta = hip_attn.get_scheduler_metadata(
        num_reqs=q.shape[0], num_heads=q.shape[1], num_kv_heads=q.shape[1],
        head_dim=q.shape[2], dtype=q.dtype, block_size=kc.shape[2],
        waves_per_workgroup=waves,
        group_start=None if starts is None else starts.to(DEV), max_group_size=gmax,
        group_order=None if perm[order] is None else torch.tensor(
            perm[order], dtype=torch.int32, device=DEV))
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    hip_attn.attention_with_kv_cache(
        q.contiguous().to(DEV), kc.to(DEV), hip_attn.v_cache_from_logical(vc).to(DEV), out,
        torch.arange(q.shape[0] + 1, dtype=torch.int32, device=DEV), lens.to(DEV),
        scale=scale, causal=False, block_table=table.to(DEV), scheduler_metadata=meta)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("seed", range(CASES))
def test_random_attention_matches_oracle(seed):
    r, dtype, head_dim, H, waves, grouped, order = draw(seed)
    scale = head_dim ** -0.5
    if grouped:
        sizes = [r.randint(1, 8) for _ in range(r.randint(1, 6))]
        enc = [r.choice([0, r.randint(1, 40), r.randint(200, 700)]) for _ in sizes]
        enc[0] = max(enc[0], 1)  # a table of at least one column
        q, kc, vc, L, table, starts = grouped_case(sizes, enc, H=H, D=head_dim, dtype=dtype,
                                                   seed=seed)
        gmax = max(sizes)
    else:
        lens = [r.choice([0, r.randint(1, 17), r.randint(18, 400)])
                for _ in range(r.randint(1, 40))]
        q, kc, vc, L, table = make_case(lens, H=H, D=head_dim, dtype=dtype, seed=seed)
        starts, gmax = None, 1
    print(f"[random] seed {seed}: {dtype} D {head_dim} H {H} rows {q.shape[0]} waves {waves} "
          f"groups {'yes' if grouped else 'no'} order {order}", flush=True)
    out = run(q, kc, vc, L, table, scale, waves, starts, gmax, order)
    check(out, q, kc, vc, L, table, scale)


@pytest.mark.parametrize("seed", range(60))
def test_random_beam_groups_fused_write_matches_two_steps_and_oracle(seed):
    """Own-tables row groups (beams sharing prefix blocks) with the KV write fused: the
    caches bit for bit those of the two-step write + attention, the outputs too at one
    wave count, and within the bars of the oracle over the written caches."""
    from test_shared_prefix_gpu import bits, oracle_check, prefix_tree_case, write_and_attend

    r = random.Random(1000 + seed)
    dtype = r.choice([torch.bfloat16, torch.float16])
    head_dim = r.choice([64, 64, 128])
    H = r.randint(1, 16)
    waves = r.choice([0, 1, 2, 4, 8])
    sizes = [r.randint(1, 8) for _ in range(r.randint(1, 8))]
    max_len = r.choice([16, 64, 300])
    print(f"[random groups] seed {seed}: {dtype} D {head_dim} H {H} groups {sizes} "
          f"waves {waves} max_len {max_len}", flush=True)
    fused, kc, vc, L, table, slots, starts = prefix_tree_case(sizes, seed, H=H, D=head_dim,
                                                              dtype=dtype, max_len=max_len)
    one, k1, v1 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, True, H=H,
                                   D=head_dim)
    two, k2, v2 = write_and_attend(fused, kc, vc, L, table, slots, starts, waves, False, H=H,
                                   D=head_dim)
    assert (bits(k1) == bits(k2)).all() and (bits(v1) == bits(v2)).all()
    if waves:
        assert (bits(one) == bits(two)).all()
    else:
        # the default wave count differs between the fused launch (FUSED_GROUP_WAVES) and
        # the plain one (the library's), so the merge of wave states rounds differently
        oracle_check(two, fused, k2, v2, L, table, H=H, D=head_dim)
    oracle_check(one, fused, k1, v1, L, table, H=H, D=head_dim)


@pytest.mark.parametrize("seed", range(40))
def test_random_decode_linear_chains_match_float64(seed):
    """vfl_linear over random shapes: x (row-major, or packed by an earlier call with
    LINEAR_Y_PACKED) times a packed weight, with and without bias and GELU.  The packed
    output holds exactly the row-major call's rows; a call on it equals the call on the
    row-major rows bit for bit; results are within one rounding of float64 (GELU: of
    GELU on the rounded pre-activation)."""
    import torch.nn.functional as F
    from test_linear_gpu import assert_one_rounding, ops, reference, unpack

    r = random.Random(2000 + seed)
    dtype = r.choice([torch.bfloat16, torch.float16])
    rows = r.choice([1, r.randint(2, 31), r.randint(32, 256)])
    k1 = 256 * r.randint(1, 16)
    # a packed output needs a multiple of 32; the chained call a multiple of 256
    n1 = 32 * r.randint(1, 40) if r.random() < 0.5 else 256 * r.randint(1, 16)
    n2 = r.randint(1, 1100)
    gelu = r.random() < 0.5
    with_bias = r.random() < 0.7
    print(f"[random linear] seed {seed}: {dtype} rows {rows} {k1} -> {n1} -> {n2} gelu {gelu} "
          f"bias {with_bias}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(rows, k1, device=DEV, generator=g).to(dtype)
    w1 = (torch.randn(n1, k1, device=DEV, generator=g) / k1**0.5).to(dtype)
    b1 = torch.randn(n1, device=DEV, generator=g).to(dtype) if with_bias else None
    o = ops()
    flags = o.LINEAR_GELU if gelu else 0
    p1 = o.pack_linear_weight(w1)
    mid = o.linear(x, p1, b1, n1, flags=flags)
    mid_packed = o.linear(x, p1, b1, n1, flags=flags | o.LINEAR_Y_PACKED)
    assert torch.equal(unpack(mid_packed, rows, n1), mid)
    pre = reference(x, w1, b1)
    if gelu:
        want = F.gelu(pre.to(dtype).double())
        ulp = 2**-8 if dtype == torch.bfloat16 else 2**-11
        err = (mid.double() - want).abs()
        assert (err <= 2.5 * ulp * pre.abs() + ulp * want.abs() + 1e-4).all()
    else:
        assert_one_rounding(mid, pre, dtype)
    if n1 % 256:
        return  # the second call needs in_features a multiple of 256
    w2 = (torch.randn(n2, n1, device=DEV, generator=g) / n1**0.5).to(dtype)
    p2 = o.pack_linear_weight(w2)
    out = o.linear(mid_packed, p2, None, n2, rows=rows, flags=o.LINEAR_X_PACKED)
    assert torch.equal(out, o.linear(mid, p2, None, n2))
    assert_one_rounding(out, reference(mid, w2, None), dtype)


@pytest.mark.parametrize("seed", range(40))
def test_random_logprob_topk_matches_processor_and_topk(seed):
    """log-softmax + generation rules + top-k over random vocab sizes, k, row counts,
    lengths and rule sets, against LogitsProcessor + torch.topk."""
    from test_decoder_ops_gpu import canon, ops as dops, reference
    from transformers import GenerationConfig

    from vflorence_amd.sampling_params import SamplingParams

    r = random.Random(3000 + seed)
    vocab = r.choice([r.randint(2, 64), r.randint(65, 5000), r.randint(5000, 60000)])
    k = r.randint(1, min(16, vocab))
    rows = r.randint(1, 300)
    tok = lambda: r.randrange(vocab)
    rules = {}
    if r.random() < 0.4:
        rules["min_length"] = r.randint(1, 8)
    if r.random() < 0.3:
        rules["forced_bos_token_id"] = tok()
    if r.random() < 0.3:
        rules["forced_eos_token_id"] = sorted({tok() for _ in range(r.randint(1, 3))})
    if r.random() < 0.4:
        rules["suppress_tokens"] = sorted({tok() for _ in range(r.randint(1, 6))})
    if r.random() < 0.3:
        rules["begin_suppress_tokens"] = sorted({tok() for _ in range(r.randint(1, 4))})
    log_softmax = r.random() < 0.7
    eos = sorted({tok() for _ in range(r.randint(1, 2))})
    print(f"[random topk] seed {seed}: vocab {vocab} k {k} rows {rows} rules {rules} "
          f"eos {eos} log_softmax {log_softmax}", flush=True)
    params = SamplingParams(eos_token_id=eos, **rules).with_defaults(
        SamplingParams.from_generation_config(GenerationConfig()))
    g = torch.Generator(device=DEV).manual_seed(seed)
    logits = torch.randn(rows, vocab, device=DEV, generator=g) * 4
    max_length, begin_index = 10, 2
    lengths = torch.tensor([r.randint(1, max_length) for _ in range(rows)], dtype=torch.int64,
                           device=DEV)
    (want_v, want_i), proc, ref = reference(logits, k, log_softmax, params, lengths, vocab,
                                            max_length, begin_index)
    got_v, got_i = dops().logprob_topk(logits, k, log_softmax=log_softmax, lengths=lengths,
                                       rules=proc.topk_rules())
    torch.testing.assert_close(got_v, want_v, rtol=1e-6, atol=1e-5)
    assert canon(ref.gather(1, got_i), got_i) == canon(want_v, want_i)
    assert ((got_i >= 0) & (got_i < vocab)).all()
