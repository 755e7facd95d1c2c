"""The decoder-step kernels against torch on the same inputs: residual + LayerNorm, and
log-softmax + generation rules + top-k against LogitsProcessor + torch.topk (whose
rules are themselves checked against transformers' processors on the CPU)."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ops():
    from vflorence_amd import decoder_ops

    return decoder_ops


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [64, 768, 1024, 2052, 4096])
def test_add_layer_norm_matches_torch(dtype, dim):
    g = torch.Generator(device=DEV).manual_seed(dim)
    rows = 37
    x = torch.randn(rows, dim, device=DEV, generator=g).to(dtype)
    r = (torch.randn(rows, dim, device=DEV, generator=g) * 3 + 1).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, device=DEV, generator=g)).to(dtype)
    b = (0.1 * torch.randn(dim, device=DEV, generator=g)).to(dtype)
    got = ops().add_layer_norm(x, r, w, b, 1e-5)
    # torch: the add stored in the element type, then LayerNorm computed in fp32
    s = (x + r).float()
    want = F.layer_norm(s, (dim,), w.float(), b.float(), 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    else:
        torch.testing.assert_close(got.float(), want, rtol=0, atol=2e-2)
        # within one rounding of the element type
        ulp = want.abs().clamp_min(1e-3) * (2**-7 if dtype == torch.bfloat16 else 2**-10)
        assert ((got.float() - want).abs() <= ulp + 1e-6).all()


def test_add_layer_norm_takes_strided_rows_and_rejects_bad_shapes():
    x = torch.randn(8, 3 * 1024, device=DEV)[:, 1024:2048]  # a row-strided view
    r = torch.randn(8, 1024, device=DEV)
    w, b = torch.ones(1024, device=DEV), torch.zeros(1024, device=DEV)
    got = ops().add_layer_norm(x, r, w, b, 1e-5)
    torch.testing.assert_close(got, F.layer_norm(x + r, (1024,), w, b, 1e-5), rtol=1e-5,
                               atol=1e-5)
    with pytest.raises(ValueError):
        ops().add_layer_norm(x, r[:, :512], w, b, 1e-5)
    from vflorence_amd._lib import HipAttnError

    with pytest.raises(HipAttnError):  # dim not a multiple of 4
        ops().add_layer_norm(r[:, :1022], r[:, :1022], w[:1022], b[:1022], 1e-5)


def reference(logits, k, log_softmax, params, lengths, vocab, max_length, begin_index):
    from vflorence_amd.layers.logits_processor import LogitsProcessor

    proc = LogitsProcessor(params, vocab_size=vocab, max_length=max_length,
                           begin_index=begin_index, device=DEV)
    scores = logits.float()
    if log_softmax:
        scores = torch.log_softmax(scores, dim=-1)
    scores = proc(None, scores.clone(), lengths)
    return torch.topk(scores, k, dim=-1), proc, scores


RULES = [
    {},
    dict(min_length=5),
    dict(forced_bos_token_id=7),
    dict(forced_eos_token_id=[2, 9]),
    dict(suppress_tokens=[0, 4, 13]),
    dict(begin_suppress_tokens=[3, 5]),
    dict(min_length=4, forced_bos_token_id=1, forced_eos_token_id=2, suppress_tokens=[2, 6],
         begin_suppress_tokens=[8]),
]


@pytest.mark.parametrize("rule", range(len(RULES)))
@pytest.mark.parametrize("vocab,k", [(50265, 8), (50265, 1), (50265, 16), (40, 16), (12, 12),
                                     (50265, 3)])
@pytest.mark.parametrize("log_softmax", [True, False])
def test_logprob_topk_matches_processor_and_topk(rule, vocab, k, log_softmax):
    from transformers import GenerationConfig

    from vflorence_amd.sampling_params import SamplingParams

    params = SamplingParams(eos_token_id=[2, 3], **RULES[rule]).with_defaults(
        SamplingParams.from_generation_config(GenerationConfig()))
    g = torch.Generator(device=DEV).manual_seed(rule * 7 + k)
    rows = 24
    logits = torch.randn(rows, vocab, device=DEV, generator=g) * 4
    max_length, begin_index = 9, 2
    lengths = torch.tensor([1, 2, 3, 4, 5, 8, 9, 2] * 3, dtype=torch.int64, device=DEV)
    (want_v, want_i), proc, ref = reference(logits, k, log_softmax, params, lengths, vocab,
                                            max_length, begin_index)
    got_v, got_i = ops().logprob_topk(logits, k, log_softmax=log_softmax, lengths=lengths,
                                      rules=proc.topk_rules())
    torch.testing.assert_close(got_v, want_v, rtol=1e-6, atol=1e-5)
    # fp32 random logits do not tie; forced tokens (score 0) do, and torch.topk orders
    # ties arbitrarily: compare the finite (score, token) lists ordered by (score, token),
    # scoring both by the reference's values
    assert canon(ref.gather(1, got_i), got_i) == canon(want_v, want_i)
    # -inf entries name real tokens
    assert ((got_i >= 0) & (got_i < vocab)).all()


def canon(values, ids):
    rows = []
    for vs, ts in zip(values.tolist(), ids.tolist()):
        rows.append(sorted((-v, t) for v, t in zip(vs, ts) if v != float("-inf")))
    return rows


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_logprob_topk_on_16bit_logits_breaks_ties_by_token(dtype):
    """16-bit logits tie often; every returned score must be the token's own processed
    score, the list sorted, and equal scores listed by increasing token id."""
    g = torch.Generator(device=DEV).manual_seed(1)
    logits = (torch.randn(64, 50265, device=DEV, generator=g) * 2).to(dtype)
    got_v, got_i = ops().logprob_topk(logits, 8, log_softmax=True)
    ref = torch.log_softmax(logits.float(), dim=-1)
    torch.testing.assert_close(got_v, ref.gather(1, got_i), rtol=1e-6, atol=1e-5)
    want_v, _ = torch.topk(ref, 8, dim=-1)
    torch.testing.assert_close(got_v, want_v, rtol=1e-6, atol=1e-5)
    same = got_v[:, 1:] == got_v[:, :-1]
    assert (got_i[:, 1:][same] > got_i[:, :-1][same]).all()
    # greedy: the first maximum, as torch.argmax returns it
    _, top1 = ops().logprob_topk(logits, 1, log_softmax=False)
    assert torch.equal(top1[:, 0], logits.float().argmax(dim=-1))


@pytest.mark.parametrize("k,log_softmax", [(8, True), (1, False)])
def test_logprob_topk_writes_pinned_host_outputs(k, log_softmax):
    """The kernel stores into pinned host tensors directly: after a stream
    synchronization they hold what the device-output call returns, and a second call
    into the same tensors overwrites every entry."""
    g = torch.Generator(device=DEV).manual_seed(11)
    outs = (torch.full((64, k), float("nan"), dtype=torch.float32, pin_memory=True),
            torch.full((64, k), -7, dtype=torch.int64, pin_memory=True))
    for step in range(2):
        logits = (torch.randn(64, 50432, device=DEV, generator=g) * 3).to(torch.bfloat16)
        logits = logits[:, :50265]
        want_v, want_i = ops().logprob_topk(logits, k, log_softmax=log_softmax)
        got_v, got_i = ops().logprob_topk(logits, k, log_softmax=log_softmax, out=outs)
        assert got_v is outs[0] and got_i is outs[1]
        torch.cuda.current_stream().synchronize()
        assert torch.equal(got_v, want_v.cpu()) and torch.equal(got_i, want_i.cpu()), step
    with pytest.raises(ValueError):
        ops().logprob_topk(logits, k, log_softmax=log_softmax,
                           out=(torch.empty(64, k), torch.empty(64, k, dtype=torch.int64)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [1.0, 32.0])
def test_embed_layer_norm_equals_lookups_then_add_layer_norm(dtype, scale):
    """One launch for the decoder's embeddings: bit for bit what the two lookups (the
    token row scaled and stored in the element type) and the residual + LayerNorm kernel
    give, over ids and positions that hit the tables' first and last rows."""
    g = torch.Generator(device=DEV).manual_seed(3)
    vocab, max_pos, dim, rows, off = 1000, 130, 1024, 77, 2
    tok = torch.randn(vocab, dim, device=DEV, generator=g).to(dtype)
    pos = torch.randn(max_pos + off, dim, device=DEV, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, device=DEV, generator=g)).to(dtype)
    b = (0.1 * torch.randn(dim, device=DEV, generator=g)).to(dtype)
    ids = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
    positions = torch.randint(0, max_pos, (rows,), device=DEV, generator=g)
    ids[:2] = torch.tensor([0, vocab - 1], device=DEV)
    positions[:2] = torch.tensor([0, max_pos - 1], device=DEV)
    got = ops().embed_layer_norm(ids, positions, tok, scale, pos, off, w, b, 1e-5)
    t = F.embedding(ids, tok)
    if scale != 1.0:
        t = t * scale
    want = ops().add_layer_norm(F.embedding(positions + off, pos), t, w, b, 1e-5)
    assert got.dtype == dtype and got.shape == (rows, dim)
    assert torch.equal(got, want)


def test_embed_layer_norm_marks_rows_with_indices_outside_the_tables():
    g = torch.Generator(device=DEV).manual_seed(4)
    tok = torch.randn(50, 64, device=DEV, generator=g).to(torch.bfloat16)
    pos = torch.randn(12, 64, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.ones(64, device=DEV, dtype=torch.bfloat16)
    b = torch.zeros(64, device=DEV, dtype=torch.bfloat16)
    ids = torch.tensor([3, 50, -1, 7, 8], device=DEV)
    positions = torch.tensor([0, 1, 2, 10, -3], device=DEV)  # + 2: 12 and -1 are outside
    got = ops().embed_layer_norm(ids, positions, tok, 1.0, pos, 2, w, b, 1e-5)
    bad = torch.tensor([False, True, True, True, True], device=DEV)
    assert torch.isnan(got[bad]).all()
    assert torch.isfinite(got[~bad]).all()
    want = ops().add_layer_norm(pos[2:3], tok[3:4], w, b, 1e-5)
    assert torch.equal(got[:1], want)
    with pytest.raises(ValueError):
        ops().embed_layer_norm(ids.int(), positions, tok, 1.0, pos, 2, w, b, 1e-5)
    with pytest.raises(RuntimeError):
        ops().embed_layer_norm(ids.cpu(), positions.cpu(), tok.cpu(), 1.0, pos.cpu(), 2, w.cpu(),
                               b.cpu(), 1e-5)
