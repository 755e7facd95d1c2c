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
