"""Write tests/golden/token_fixtures.json: token ids that transformers' BART generates.

Run once on the CPU (``python tests/golden/make_token_fixtures.py``).  transformers is
the independent library oracle for decoded tokens: the engine must reproduce its
greedy and beam-search outputs.  Weights come from
``vflorence_amd.utils.loader.synthetic_state_dict`` (a hash of seed, name and index,
identical on CPU and GPU), so the tests rebuild them instead of storing them; each
config records the weights' checksum.

Each request is generated on its own (batch 1, no padding); the engine later runs
them batched.  Every case also records, per request and per step, the margin that decides the
step: greedy, the gap between the best and second-best processed score; beam search,
the gap between the ``num_beams``-th and the next accumulated score (which
candidates live on), and at the last step also between the best two (which
hypothesis is returned).  A fp32 GPU run may only take a different token where such a gap is
within float noise, and a 16-bit run's first differing step can be read against it.

The beam cases at BART-large and Florence-2-base shapes follow the reference's own
parity settings (tests/verify_parity.py:70-108,177): BART with 4 beams, EOS
suppressed (``min_length`` past ``max_tokens``), length penalty 2 and no repeated
3-grams; Florence-2-base with 3 beams and neutral decoding that stops at EOS.  Their
prompts are drawn from seeded streams; a prompt whose decisive margin at some step
is below 1e-4 (a tie within fp32 rounding of the accumulated scores) is skipped and
listed with its margin, and each case stores the prompts it kept.

The reachable-EOS cases (``bart_large_eos``, ``florence2_base_eos``; refreshed alone by
``python tests/golden/make_token_fixtures.py eos``) add a bias to EOS's final logit so
that hypotheses end at different steps, with early stopping on and off; their margins
also include the gap between the best two final hypothesis scores (which finished
hypothesis is returned).
"""

from __future__ import annotations

import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from transformers import BartConfig, BartForConditionalGeneration  # noqa: E402

from vflorence_amd.utils.loader import state_dict_checksum, synthetic_state_dict  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "token_fixtures.json")

SMALL = dict(vocab_size=96, d_model=128, encoder_layers=2, decoder_layers=2,
             encoder_attention_heads=2, decoder_attention_heads=2, encoder_ffn_dim=256,
             decoder_ffn_dim=256, max_position_embeddings=256, bos_token_id=0, pad_token_id=1,
             eos_token_id=2, decoder_start_token_id=2, forced_eos_token_id=None,
             tie_word_embeddings=False)
# BartConfig() defaults are BART-large.  The LM head is untied: with random weights a
# tied head scores the token just fed far above the rest (the residual stream keeps its
# embedding), so generation would echo the start token, which is EOS, and stop at once.
LARGE = dict(forced_eos_token_id=None, tie_word_embeddings=False)
# Florence-2-base's text model is a BART of these sizes; its decoder reads 577 visual
# tokens plus a 10-token prompt, stood in for here by 587 encoder token ids.
FLORENCE_BASE = dict(vocab_size=51289, d_model=768, encoder_layers=6, decoder_layers=6,
                     encoder_attention_heads=12, decoder_attention_heads=12,
                     encoder_ffn_dim=3072, decoder_ffn_dim=3072, max_position_embeddings=1024,
                     forced_eos_token_id=None, tie_word_embeddings=False)

# every field set explicitly: nothing is inherited from a generation config
BASE = dict(max_tokens=24, num_beams=1, repetition_penalty=1.0, eos_token_id=[2],
            length_penalty=1.0, no_repeat_ngram_size=0, min_length=0,
            forced_bos_token_id=None, forced_eos_token_id=None, suppress_tokens=[],
            begin_suppress_tokens=[], early_stopping=False)

SMALL_CASES = {
    "greedy": {},
    "greedy_rules": dict(repetition_penalty=1.3, no_repeat_ngram_size=3, min_length=5),
    "greedy_forced": dict(forced_bos_token_id=0, forced_eos_token_id=2, suppress_tokens=[5, 6],
                          begin_suppress_tokens=[7], max_tokens=12),
    "beam2": dict(num_beams=2, max_tokens=16),
    "beam4_early": dict(num_beams=4, max_tokens=16, early_stopping=True, min_length=4,
                        length_penalty=0.8),
    "beam4_rules": dict(num_beams=4, max_tokens=12, no_repeat_ngram_size=2,
                        repetition_penalty=1.2),
}


def prompts(vocab: int, lengths: list[int], seed: int) -> list[list[int]]:
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(3, vocab, (n,), generator=g).tolist() for n in lengths]


class _CandidateGaps:
    """Records, at every beam-search step, the margin that decides it: the gap between
    the ``num_beams``-th and the next accumulated score over all beams (which candidates
    continue) and, at the last step, also the gap between the best two (which hypothesis
    is returned).  That is the whole decision when no candidate finishes before the last
    step (the BART-large and Florence-2-base beam cases); with earlier finishes it is a
    partial view.  Wraps transformers' ``_get_top_k_continuations``, which receives
    those scores."""

    def __init__(self, model, num_beams: int, max_tokens: int):
        self.model, self.gaps = model, []
        self.num_beams, self.max_tokens = num_beams, max_tokens
        self._orig = model._get_top_k_continuations
        model._get_top_k_continuations = self._hook

    def _hook(self, *args, **kwargs):
        acc = kwargs["accumulated_log_probs"]
        nb = self.num_beams
        top = acc.topk(nb + 1, dim=-1).values[0]
        gap = float(top[nb - 1] - top[nb])
        if len(self.gaps) == self.max_tokens - 1:
            gap = min(gap, float(top[0] - top[1]))
        self.gaps.append(gap if math.isfinite(gap) else None)
        return self._orig(*args, **kwargs)

    def close(self):
        self.model._get_top_k_continuations = self._orig


def hf_generate(model, ids: list[int], params: dict, final_gap: bool = False):
    kw = dict(max_new_tokens=params["max_tokens"], num_beams=params["num_beams"], do_sample=False,
              repetition_penalty=params["repetition_penalty"], eos_token_id=params["eos_token_id"],
              length_penalty=params["length_penalty"],
              no_repeat_ngram_size=params["no_repeat_ngram_size"],
              min_length=params["min_length"], early_stopping=params["early_stopping"],
              forced_bos_token_id=params["forced_bos_token_id"],
              forced_eos_token_id=params["forced_eos_token_id"],
              suppress_tokens=params["suppress_tokens"] or None,
              begin_suppress_tokens=params["begin_suppress_tokens"] or None,
              decoder_start_token_id=model.config.decoder_start_token_id,
              pad_token_id=model.config.pad_token_id, output_scores=True,
              return_dict_in_generate=True)
    if final_gap and params["num_beams"] > 1:
        # every kept hypothesis comes back with its final score: the gap between the best
        # two decides which one is returned (whatever step they finished at)
        kw["num_return_sequences"] = params["num_beams"]
    recorder = (_CandidateGaps(model, params["num_beams"], params["max_tokens"])
                if params["num_beams"] > 1 else None)
    try:
        with torch.no_grad():
            out = model.generate(torch.tensor([ids]),
                                 attention_mask=torch.ones(1, len(ids), dtype=torch.long), **kw)
    finally:
        if recorder is not None:
            recorder.close()
    tokens = out.sequences[0].tolist()[1:]
    if params["num_beams"] == 1:
        gaps = [float(s[0].topk(2).values.diff().abs()) for s in out.scores]
        return tokens, gaps
    pad = model.config.pad_token_id
    gaps = recorder.gaps
    if final_gap:
        final = out.sequences_scores
        gaps = gaps + [float(final[0] - final[1])]
    return [t for t in tokens if t != pad], gaps


def min_gap(gaps):
    finite = [g for g in gaps or () if g is not None]
    return min(finite) if finite else None


def case_record(params, outs):
    """Tokens per request, each request's per-step gaps and their minimum."""
    return {"params": params, "tokens": [t for t, _ in outs],
            "gaps": [[None if g is None else round(g, 7) for g in gp] for _, gp in outs],
            "min_gap": [min_gap(gp) for _, gp in outs]}


def build(config_kwargs: dict, eos_bias: float = 0.0):
    config = BartConfig(**config_kwargs)
    sd = synthetic_state_dict(config, seed=0)
    if eos_bias:
        sd = with_eos_bias(sd, config.eos_token_id, eos_bias)
    model = BartForConditionalGeneration(config).eval()
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and not [k for k in missing if "embed_tokens" not in k
                                   and k != "lm_head.weight"], (missing, unexpected)
    return config, model, state_dict_checksum(sd)


# The reference's beam parity settings (tests/verify_parity.py:81-87): EOS suppressed
# so every beam runs max_tokens steps, length penalty 2, no repeated 3-grams.
BART_BEAM4 = {**BASE, "max_tokens": 24, "num_beams": 4, "min_length": 25,
              "length_penalty": 2.0, "no_repeat_ngram_size": 3}
# The same without the history rule: the engine then takes its candidates from the
# fused log-softmax + rules + top-k kernel instead of the torch path.
BART_BEAM4_FUSED = {**BASE, "max_tokens": 24, "num_beams": 4, "min_length": 25}
# Florence-2's neutral decoding with 3 beams (tests/verify_parity.py:135-139): stops
# at EOS.
FLORENCE_BEAM3 = {**BASE, "max_tokens": 32, "num_beams": 3}


# A beam case keeps a prompt only if every step's decisive margin is at least this: a
# smaller one is a tie within the rounding of fp32 accumulated scores (one ulp at 128 is
# 1.5e-5), which no other summation order can be required to break the same way.
BEAM_MARGIN = 1e-4


def beam_case(model, vocab: int, params: dict, count: int, length_fn, seed: int, tag: str,
              final_gap: bool = False):
    """``count`` prompts drawn in order from a seeded stream (lengths from ``length_fn``),
    each generated with ``params``; a prompt with a decisive margin below BEAM_MARGIN is
    skipped and recorded in ``skipped``."""
    g = torch.Generator().manual_seed(seed)
    kept, outs, skipped = [], [], []
    while len(kept) < count:
        n = length_fn(g)
        ids = torch.randint(3, vocab, (n,), generator=g).tolist()
        tokens, gaps = hf_generate(model, ids, params, final_gap)
        margin = min_gap(gaps)
        print(tag, n, len(tokens), margin, flush=True)
        if margin is None or margin < BEAM_MARGIN:
            skipped.append({"length": n, "min_gap": margin})
            continue
        kept.append(ids)
        outs.append((tokens, gaps))
    record = case_record(params, outs)
    record["prompts"] = kept
    record["skipped"] = skipped
    return record


def florence2_base() -> dict:
    config, model, checksum = build(FLORENCE_BASE)
    reqs = prompts(config.vocab_size, [587] * 6, seed=4)
    params = {**BASE, "max_tokens": 32}
    outs = [hf_generate(model, ids, params) for ids in reqs]
    print("florence2_base", [len(t) for t, _ in outs], flush=True)
    cases = {"greedy32": case_record(params, outs)}
    cases["beam3"] = beam_case(model, config.vocab_size, FLORENCE_BEAM3, 6, lambda g: 587,
                               seed=5, tag="florence2_base beam3")
    return {"config": FLORENCE_BASE, "checksum": checksum, "prompts": reqs, "cases": cases}


def with_eos_bias(state_dict: dict, eos: int, bias: float) -> dict:
    """The checkpoint with ``bias`` added to ``final_logits_bias[0, eos]`` (one fp32 add,
    the same bits on any device)."""
    out = dict(state_dict)
    flb = out["final_logits_bias"].clone()
    flb[0, eos] += bias
    out["final_logits_bias"] = flb
    return out


# Reachable EOS at real depth (the reference's early-stopping check,
# tests/test_parity.py:88-122: an EOS logit bias plus min_length so that beams finish
# at different steps).  With random weights every token's log-probability sits near
# -ln(vocab); the bias lifts EOS to the edge of the kept candidates, so hypotheses end
# at different steps and the EOS rank gate, finished-hypothesis scoring and both
# early-stopping rules decide the outputs.  Biases chosen by a sweep over the two
# shapes (BART-large: 1.8 never ends before 24 tokens on most prompts, 1.9 ends every
# prompt at min_length; Florence-2-base: 1.5 ends prompts at 10-13 tokens and the two
# early-stopping rules part).
EOS_CASES = {
    "bart_large_eos": dict(config=LARGE, eos_bias=1.85, beams=4, max_tokens=24, count=8,
                           lengths=lambda g: int(torch.randint(128, 1025, (1,), generator=g)),
                           seed=8),
    "florence2_base_eos": dict(config=FLORENCE_BASE, eos_bias=1.5, beams=3, max_tokens=32,
                               count=6, lengths=lambda g: 587, seed=9),
}


def eos_fixtures() -> dict:
    out = {}
    for name, spec in EOS_CASES.items():
        config, model, checksum = build(spec["config"], spec["eos_bias"])
        cases = {}
        for early in (False, True):
            params = {**BASE, "max_tokens": spec["max_tokens"], "num_beams": spec["beams"],
                      "min_length": 4, "early_stopping": early}
            key = f"beam{spec['beams']}_eos" + ("_early" if early else "")
            cases[key] = beam_case(model, config.vocab_size, params, spec["count"],
                                   spec["lengths"], seed=spec["seed"], tag=f"{name} {key}",
                                   final_gap=True)
        out[name] = {"config": spec["config"], "eos_bias": spec["eos_bias"],
                     "checksum": checksum, "cases": cases}
    return out


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    fixtures = {"_provenance": (
        "transformers " + __import__("transformers").__version__ + " BartForConditionalGeneration "
        "generate() on CPU, fp32, weights synthetic_state_dict(seed=0); tests/golden/"
        "make_token_fixtures.py")}

    config, model, checksum = build(SMALL)
    lengths = [5, 17, 16, 33, 64, 100]
    reqs = prompts(config.vocab_size, lengths, seed=1)
    small = {"config": SMALL, "checksum": checksum, "prompts": reqs, "cases": {}}
    for name, over in SMALL_CASES.items():
        params = {**BASE, **over}
        outs = [hf_generate(model, ids, params) for ids in reqs]
        small["cases"][name] = case_record(params, outs)
        print(name, [len(t) for t, _ in outs], flush=True)
    fixtures["small"] = small

    t0 = time.time()
    config, model, checksum = build(LARGE)
    g = torch.Generator().manual_seed(2)
    lengths = torch.randint(128, 1025, (8,), generator=g).tolist()
    reqs = prompts(config.vocab_size, lengths, seed=3)
    params = {**BASE, "max_tokens": 64}
    outs = []
    for ids in reqs:
        outs.append(hf_generate(model, ids, params))
        print("large", len(ids), len(outs[-1][0]), f"{time.time() - t0:.0f}s", flush=True)
    cases = {"greedy64": case_record(params, outs)}
    for name, params, seed in (("beam4", BART_BEAM4, 6), ("beam4_fused", BART_BEAM4_FUSED, 7)):
        cases[name] = beam_case(
            model, config.vocab_size, params, 8,
            lambda g: int(torch.randint(128, 1025, (1,), generator=g)), seed=seed,
            tag=f"large {name}")
    fixtures["bart_large"] = {"config": LARGE, "checksum": checksum, "prompts": reqs,
                              "cases": cases}
    fixtures["florence2_base"] = florence2_base()
    fixtures.update(eos_fixtures())
    with open(OUT, "w") as f:
        json.dump(fixtures, f)
    print("wrote", OUT)


if __name__ == "__main__":
    if sys.argv[1:] == ["eos"]:  # add or refresh only the reachable-EOS sections
        torch.set_num_threads(min(8, os.cpu_count() or 1))
        with open(OUT) as f:
            fixtures = json.load(f)
        fixtures.update(eos_fixtures())
        with open(OUT, "w") as f:
            json.dump(fixtures, f)
        print("wrote", OUT)
    else:
        main()
