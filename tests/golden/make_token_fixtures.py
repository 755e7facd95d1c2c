"""Write tests/golden/token_fixtures.json: token ids that transformers' BART generates.

Run once on the CPU (``python tests/golden/make_token_fixtures.py``).  transformers is
the independent library oracle for decoded tokens: the engine must reproduce its
greedy and beam-search outputs.  Weights come from
``vflorence_amd.utils.loader.synthetic_state_dict`` (a hash of seed, name and index,
identical on CPU and GPU), so the tests rebuild them instead of storing them; each
config records the weights' checksum.

Each request is generated on its own (batch 1, no padding); the engine later runs
them batched.  Greedy cases also record, per request, the smallest gap between the
best and second-best processed score over its steps: a fp32 GPU run may only take a
different token where that gap is within float noise.
"""

from __future__ import annotations

import json
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


def hf_generate(model, ids: list[int], params: dict):
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
    with torch.no_grad():
        out = model.generate(torch.tensor([ids]), attention_mask=torch.ones(1, len(ids),
                                                                          dtype=torch.long), **kw)
    tokens = out.sequences[0].tolist()[1:]
    if params["num_beams"] == 1:
        gaps = [float(s[0].topk(2).values.diff().abs()) for s in out.scores]
        return tokens, min(gaps) if gaps else None
    pad = model.config.pad_token_id
    return [t for t in tokens if t != pad], None


def build(config_kwargs: dict):
    config = BartConfig(**config_kwargs)
    sd = synthetic_state_dict(config, seed=0)
    model = BartForConditionalGeneration(config).eval()
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and not [k for k in missing if "embed_tokens" not in k
                                   and k != "lm_head.weight"], (missing, unexpected)
    return config, model, state_dict_checksum(sd)


def florence2_base() -> dict:
    config, model, checksum = build(FLORENCE_BASE)
    reqs = prompts(config.vocab_size, [587] * 6, seed=4)
    params = {**BASE, "max_tokens": 32}
    outs = [hf_generate(model, ids, params) for ids in reqs]
    print("florence2_base", [len(t) for t, _ in outs], flush=True)
    return {"config": FLORENCE_BASE, "checksum": checksum, "prompts": reqs,
            "cases": {"greedy32": {"params": params, "tokens": [t for t, _ in outs],
                                   "min_gap": [gp for _, gp in outs]}}}


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
        small["cases"][name] = {"params": params, "tokens": [t for t, _ in outs],
                                "min_gap": [g for _, g in outs]}
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
    fixtures["bart_large"] = {"config": LARGE, "checksum": checksum, "prompts": reqs,
                              "cases": {"greedy64": {"params": params,
                                                     "tokens": [t for t, _ in outs],
                                                     "min_gap": [gp for _, gp in outs]}}}
    fixtures["florence2_base"] = florence2_base()
    with open(OUT, "w") as f:
        json.dump(fixtures, f)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
