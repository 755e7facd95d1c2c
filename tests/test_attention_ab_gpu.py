"""bf16 beam search with the attention ops isolated: an A/B on one GPU.

The same engine (same weights, GEMMs, LayerNorms, sampling kernels) decodes each case
twice:

* run A takes the gfx950 attention kernels, as in production;
* run B replaces only the two attention ops' arithmetic by a reference attention: a
  dense gather by block table and float32 ``softmax(scale q K^T) V`` in torch on the
  GPU, rounded to the element type once.  The KV slot write stays the library's
  scatter, which is bit-exact (tests/test_kernels_gpu.py).

Any difference between A and B therefore comes from the attention ops alone, not from
bf16 weights or GEMM rounding -- the separation the reference's bf16 bar
("same length", tests/verify_parity.py:59-67) cannot make.

Run B also computes, at every step and before its own forward, run A's logits on B's
state (the HIP forward first, then the reference forward, whose KV writes replace the
HIP forward's at the same slots).  That gives the one-step change a candidate's
log-probability takes from the attention ops, ``delta_t``; it must stay below a stated
bound (STEP_ULPS units in the last place of the bf16 logit).  A request's outputs may
then differ between A and B only where B's decisive margin at the first diverging
decision is below what the accumulated attention perturbation can reach
(FLIP_FACTOR x the sum of delta over the steps so far).

What the runs show: with bf16 logits, candidates' scores are quantised to the
logits' rounding step (2^-5 for logits in [4, 8)), so decisive margins of one step
or exact ties are common, and a one-step change of one logit rounding -- all that
the attention ops cause -- decides them.  That is why bf16 token identity across
attention implementations (the reference's own included) cannot be asked for.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "token_fixtures.json")

# The largest one-step change the attention ops may cause in a decoded candidate's
# logit, in rounding steps of the row's largest candidate logit (bf16).  The two
# attention paths agree to within bf16's rounding of their outputs (relative 2^-8);
# carried through the decoder's post-LayerNorm layers that moves the row's logits by
# about one such step before the LM head rounds them (measured: at most 2 steps at
# BART-large depth, 1 at Florence-2-base); 4 leaves room for a box or build that rounds
# one step further.  The attention outputs themselves are held to the float64 oracle by
# the kernel tests; this bound is about what reaches the tokens.
STEP_ULPS = 4
# Two candidates can swap when their margin is below the sum of their perturbations:
# each accumulated score moves by at most the sum of the one-step changes so far.
FLIP_FACTOR = 2.0


def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


def reference_attention(query, k_cache, v_cache, seq_lens, block_table, scale):
    """float32 ``softmax(scale q K^T) V`` over each row's first ``seq_lens[r]`` tokens
    of the blocks its table lists, rounded to the query's dtype (zero for empty rows)."""
    from vflorence_amd import hip_attn

    n, h, d = query.shape
    bs = k_cache.shape[2]
    table = block_table.long()
    w = table.shape[1]
    k = k_cache[table].permute(0, 2, 1, 3, 4).reshape(n, h, w * bs, d).float()
    v = hip_attn.v_cache_logical(v_cache[table].flatten(0, 1)).view(n, w, h, bs, d)
    v = v.permute(0, 2, 1, 3, 4).reshape(n, h, w * bs, d).float()
    s = torch.matmul(k, query.float().unsqueeze(-1)).squeeze(-1) * scale  # [n, h, T]
    lens = seq_lens.long()
    mask = torch.arange(w * bs, device=query.device)[None, :] >= lens[:, None]
    s = s.masked_fill(mask[:, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1).nan_to_num(0.0)
    out = torch.matmul(p.unsqueeze(-2), v).squeeze(-2)
    return torch.where((lens > 0)[:, None, None], out, 0.0).to(query.dtype)


class AttentionOps:
    """Stands in for ``hip_attn`` inside the attention op bodies: ``mode`` "hip"
    forwards to the gfx950 kernels, "ref" computes the attention with
    ``reference_attention`` (the KV write stays the library's scatter)."""

    def __init__(self, real):
        self.real, self.mode = real, "hip"

    def __getattr__(self, name):
        return getattr(self.real, name)

    def attention_with_kv_cache(self, query, k_cache, v_cache, out, query_start_loc, seq_lens,
                                *, scale, causal=False, block_table, scheduler_metadata=None):
        if self.mode == "hip":
            return self.real.attention_with_kv_cache(
                query, k_cache, v_cache, out, query_start_loc, seq_lens, scale=scale,
                causal=causal, block_table=block_table, scheduler_metadata=scheduler_metadata)
        out.copy_(reference_attention(query, k_cache, v_cache, seq_lens, block_table, scale))

    def self_attention_with_kv_write(self, query, key, value, k_cache, v_cache, out, seq_lens,
                                     slot_mapping, *, scale, block_table, scheduler_metadata):
        if self.mode == "hip":
            return self.real.self_attention_with_kv_write(
                query, key, value, k_cache, v_cache, out, seq_lens, slot_mapping, scale=scale,
                block_table=block_table, scheduler_metadata=scheduler_metadata)
        self.real.reshape_and_cache(key, value, k_cache, v_cache, slot_mapping)
        out.copy_(reference_attention(query, k_cache, v_cache, seq_lens, block_table, scale))


class BeamRecorder:
    """Per request and decode step: the running hypotheses at the step's start and the
    margin that decides the step (recomputed from the rows' accumulated scores and the
    step's candidates with the engine's rules: the num_beams-th against the next
    candidate; with early stopping off, the worst kept finished hypothesis against the
    best live one; at the last step, the best two finished hypotheses)."""

    def __init__(self, params):
        self.p = params
        self.states: dict[int, list] = {}
        self.margins: dict[int, list] = {}
        self.finished: dict[int, list] = {}
        self.ended_at: dict[int, int] = {}
        self.step = 0

    def before(self, rows):
        for rid in {r.request_id for r in rows}:
            hyps = tuple(sorted(tuple(r.token_ids) for r in rows if r.request_id == rid))
            self.states.setdefault(rid, []).append(hyps)

    def after(self, rows, top, ids):
        p, nb = self.p, self.p.num_beams
        eos = set(p.eos_ids())
        i = 0
        while i < len(rows):
            rid = rows[i].request_id
            j = i
            while j < len(rows) and rows[j].request_id == rid:
                j += 1
            cands = sorted(((rows[r].cum_logprob + float(top[r, c]), r, int(ids[r, c]))
                            for r in range(i, j) for c in range(top.shape[1])),
                           key=lambda c: -c[0])
            vals = [c[0] for c in cands]
            margin = vals[nb - 1] - vals[nb] if len(vals) > nb else math.inf
            fin = self.finished.setdefault(rid, [])
            live = []
            for rank, (value, r, tok) in enumerate(cands):
                if rank >= nb and len(live) >= nb:
                    break
                generated = len(rows[r].token_ids)  # the start token counts as the prompt
                if tok in eos or generated >= p.max_tokens:
                    if rank < nb:
                        fin.append(value / max(generated, 1) ** p.length_penalty)
                elif len(live) < nb:
                    live.append(value / max(generated, 1) ** p.length_penalty)
            fin.sort(reverse=True)
            del fin[nb:]
            done = not live
            if not done and len(fin) >= nb:
                if p.early_stopping:
                    done = True
                else:
                    margin = min(margin, abs(fin[-1] - max(live)))
                    done = fin[-1] >= max(live)
            if done:
                if len(fin) >= 2:
                    margin = min(margin, fin[0] - fin[1])
                self.ended_at[rid] = self.step
            self.margins.setdefault(rid, []).append(margin)
            i = j
        self.step += 1


def first_divergence(a: list, b: list):
    """The first decision step whose outcome differs between two per-step state lists
    (a list that ends earlier ended at that step)."""
    for t in range(1, max(len(a), len(b))):
        sa = a[t] if t < len(a) else None
        sb = b[t] if t < len(b) else None
        if sa != sb:
            return t - 1
    return None


def run(llm, ops, requests, params, teacher_forced: bool):
    """Generate with a recorder on every step; with ``teacher_forced`` the committed
    forward is the reference one, after a HIP forward on the same state whose logits
    are compared.  Returns (tokens, recorder, per-step deltas)."""
    from vflorence_amd import SamplingParams

    runner, sched = llm.runner, llm.scheduler
    sp = SamplingParams(**params).with_defaults(llm._sampling_params)
    rec, deltas, ulps = BeamRecorder(sp), [], []
    real_run, model = runner.run, runner.model
    rows_now = []
    step_logits = {}

    def forward(input_ids, positions):
        if not teacher_forced:
            return model(input_ids, positions)
        ops.mode = "hip"
        step_logits["hip"] = model(input_ids, positions).float()
        ops.mode = "ref"
        return model(input_ids, positions)

    def recorded_run(batch):
        rows_now[:] = sched.running
        rec.before(rows_now)
        out = real_run(batch)
        if out is None:
            return out
        top, ids = out
        rec.after(rows_now, top, ids)
        if teacher_forced:
            n = batch.num_rows
            xa, xb = step_logits["hip"][:n], step_logits["ref"][:n]
            a = torch.log_softmax(xa, dim=-1)
            b = torch.log_softmax(xb, dim=-1)
            cand = b.topk(2 * sp.num_beams, dim=-1).indices
            deltas.append(float((a.gather(1, cand) - b.gather(1, cand)).abs().max()))
            ca, cb = xa.gather(1, cand), xb.gather(1, cand)
            # bf16 keeps 8 significant bits: a logit in [2^e, 2^(e+1)) rounds to 2^(e-7).
            # The unit is that step for the row's largest candidate logit: a change of
            # the hidden state moves the row's logits by similar absolute amounts.
            mag = torch.maximum(ca.abs(), cb.abs()).amax(dim=1, keepdim=True)
            ulp = torch.exp2(torch.floor(torch.log2(mag.clamp_min(2.0**-100))) - 7)
            ulps.append(float(((ca - cb).abs() / ulp).max()))
        return out

    def forward_keep(input_ids, positions):
        logits = forward(input_ids, positions)
        step_logits["ref"] = logits.float()
        return logits

    runner.run, runner.decode_fn = recorded_run, forward_keep
    try:
        outs = llm.generate([__import__("vflorence_amd").Request(p) for p in requests], sp)
    finally:
        runner.run, runner.decode_fn = real_run, model
        ops.mode = "hip"
    return [o.completion_token_ids for o in outs], rec, deltas, ulps


def engine(fx, dtype, **limits):
    from transformers import BartConfig

    from vflorence_amd import LLM
    from vflorence_amd.utils.loader import state_dict_checksum, synthetic_state_dict

    cfg = BartConfig(**fx["config"])
    sd = synthetic_state_dict(cfg, seed=0, device="cuda")
    if fx.get("eos_bias"):
        flb = sd["final_logits_bias"].clone()
        flb[0, cfg.eos_token_id] += fx["eos_bias"]
        sd["final_logits_bias"] = flb
    assert state_dict_checksum(sd) == fx["checksum"], "GPU-made weights differ from the fixture's"
    return LLM(cfg, state_dict=sd, dtype=dtype, cuda_graphs=False, **limits)


CASES = {  # fixture, case, engine limits
    "bart_large_beam4": ("bart_large", "beam4", dict(max_num_seqs=32, max_decoder_len=24,
                                                      max_encoder_len=1024)),
    "bart_large_beam4_fused": ("bart_large", "beam4_fused",
                               dict(max_num_seqs=32, max_decoder_len=24, max_encoder_len=1024)),
    "florence2_base_beam3": ("florence2_base", "beam3",
                             dict(max_num_seqs=18, max_decoder_len=32, max_encoder_len=587)),
    "bart_large_beam4_eos": ("bart_large_eos", "beam4_eos",
                             dict(max_num_seqs=32, max_decoder_len=24, max_encoder_len=1024)),
    "florence2_base_beam3_eos_early": ("florence2_base_eos", "beam3_eos_early",
                                       dict(max_num_seqs=18, max_decoder_len=32,
                                            max_encoder_len=587)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_bf16_beam_tokens_differ_only_where_attention_rounding_can_flip(name, monkeypatch):
    from vflorence_amd import hip_attn
    from vflorence_amd.layers import attention

    fixture, case, limits = CASES[name]
    fx = fixtures()[fixture]
    c = fx["cases"][case]
    prompts = c.get("prompts", fx.get("prompts"))
    ops = AttentionOps(hip_attn)
    monkeypatch.setattr(attention, "hip_attn", ops)
    llm = engine(fx, torch.bfloat16, **limits)
    got_a, rec_a, _, _ = run(llm, ops, prompts, c["params"], teacher_forced=False)
    got_b, rec_b, deltas, ulps = run(llm, ops, prompts, c["params"], teacher_forced=True)

    print(f"[attention A/B] {name}: one-step attention change of a candidate's log-prob: "
          f"max {max(deltas):.4f}, mean {np.mean(deltas):.4f} over {len(deltas)} steps; of "
          f"its bf16 logit: at most {max(ulps):.2f} rounding steps", flush=True)
    assert max(ulps) <= STEP_ULPS, f"attention moved a candidate logit by {max(ulps):.2f} ulp"
    # the recorder's restatement of the engine's finishing rule agrees with the engine
    for rid, states in rec_b.states.items():
        assert rec_b.ended_at[rid] == len(states) - 1, rid

    # request ids run on across the two generate calls: map each run's in order
    ids_a, ids_b = sorted(rec_a.states), sorted(rec_b.states)
    assert len(ids_a) == len(ids_b) == len(got_a)
    same, report = 0, []
    for r, (a, b) in enumerate(zip(got_a, got_b)):
        sa, sb, mb = rec_a.states[ids_a[r]], rec_b.states[ids_b[r]], rec_b.margins[ids_b[r]]
        t = first_divergence(sa, sb)
        if a == b and t is None:
            same += 1
            continue
        if t is None:  # same hypotheses throughout, another finished one returned
            t = len(sb) - 1
        bound = FLIP_FACTOR * sum(deltas[: t + 1])
        margin = mb[t]
        report.append(f"request {r}: first diverging decision at step {t}, reference margin "
                      f"{margin:.4f}, bound {bound:.4f}")
        assert margin < bound, report[-1]
    print(f"[attention A/B] {name}: {same}/{len(got_a)} requests token-identical"
          + ("; " + "; ".join(report) if report else ""), flush=True)
