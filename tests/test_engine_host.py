"""Host-side engine logic on the CPU: logits rules against transformers' processors,
beam-candidate selection, the scheduler's beam gate (the reference's known answers),
block-manager invariants, the synthetic checkpoint, and the BART encoder against
transformers' (dense part only: the decoder's paged attention needs the GPU)."""

import json
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from vflorence_amd.engine.block_manager import BlockManager
from vflorence_amd.engine.scheduler import Scheduler
from vflorence_amd.engine.sequence import Sequence
from vflorence_amd.layers.logits_processor import LogitsProcessor
from vflorence_amd.sampling_params import SamplingParams

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
VOCAB = 41
EOS = [2, 7]


def defaults():
    from transformers import GenerationConfig

    return SamplingParams.from_generation_config(GenerationConfig())


def hf_rules(params, history, scores, max_length, begin_index):
    """transformers' processors for ``params`` over one row's unpadded history."""
    from transformers import LogitsProcessorList
    from transformers.generation import logits_process as lp

    procs = LogitsProcessorList()
    if params.repetition_penalty != 1.0:
        procs.append(lp.RepetitionPenaltyLogitsProcessor(params.repetition_penalty))
    if params.no_repeat_ngram_size > 0:
        procs.append(lp.NoRepeatNGramLogitsProcessor(params.no_repeat_ngram_size))
    if params.min_length > 0:
        procs.append(lp.MinLengthLogitsProcessor(params.min_length, sorted(EOS)))
    if params.forced_bos_token_id is not None:
        procs.append(lp.ForcedBOSTokenLogitsProcessor(params.forced_bos_token_id))
    if params.forced_eos_token_id is not None:
        procs.append(lp.ForcedEOSTokenLogitsProcessor(max_length, params.forced_eos_token_id))
    if params.suppress_tokens:
        procs.append(lp.SuppressTokensLogitsProcessor(params.suppress_tokens))
    if params.begin_suppress_tokens:
        procs.append(lp.SuppressTokensAtBeginLogitsProcessor(params.begin_suppress_tokens,
                                                             begin_index))
    return procs(history, scores)


RULES = [
    {},
    dict(repetition_penalty=1.7),
    dict(repetition_penalty=0.6),
    dict(no_repeat_ngram_size=1),
    dict(no_repeat_ngram_size=2),
    dict(no_repeat_ngram_size=3),
    dict(min_length=4),
    dict(forced_bos_token_id=5),
    dict(forced_eos_token_id=[3, 9]),
    dict(suppress_tokens=[1, 4, 40]),
    dict(begin_suppress_tokens=[0, 6]),
    dict(repetition_penalty=1.3, no_repeat_ngram_size=2, min_length=6, forced_bos_token_id=8,
         forced_eos_token_id=2, suppress_tokens=[11], begin_suppress_tokens=[12]),
]


@pytest.mark.parametrize("rule", range(len(RULES)))
def test_logits_rules_match_transformers_on_ragged_rows(rule):
    params = SamplingParams(eos_token_id=EOS, **RULES[rule]).with_defaults(defaults())
    max_length, begin_index = 9, 2
    g = torch.Generator().manual_seed(rule)
    lengths = [1, 2, 3, 4, 5, 8, 2, 7]
    # small alphabet so n-grams repeat
    histories = [torch.randint(0, 6, (n,), generator=g) for n in lengths]
    scores = torch.randn(len(lengths), VOCAB, generator=g) * 3
    width = max(lengths)
    padded = torch.stack([torch.cat([torch.full((width - len(h),), -1), h]) for h in histories])
    proc = LogitsProcessor(params, vocab_size=VOCAB, max_length=max_length,
                           begin_index=begin_index, device="cpu")
    got = proc(padded if proc.needs_history else None, scores.clone(),
               torch.tensor(lengths, dtype=torch.long))
    for r, h in enumerate(histories):
        want = hf_rules(params, h.unsqueeze(0), scores[r:r + 1].clone(), max_length, begin_index)
        torch.testing.assert_close(got[r:r + 1], want, rtol=0, atol=0)


def test_out_of_vocab_rule_tokens_are_dropped():
    params = SamplingParams(eos_token_id=[2, 500], suppress_tokens=[3, 999], min_length=5,
                            forced_bos_token_id=700).with_defaults(defaults())
    proc = LogitsProcessor(params, vocab_size=VOCAB, max_length=9, begin_index=1, device="cpu")
    scores = torch.zeros(2, VOCAB)
    proc(None, scores, torch.tensor([1, 2]))
    assert proc.forced_bos is None
    assert torch.isinf(scores[:, 3]).all() and torch.isinf(scores[:, 2]).all()
    assert torch.isfinite(scores[:, 4]).all()


def beam_search(seqs, scores, params):
    from vflorence_amd.engine.model_runner import ModelRunner

    return ModelRunner._beam_search(None, seqs, scores, params)


def test_beam_candidates_match_flattened_topk():
    """Per-row top-k, then a per-request merge == top-k over the request's flattened
    (rows x vocab) scores (the reference's test_engine.py:250-277 check)."""
    torch.manual_seed(0)
    for eos, vocab in (([2], 32), ([2, 3, 4], 32), ([2], 5)):
        params = SamplingParams(num_beams=4, eos_token_id=eos).with_defaults(defaults())
        keep = max(2, 1 + len(eos)) * 4
        seqs = [Sequence(r, [1], [3], params) for r in (0, 0, 0, 0, 1, 2, 2)]
        for seq in seqs:
            seq.cum_logprob = -torch.rand(()).item()
        scores = torch.log_softmax(torch.randn(len(seqs), vocab), dim=-1)
        scores[-1, :2] = float("-inf")
        got = beam_search(seqs, scores.clone(), params)
        total = scores + torch.tensor([s.cum_logprob for s in seqs]).unsqueeze(-1)
        for rid in (0, 1, 2):
            rows = [i for i, s in enumerate(seqs) if s.request_id == rid]
            values, idx = torch.topk(total[rows].flatten(), min(keep, len(rows) * vocab))
            want = [(rows[i // vocab], i % vocab, v) for i, v in zip(idx.tolist(), values.tolist())]
            row_of = {id(s): i for i, s in enumerate(seqs)}
            assert [(row_of[id(p)], t, c) for p, t, c in got[rid]] == want


def test_beam_gate_reference_cases():
    """The reference's known answers for the EOS/rank gate (tests/test_beam.py:22-32)."""
    cases = json.load(open(os.path.join(GOLDEN, "reference_kats.json")))["beam_gate"]["cases"]
    for stopped, num_beams, want_finished, want_live in cases:
        eos = [100 + r for r in range(len(stopped))]
        params = SamplingParams(num_beams=num_beams, max_tokens=10, eos_token_id=eos,
                                early_stopping=False).with_defaults(defaults())
        sched = Scheduler(SimpleNamespace(max_num_seqs=8, num_blocks=8, block_size=16))
        parent = Sequence(0, [1], [3], params)
        sched.add(parent)
        seqs, _ = sched.schedule()
        cands = [(parent, (100 + r) if s else r, (-10.0 - r) if s else -float(r))
                 for r, s in enumerate(stopped)]
        outputs = sched.postprocess(seqs, {0: cands})
        if outputs:
            best = outputs[0][1].completion_token_ids[-1] - 100
            finished, live = list(range(best, num_beams)), []
        else:
            finished = [s.completion_token_ids[-1] - 100 for s in sched._finished_beams[0]]
            live = [s.completion_token_ids[-1] for s in sched.running]
        assert (finished, live) == (want_finished, want_live), stopped


def test_scheduler_admission_counts_beams_and_keeps_beams_adjacent():
    params = SamplingParams(num_beams=3, max_tokens=8, eos_token_id=[]).with_defaults(defaults())
    sched = Scheduler(SimpleNamespace(max_num_seqs=7, num_blocks=64, block_size=16))
    for r in range(3):
        sched.add(Sequence(r, [1], [3], params))
    seqs, copies = sched.schedule()
    assert [s.request_id for s in seqs] == [0, 1] and not copies  # 3 + 3 <= 7 < 9
    cands = {r: [(seqs[r], 10 + k, -0.1 * k) for k in range(6)] for r in (0, 1)}
    assert sched.postprocess(seqs, cands) == []
    seqs, copies = sched.schedule()
    assert [s.request_id for s in seqs] == [0, 0, 0, 1, 1, 1]
    # three children share their parent's one block; all but the last writer copy it
    assert len(copies) == 4 and len({d for _, d in copies}) == 4


def test_block_manager_invariants_under_random_forks():
    import random

    rng = random.Random(0)
    bm = BlockManager(64, 16)
    params = SamplingParams(max_tokens=200, eos_token_id=[]).with_defaults(defaults())
    live = [Sequence(0, [1], [3], params)]
    for step in range(120):
        for seq in live:
            bm.ensure_capacity(seq)
            seq.num_cached_tokens += 1
            seq.append_token(5)
        if len(live) < 4 and rng.random() < 0.3:
            parent = rng.choice(live)
            child = parent.fork(6)
            child.num_cached_tokens = parent.num_cached_tokens
            bm.fork(parent, child)
            live.append(child)
        if len(live) > 1 and rng.random() < 0.1:
            bm.deallocate(live.pop(rng.randrange(len(live))))
        used = {b for s in live for b in s.block_table}
        assert sum(bm.ref_counts) == sum(len(s.block_table) for s in live)
        assert bm.num_free_blocks + len(used) == bm.num_blocks
        for s in live:  # every row's write block is private after ensure_capacity
            assert bm.ref_counts[s.block_table[(s.num_cached_tokens - 1) // 16]] >= 1
    for s in live:
        bm.deallocate(s)
    assert bm.num_free_blocks == 64 and not any(bm.ref_counts)


class _ForkAllScheduler(Scheduler):
    """The reference's beam bookkeeping verbatim in effect: fork every live child from
    its parent, then deallocate every parent (vflorence/engine/scheduler.py:120-126)."""

    def _postprocess_beam(self, seqs, candidates_by_request):
        outputs = []
        for request_id, candidates in candidates_by_request.items():
            sp = candidates[0][0].sampling_params
            finished = self._finished_beams[request_id]
            live = []
            for rank, (parent, token, cum) in enumerate(candidates):
                if rank >= sp.num_beams and len(live) >= sp.num_beams:
                    break
                child = parent.fork(token, cum)
                if token in sp.eos_ids() or child.num_generated >= sp.max_tokens:
                    if rank < sp.num_beams:
                        finished.append(child)
                elif len(live) < sp.num_beams:
                    live.append((parent, child))
            finished.sort(key=lambda q: q.score, reverse=True)
            del finished[sp.num_beams:]
            best = max((c.score for _, c in live), default=float("-inf"))
            if not live or (len(finished) >= sp.num_beams and (
                    sp.early_stopping or finished[-1].score >= best)):
                self._finished_beams.pop(request_id, None)
                outputs.append((request_id, finished[0].to_output()))
            else:
                for parent, child in live:
                    self.block_manager.fork(parent, child)
                    self.running.append(child)
        for seq in seqs:
            self.running.remove(seq)
            self.block_manager.deallocate(seq)
        return outputs


@pytest.mark.parametrize("early_stopping,length_penalty", [(False, 1.0), (True, 1.0),
                                                             (False, 2.0), (False, -0.5)])
def test_beam_table_handover_keeps_the_reference_block_state(early_stopping, length_penalty):
    """Handing a parent's table to its first live child instead of fork + deallocate,
    and forking only the candidates that are kept, leave every step's block tables,
    copy-on-write pairs, reference counts, free list (order included) and outputs
    identical to forking every child."""
    import random

    def run(cls, seed):
        rng = random.Random(seed)
        params = SamplingParams(num_beams=4, max_tokens=60, eos_token_id=[2],
                                early_stopping=early_stopping,
                                length_penalty=length_penalty).with_defaults(defaults())
        sched = cls(SimpleNamespace(max_num_seqs=24, num_blocks=160, block_size=16))
        for r in range(6):
            sched.add(Sequence(r, [1], [3], params))
        trace = []
        while not sched.is_finished():
            seqs, copies = sched.schedule()
            bm = sched.block_manager
            trace.append(([list(s.block_table) for s in seqs], list(copies),
                          list(bm.ref_counts), list(bm.free_block_ids)))
            cands = {}
            for s in seqs:
                row = []
                for _ in range(3):  # a few children per parent, EOS now and then
                    tok = 2 if rng.random() < 0.03 else rng.randrange(3, 50)
                    row.append((s, tok, s.cum_logprob - rng.random()))
                cands.setdefault(s.request_id, []).extend(row)
            for rid in cands:
                cands[rid].sort(key=lambda c: -c[2])
            outs = sched.postprocess(seqs, cands)
            trace.append(sorted((rid, o.completion_token_ids) for rid, o in outs))
        return trace

    for seed in range(4):
        assert run(Scheduler, seed) == run(_ForkAllScheduler, seed)


def test_synthetic_checkpoint_is_deterministic_and_loads_into_transformers():
    from transformers import BartConfig, BartForConditionalGeneration

    from vflorence_amd.utils.loader import state_dict_checksum, synthetic_state_dict

    cfg = BartConfig(vocab_size=50, d_model=128, encoder_layers=1, decoder_layers=1,
                     encoder_attention_heads=2, decoder_attention_heads=2, encoder_ffn_dim=64,
                     decoder_ffn_dim=64, max_position_embeddings=64, tie_word_embeddings=False)
    a, b = synthetic_state_dict(cfg, seed=0), synthetic_state_dict(cfg, seed=0)
    assert state_dict_checksum(a) == state_dict_checksum(b)
    assert state_dict_checksum(a) != state_dict_checksum(synthetic_state_dict(cfg, seed=1))
    assert torch.equal(a["model.encoder.embed_tokens.weight"], a["model.shared.weight"])
    assert not torch.equal(a["lm_head.weight"], a["model.shared.weight"])
    w = a["model.decoder.layers.0.fc1.weight"]
    assert abs(w.std().item() - 0.02) < 2e-3 and abs(w.mean().item()) < 2e-3
    BartForConditionalGeneration(cfg).load_state_dict(a, strict=True)


def test_encoder_matches_transformers():
    """The dense half of the model, on the CPU: fused-projection loading + encoder."""
    from transformers import BartConfig, BartForConditionalGeneration as HF

    from vflorence_amd.layers.bart import BartForConditionalGeneration, fuse_projections
    from vflorence_amd.utils.loader import synthetic_state_dict

    cfg = BartConfig(vocab_size=60, d_model=128, encoder_layers=2, decoder_layers=1,
                     encoder_attention_heads=2, decoder_attention_heads=2, encoder_ffn_dim=96,
                     decoder_ffn_dim=96, max_position_embeddings=80, tie_word_embeddings=False)
    sd = synthetic_state_dict(cfg, seed=4)
    hf = HF(cfg).eval()
    hf.load_state_dict(sd, strict=True)
    mine = BartForConditionalGeneration(cfg).eval()
    fused = dict(sd)
    fuse_projections(mine, fused)
    mine.load_state_dict(fused, strict=True)
    ids = torch.randint(3, 60, (3, 37), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        want = hf.model.encoder(input_ids=ids).last_hidden_state
        got = mine.encode(ids)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_vectorised_beam_merge_equals_the_general_merge():
    """Equal-size adjacent beam groups take the vectorised merge; it must list the same
    candidates in the same order as the row-by-row stable sort, ties included."""
    from vflorence_amd.engine import model_runner as mr

    params = SamplingParams(num_beams=3, eos_token_id=[2]).with_defaults(defaults())
    g = torch.Generator().manual_seed(3)
    for rows_per_req, vocab in ((3, 40), (1, 40), (3, 4)):
        seqs = [Sequence(r, [1], [3], params) for r in range(5) for _ in range(rows_per_req)]
        for s in seqs:
            s.cum_logprob = -float(torch.rand((), generator=g))
        scores = torch.log_softmax(torch.randn(len(seqs), vocab, generator=g), dim=-1)
        scores[:, 5:9] = -1.0  # exact ties inside and across rows
        scores[1, :] = float("-inf")
        keep = max(2, 1 + len(params.eos_ids())) * params.num_beams
        top, ids = torch.topk(scores, min(keep, vocab), dim=-1)
        top = top + torch.tensor([s.cum_logprob for s in seqs]).unsqueeze(-1)
        fast = mr._merge_equal_beam_groups(seqs, top.numpy(), ids.numpy(), keep)
        assert fast is not None
        general = {}
        for s, row_s, row_i in zip(seqs, top.tolist(), ids.tolist()):
            general.setdefault(s.request_id, []).extend(zip([s] * len(row_i), row_i, row_s))
        for c in general.values():
            c.sort(key=lambda x: x[2], reverse=True)
            del c[keep:]
        assert fast == general
    # unequal or interleaved groups are left to the general merge
    seqs = [Sequence(r, [1], [3], params) for r in (0, 0, 1)]
    assert mr._merge_equal_beam_groups(seqs, np.zeros((3, 2), np.float32),
                                       np.zeros((3, 2), np.int64), 4) is None
    seqs = [Sequence(r, [1], [3], params) for r in (0, 1, 0, 1)]
    assert mr._merge_equal_beam_groups(seqs, np.zeros((4, 2), np.float32),
                                       np.zeros((4, 2), np.int64), 4) is None
