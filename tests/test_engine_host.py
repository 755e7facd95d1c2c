"""Host-side engine logic on the CPU: logits rules against transformers' processors;
the native host core (block pool, admission, step metadata, greedy and beam updates)
against the reference's known answers and, step by step on random workloads, against
the oracle's restatement of the reference's bookkeeping (oracle/engine_host.py); the
synthetic checkpoint; and the BART encoder against transformers' (dense part only:
the decoder's paged attention needs the GPU)."""

import json
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.engine_host import HostOracle
from vflorence_amd.engine.block_manager import BlockManager
from vflorence_amd.engine.model_runner import launch_slots, row_buckets
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


# --------------------------------------------------------------------------------------
# the native host core
# --------------------------------------------------------------------------------------
def host_views(rows: int, width: int) -> dict:
    """Numpy buffers of one packed step (the pinned staging layout's fields)."""
    i64 = {k: np.zeros(rows, np.int64) for k in ("input_ids", "positions", "slots", "lengths",
                                                 "copy_src", "copy_dst", "row_requests")}
    i32 = dict(context_lens=np.zeros(rows, np.int32), order=np.zeros(rows, np.int32),
               group_start=np.zeros(rows + 1, np.int32), tables=np.zeros((rows, width), np.int32))
    return {**i64, **i32}


def config(max_num_seqs, num_blocks, block_size=16):
    return SimpleNamespace(max_num_seqs=max_num_seqs, num_blocks=num_blocks,
                           block_size=block_size)


def run_greedy(sched, tokens_for_step):
    """Drive ``sched`` to completion with host-made greedy tokens; returns outputs."""
    outs = {}
    step = 0
    while not sched.is_finished():
        batch = sched.schedule()
        toks = np.array([tokens_for_step(step, r) for r in range(batch.num_rows)], np.int64)
        outs.update(sched.postprocess(batch, toks))
        step += 1
    return outs


def test_exact_block_budget_fits():
    """A request whose tokens fill its one block exactly runs with a one-block pool
    (the reference's tests/test_engine.py:182-189)."""
    params = SamplingParams(max_tokens=16, min_length=17, eos_token_id=[2]).with_defaults(
        defaults())
    sched = Scheduler(config(max_num_seqs=1, num_blocks=1))
    sched.add(Sequence(0, [1], [3, 4, 5], params))
    outs = run_greedy(sched, lambda step, r: 5)
    assert len(outs[0].completion_token_ids) == 16
    bm = sched.block_manager
    assert bm.num_free_blocks == 1 and not any(bm.ref_counts)


def test_shared_beams_fit_two_blocks():
    """Two beams share their prompt block; with a two-block pool the copy-on-write of
    the shared partial block still fits (tests/test_engine.py:361-366)."""
    params = SamplingParams(max_tokens=3, num_beams=2, min_length=4, eos_token_id=[2]
                            ).with_defaults(defaults())
    sched = Scheduler(config(max_num_seqs=2, num_blocks=2))
    sched.add(Sequence(0, [1], [3, 4, 5], params))
    outs = {}
    while not sched.is_finished():
        batch = sched.schedule()
        rows = batch.num_rows
        scores = np.tile(np.array([[-0.1, -0.2, -0.3, -0.4]], np.float32), (rows, 1))
        ids = np.tile(np.array([[10, 11, 12, 13]], np.int64), (rows, 1))
        outs.update(sched.postprocess(batch, (scores, ids)))
    assert len(outs[0].completion_token_ids) == 3
    assert sched.block_manager.num_free_blocks == 2


def test_copy_budget_counts_a_shared_block_once_its_owner_left():
    """Two children of one parent share its block: both must copy while the parent
    holds it (2 new blocks); once the parent lets go, the last writer keeps it in place
    (1 new block) -- the reference's tests/test_engine.py:368-380."""
    params = SamplingParams().with_defaults(defaults())
    bm = BlockManager(8, 16)
    parent = Sequence(0, [1], [3], params)
    assert bm.ensure_capacity(parent) is None
    parent.num_cached_tokens = 1
    children = [parent.fork(4, 0.0), parent.fork(5, 0.0)]
    for child in children:
        bm.fork(parent, child)
    assert bm.required_new_blocks(children) == 2
    bm.deallocate(parent)
    assert bm.required_new_blocks(children) == 1


def test_copy_on_write_pair_and_counts():
    """A fork writing into its parent's shared block moves to a fresh block; the pair
    names both and each block keeps one holder (tests/test_engine.py:382-393)."""
    params = SamplingParams().with_defaults(defaults())
    bm = BlockManager(8, 16)
    parent = Sequence(0, [1], [3], params)
    assert bm.ensure_capacity(parent) is None
    parent.num_cached_tokens = 1
    child = parent.fork(4, 0.0)
    bm.fork(parent, child)
    src = parent.block_table[0]
    pair = bm.ensure_capacity(child)
    assert pair == (src, child.block_table[0]) and child.block_table == [pair[1]]
    assert (bm.ref_counts[src], bm.ref_counts[pair[1]]) == (1, 1)
    # free list: FIFO, freed blocks at the back, a table freed last block first
    bm.deallocate(parent)
    assert bm.free_block_ids[-1] == src
    with pytest.raises(RuntimeError, match="KV cache is full"):
        full = BlockManager(1, 16)
        a = Sequence(0, [1], [3], params)
        full.ensure_capacity(a)
        full.ensure_capacity(Sequence(1, [1], [3], params))


def test_beam_gate_reference_cases():
    """The reference's known answers for the EOS/rank gate (tests/test_beam.py:22-57):
    candidates taken in the listed rank order -- stopped ones (EOS) scored below the
    live ones so no early stop intervenes -- keep a stopped candidate only within the
    first num_beams ranks, and live ones fill num_beams running beams.  Pins the
    oracle's walk; the host core is held to the oracle on merged candidates below."""
    cases = json.load(open(os.path.join(GOLDEN, "reference_kats.json")))["beam_gate"]["cases"]
    for stopped, num_beams, want_finished, want_live in cases:
        eos = [100 + r for r in range(len(stopped))]
        orc = HostOracle(8, 16, 8)
        orc.add(0, [1], num_beams, 10, eos, 1.0, False)
        orc.schedule()
        parent = orc.running[0]
        cands = {0: [(parent, (100 + r) if s else r, (-10.0 - r) if s else -float(r))
                     for r, s in enumerate(stopped)]}
        outputs = orc.walk(cands)
        if outputs:
            best = outputs[0][1][-1] - 100
            finished, live = list(range(best, num_beams)), []
        else:
            finished = [h.tokens[-1] - 100 for h in orc.finished_beams[0]]
            live = [h.tokens[-1] for h in orc.running]
        assert (finished, live) == (want_finished, want_live), stopped


def test_beam_gate_on_the_host_core():
    """The gate's cases where the listed ranks are also the score order (every stopped
    candidate below the live ones, or none live): the host core keeps the same
    finished and live ranks."""
    for stopped, num_beams, want_finished, want_live in (
            ([False, False, True, True], 2, [], [0, 1]),
            ([True, True, True], 2, [0, 1], [])):
        eos = [100 + r for r in range(len(stopped))]
        params = SamplingParams(num_beams=num_beams, max_tokens=10, eos_token_id=eos,
                                early_stopping=False).with_defaults(defaults())
        ids = np.array([[(100 + r) if s else r for r, s in enumerate(stopped)]], np.int64)
        scores = -np.arange(len(stopped), dtype=np.float32)[None, :]
        sched = Scheduler(config(max_num_seqs=8, num_blocks=8))
        sched.add(Sequence(0, [1], [3], params))
        outputs = sched.postprocess(sched.schedule(), (scores, ids))
        if outputs:
            best = outputs[0][1].completion_token_ids[-1] - 100
            finished, live = list(range(best, num_beams)), []
        else:
            finished = [] if not sched.num_pending_beams else None
            live = [r.token_ids[-1] for r in sched.running]
        assert (finished, live) == (want_finished, want_live), stopped


def test_oracle_merge_equals_flattened_topk():
    """The oracle's per-request merge (each row's top-k plus its cumulative log-prob,
    best first) equals top-k over the request's flattened rows x vocab scores (the
    reference's tests/test_engine.py:250-277 check)."""
    torch.manual_seed(0)
    for eos, vocab in (([2], 32), ([2, 3, 4], 32), ([2], 5)):
        nb = 4
        keep = max(2, 1 + len(eos)) * nb
        rids = [0, 0, 0, 0, 1, 2, 2]
        cums = [-float(torch.rand(())) for _ in rids]
        scores = torch.log_softmax(torch.randn(len(rids), vocab), dim=-1)
        top, ids = torch.topk(scores, min(keep, vocab), dim=-1)
        orc = HostOracle(64, 16, 64)
        for rid in (0, 1, 2):
            orc.add(rid, [1], nb, 50, eos, 1.0, False)
        orc.schedule()
        # shape the running rows as the rids above, with the given cumulative scores
        proto = {h.rid: h for h in orc.running}
        orc.running = [proto[r].child(9, c) for r, c in zip(rids, cums)]
        for h in orc.running:
            h.tokens = h.tokens[:-1]
        merged = {}
        for r, h in enumerate(orc.running):
            vals = top[r].numpy().astype(np.float32) + np.float32(h.cum)
            merged.setdefault(h.rid, []).extend(
                (r, int(t), float(v)) for t, v in zip(ids[r].tolist(), vals))
        total = (scores + torch.tensor(cums).unsqueeze(-1)).float()
        for rid in (0, 1, 2):
            rows = [i for i, r in enumerate(rids) if r == rid]
            vals, idx = torch.topk(total[rows].flatten(), min(keep, len(rows) * vocab))
            want = [(rows[i // vocab], i % vocab) for i in idx.tolist()]
            got = sorted(merged[rid], key=lambda c: c[2], reverse=True)[:keep]
            assert [(r, t) for r, t, _ in got] == want


def test_scheduler_admission_counts_beams_and_keeps_beams_adjacent():
    params = SamplingParams(num_beams=3, max_tokens=8, eos_token_id=[]).with_defaults(defaults())
    sched = Scheduler(config(max_num_seqs=7, num_blocks=64))
    for r in range(3):
        sched.add(Sequence(r, [1], [3], params))
    batch = sched.schedule()
    assert [s.request_id for s in batch.fresh] == [0, 1] and batch.num_pairs == 0  # 3+3 <= 7 < 9
    scores = np.tile(-0.1 * np.arange(6, dtype=np.float32), (2, 1))
    ids = np.tile(10 + np.arange(6, dtype=np.int64), (2, 1))
    assert sched.postprocess(batch, (scores, ids)) == []
    batch = sched.schedule()
    assert [r.request_id for r in sched.running] == [0, 0, 0, 1, 1, 1]
    # three children share their parent's one block; all but the last writer copy it
    views = host_views(8, 4)
    # views too small, of another width, or of the wrong dtype are refused before the
    # host core writes into them
    with pytest.raises(ValueError):
        sched.core.pack(8, 4, 8, host_views(4, 4))
    with pytest.raises(ValueError):
        sched.core.pack(8, 4, 8, host_views(8, 2))
    with pytest.raises(ValueError):
        sched.core.pack(8, 4, 8, {**host_views(8, 4), "order": np.zeros(8, np.int64)})
    sched.core.pack(8, 4, 8, views)
    pairs = list(zip(views["copy_src"][:batch.num_pairs], views["copy_dst"][:batch.num_pairs]))
    assert batch.num_pairs == 4 and len({d for _, d in pairs}) == 4
    # an array replaced under its name is written, not the one it replaced
    old, views["copy_src"] = views["copy_src"], np.full(8, -7, np.int64)
    sched.core.pack(8, 4, 8, views)
    assert list(views["copy_src"][:4]) == list(old[:4])


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


def random_candidates(rng, rows, k, vocab, eos_rate):
    """Each row's best-first (scores, ids): distinct ids, scores on a 1/8 grid so exact
    ties occur inside and across rows; EOS (token 2) now and then."""
    ids = np.stack([rng.choice(np.arange(3, vocab), size=k, replace=False) for _ in range(rows)])
    eos = rng.random((rows, k)) < eos_rate
    ids[eos] = 2
    for r in range(rows):  # keep ids distinct after placing EOS
        seen = set()
        for c in range(k):
            while ids[r, c] in seen:
                ids[r, c] = rng.integers(3, vocab)
            seen.add(ids[r, c])
    scores = -np.sort(np.round(rng.exponential(1.5, (rows, k)) * 8) / 8, axis=1)
    return scores.astype(np.float32), ids.astype(np.int64)


@pytest.mark.parametrize("beams,early,lp,seed,shuffled", [
    (1, False, 1.0, 0, False), (1, False, 1.0, 1, False), (4, False, 1.0, 2, False),
    (4, True, 1.0, 3, False), (3, False, 2.0, 4, False), (4, False, -0.5, 5, False),
    (2, False, 1.0, 6, False), (8, False, 1.0, 7, False), (4, False, 1.0, 8, True),
    (3, True, 2.0, 9, True)])
def test_host_core_equals_the_oracle_step_by_step(beams, early, lp, seed, shuffled):
    """Continuous batching with seeded arrivals, greedy or beam search with random
    candidates: every step the core admits the same requests, packs the reference's
    metadata formulas, makes the same copy-on-write pairs, leaves the same holder
    counts and free list (order included), the same running rows (tokens, tables,
    cumulative scores) and finishes the same requests with the same tokens as the
    oracle's literal restatement.  ``shuffled``: each row's candidates come in a random
    order on half the rows (the core's sorting path instead of its merge of best-first
    rows)."""
    rng = np.random.default_rng(seed)
    bs, max_seqs, num_blocks = 16, 24, 200
    max_tokens = 40
    params = SamplingParams(num_beams=beams, max_tokens=max_tokens, eos_token_id=[2],
                            early_stopping=early, length_penalty=lp).with_defaults(defaults())
    sched = Scheduler(config(max_num_seqs=max_seqs, num_blocks=num_blocks))
    orc = HostOracle(num_blocks, bs, max_seqs)
    arrivals = sorted(rng.integers(0, 30, size=14).tolist())
    rid, step, seen_pairs, seen_groups = 0, 0, 0, 0
    keep = max(2, 1 + 1) * beams
    while arrivals or not sched.is_finished():
        while arrivals and arrivals[0] <= step:
            arrivals.pop(0)
            prompt = [1] if rng.random() < 0.7 else [1, 4]
            sched.add(Sequence(rid, prompt, [3], params))
            orc.add(rid, prompt, beams, max_tokens, [2], lp, early)
            rid += 1
        batch = sched.schedule()
        assert [s.request_id for s in batch.fresh] == orc.schedule()
        n = batch.num_rows
        assert n == len(orc.running)
        if n:
            padded = n + int(rng.integers(0, 3))
            views = host_views(padded, 8)
            grouped = sched.core.pack(padded, 8, 8, views)
            want = orc.metadata()
            for name in ("input_ids", "positions", "slots", "lengths", "context_lens",
                         "row_requests"):
                assert views[name][:n].tolist() == want[name], name
            for r, t in enumerate(want["tables"]):
                assert views["tables"][r].tolist() == t + [0] * (8 - len(t))
            assert not views["tables"][n:].any() and (views["slots"][n:] == -1).all()
            pairs = list(zip(views["copy_src"][:batch.num_pairs].tolist(),
                             views["copy_dst"][:batch.num_pairs].tolist()))
            assert pairs == orc.pairs
            seen_pairs += len(pairs)
            rids = want["row_requests"]
            if grouped:
                seen_groups += 1
                starts = views["group_start"]
                assert starts[0] == 0 and starts[-1] == padded
                for g in range(len(starts) - 1):  # each group: rows of one request
                    assert len({rids[r] for r in range(starts[g], min(starts[g + 1], n))}) <= 1
                # once every request runs all its beams (a new request runs one row on
                # its first step), the groups fit the runner's sized launches
                groups = int(np.searchsorted(starts, padded))
                per_request = [rids.count(q) for q in set(rids)]
                if all(c == beams for c in per_request):
                    assert groups <= launch_slots(padded, n - 1, beams, 8)
            else:
                order = views["order"][:padded].tolist()
                ctx = views["context_lens"][:padded].tolist()
                assert order == sorted(range(padded), key=lambda r: -ctx[r])
        bm = sched.block_manager
        assert bm.ref_counts == orc.pool.refs
        assert bm.free_block_ids == list(orc.pool.free)
        if n == 0:
            step += 1
            continue
        if beams == 1:
            toks = rng.integers(3, 60, n)
            toks[rng.random(n) < 0.05] = 2
            got, want = sched.postprocess(batch, toks), orc.greedy(toks)
        else:
            scores, ids = random_candidates(rng, n, keep, 60, 0.04)
            if shuffled:
                for r in np.flatnonzero(rng.random(n) < 0.5):
                    perm = rng.permutation(keep)
                    scores[r], ids[r] = scores[r][perm], ids[r][perm]
            got, want = sched.postprocess(batch, (scores, ids)), orc.beam(scores, ids)
        assert [(r, o.completion_token_ids) for r, o in got] == want
        rows = sched.running
        assert [(r.request_id, r.token_ids, r.block_table, r.num_cached_tokens)
                for r in rows] == [(h.rid, h.tokens, h.table, h.cached) for h in orc.running]
        assert [r.cum_logprob for r in rows] == [h.cum for h in orc.running]
        step += 1
    assert sched.block_manager.num_free_blocks == num_blocks
    assert rid == 14 and step > 10
    if beams > 1:
        assert seen_pairs > 0 and seen_groups > 0


@pytest.mark.parametrize("beams", [1, 2, 3, 4, 5, 8, 10])
def test_launch_slots_cover_every_batch_of_a_bucket(beams):
    """For every row bucket and every batch of whole requests that pads to it, the
    groups the packed step forms (requests cut every 8 rows, padding rows in groups of
    8) fit the launch's slots, and the slots are no more than the bucket's rows."""
    buckets = row_buckets(512)
    for i, padded in enumerate(buckets):
        below = buckets[i - 1] if i else 0
        slots = launch_slots(padded, below, beams, 8)
        assert slots <= padded
        for n in range(below + 1, padded + 1):
            if n % beams:
                continue
            groups = n // beams * -(-beams // 8) + -(-(padded - n) // 8)
            assert groups <= slots, (padded, n)
    assert launch_slots(256, 224, 4, 8) == 64  # 64 requests x 4 beams: 64 of 256 slots


def test_pool_full_raises_and_abort_frees_everything():
    """A step the pool cannot cover raises "KV cache is full" before any block moves;
    reset() returns every block (the engine's abort)."""
    params = SamplingParams(max_tokens=40, eos_token_id=[]).with_defaults(defaults())
    sched = Scheduler(config(max_num_seqs=4, num_blocks=3))
    for r in range(4):
        sched.add(Sequence(r, [1], [3], params))
    with pytest.raises(RuntimeError, match="KV cache is full"):
        sched.schedule()
    assert sched.block_manager.num_free_blocks == 3
    sched.reset()
    assert sched.is_finished() and sched.block_manager.free_block_ids == [0, 1, 2]


def test_pool_full_leaves_the_admission_queue_as_it_was():
    """A step the pool cannot cover raises before anything changes: the requests it was
    about to admit are still waiting, in order, so a caller that catches the error and
    makes room (here: aborts a request) steps on without a reset."""
    params = SamplingParams(max_tokens=40, eos_token_id=[]).with_defaults(defaults())
    sched = Scheduler(config(max_num_seqs=4, num_blocks=3))
    for r in range(4):
        sched.add(Sequence(r, [1], [3], params))
    for _ in range(2):  # the failure repeats identically
        with pytest.raises(RuntimeError, match="KV cache is full"):
            sched.schedule()
        assert sched.core.num_waiting == 4 and sched.num_running == 0
        assert [s.request_id for s in sched.waiting] == [0, 1, 2, 3]
        assert sched.block_manager.num_free_blocks == 3
    assert sched.abort_request(3)
    batch = sched.schedule()
    assert [s.request_id for s in batch.fresh] == [0, 1, 2] and batch.num_rows == 3
    assert sched.block_manager.num_free_blocks == 0


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


def test_packed_encoder_matches_transformers_per_prompt():
    """Prompts of several lengths stored back to back and encoded in one forward
    (attention per run of equal-length prompts) give each prompt transformers' encoder
    output on its own; segments that leave a gap or miss tokens are refused."""
    from transformers import BartConfig, BartForConditionalGeneration as HF

    from vflorence_amd.layers.bart import BartForConditionalGeneration, fuse_projections
    from vflorence_amd.utils.loader import synthetic_state_dict

    cfg = BartConfig(vocab_size=60, d_model=128, encoder_layers=2, decoder_layers=1,
                     encoder_attention_heads=2, decoder_attention_heads=2, encoder_ffn_dim=96,
                     decoder_ffn_dim=96, max_position_embeddings=80, tie_word_embeddings=False)
    sd = synthetic_state_dict(cfg, seed=5)
    hf = HF(cfg).eval()
    hf.load_state_dict(sd, strict=True)
    mine = BartForConditionalGeneration(cfg).eval()
    fused = dict(sd)
    fuse_projections(mine, fused)
    mine.load_state_dict(fused, strict=True)
    g = torch.Generator().manual_seed(1)
    # runs as the runner stores them: equal lengths adjacent, in first-seen order
    runs = [(37, 2), (12, 2), (5, 1), (64, 1)]
    prompts, segments, start = [], [], 0
    for length, count in runs:
        prompts += [torch.randint(3, 60, (length,), generator=g) for _ in range(count)]
        segments.append((start, count, length))
        start += count * length
    ids = torch.cat(prompts)
    positions = torch.cat([torch.arange(len(p)) for p in prompts])
    with torch.no_grad():
        got = mine.encode_packed(ids, positions, segments)
        at = 0
        for p in prompts:
            want = hf.model.encoder(input_ids=p[None]).last_hidden_state[0]
            torch.testing.assert_close(got[at: at + len(p)], want, rtol=1e-5, atol=1e-5)
            at += len(p)
        with pytest.raises(ValueError, match="does not start"):
            mine.encode_packed(ids, positions, [(0, 2, 37), (80, 2, 12)])
        with pytest.raises(ValueError, match="segments cover"):
            mine.encode_packed(ids, positions, segments[:-1])


def test_request_runs_are_the_page_comparison_groups():
    """The runner's cross-attention groups from the rows' request ids equal
    ``beam_groups``' runs of rows sharing encoder pages (cut at 8 rows), padding rows
    included, over random batches of 1-12 beams per request."""
    from vflorence_amd.engine.model_runner import request_runs
    from vflorence_amd.layers.attention import beam_groups

    rng = np.random.default_rng(7)
    empty = torch.zeros(0, dtype=torch.int32)
    for _ in range(200):
        rows, pages, lens, page = [], [], [], 0
        for rid in rng.permutation(40)[: int(rng.integers(1, 12))]:
            beams, length = int(rng.integers(1, 13)), int(rng.integers(1, 300))
            mine = torch.arange(page, page + -(-length // 16), dtype=torch.int32)
            page += len(mine)
            rows += [int(rid)] * beams
            pages += [mine] * beams
            lens += [length] * beams
        n = len(rows)
        padded = n + int(rng.integers(0, 20))
        want = beam_groups(pages + [empty] * (padded - n), lens + [0] * (padded - n))
        assert request_runs(np.asarray(rows, np.int64), padded, 8) == want


def test_page_table_fill_matches_row_by_row():
    """The staging's one-scatter page table equals filling it row by row, zero-padded,
    for tensors, numpy arrays and rows repeating one object; rows past the batch keep
    what they held."""
    from vflorence_amd.layers.attention import _fill_page_table

    rng = np.random.default_rng(3)
    table = rng.integers(1, 9, (40, 12)).astype(np.int32)
    before = table.copy()
    shared = torch.tensor([5, 6, 7], dtype=torch.int32)
    pages = [shared, shared, np.array([1, 2], np.int32), torch.zeros(0, dtype=torch.int32),
             np.arange(12, dtype=np.int32), [3, 4, 9]]
    _fill_page_table(table, pages)
    for i, p in enumerate(pages):
        p = np.asarray(p.numpy() if isinstance(p, torch.Tensor) else p)
        assert table[i, : len(p)].tolist() == p.tolist() and not table[i, len(p):].any()
    assert (table[len(pages):] == before[len(pages):]).all()
    _fill_page_table(table, [torch.zeros(0, dtype=torch.int32)] * 3)
    assert not table[:3].any()
