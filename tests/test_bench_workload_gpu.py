"""The benchmarked decode workload itself, checked against the oracle.

bench.py times 64 requests x 4 beams at BART-large attention shapes in bf16 (16 heads
x 64, 16-token blocks, encoder lengths U[256, 1024]) over a 128-step beam search whose
forks make copy-on-write pairs every step, one captured HIP graph per decode step.
Here the same workload is built over 2 of its 12 layers (every layer of the bench is
the same computation on its own pools), the bench's own graphs are replayed in order,
and:

* at steps 0, 15, 16, 64 and 127 every row of self- and cross-attention output is
  compared with the float64 oracle (bf16: 2e-2 absolute);
* every self-attention pool on the device equals, bit for bit, a host mirror to which
  the oracle's copy_blocks and reshape_and_cache were applied step by step;
* the schedule's copy-on-write volume is the bench's definition: round(10% of the
  blocks in use) pairs after each step, at most beams - 1 forks per request, about 48
  pairs per step.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CHECK_STEPS = (0, 15, 16, 64, 127)
LAYERS = 2
TOL = dict(rtol=0.0, atol=2e-2)


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def as_f64(bits: np.ndarray) -> np.ndarray:
    return orc.bf16_bits_to_f64(bits)


def cross_oracle(wl, layer: int) -> np.ndarray:
    """Cross-attention of one layer over the pages the rows use (gathered to the host,
    tables renumbered into the gathered pool)."""
    from vflorence_amd import hip_attn

    attn = wl["layers"][layer].encoder_attn
    used = sorted({int(p) for pages in wl["pages"] for p in pages.tolist()})
    index = {p: i for i, p in enumerate(used)}
    sel = torch.tensor(used, dtype=torch.int64, device=attn.k_cache.device)
    k = as_f64(host_bits(attn.k_cache.index_select(0, sel)))
    v = as_f64(host_bits(hip_attn.v_cache_logical(attn.v_cache.index_select(0, sel))))
    width = max(len(p) for p in wl["pages"])
    table = np.zeros((len(wl["pages"]), width), dtype=np.int32)
    for r, pages in enumerate(wl["pages"]):
        table[r, : len(pages)] = [index[int(p)] for p in pages.tolist()]
    q = as_f64(host_bits(wl["qc"][layer]))
    lens = np.array(wl["enc_rows"], dtype=np.int32)
    return orc.paged_attention(q, k, v, lens, table, 64**-0.5)


def test_benchmarked_beam_workload_matches_the_oracle():
    import bench
    from vflorence_amd import hip_attn

    wl = bench.build_workload(torch, seed=0, num_layers=LAYERS)
    plans = wl["plans"]
    rows = bench.REQUESTS * bench.BEAMS
    assert len(plans) == bench.DECODE_STEPS and all(len(p.context_lens) == rows for p in plans)

    # copy-on-write volume of the schedule (the bench's definition)
    pairs = [len(p.copies) for p in plans]
    in_use = [len({b for t in p.block_tables for b in t}) for p in plans]
    for t in range(1, len(plans)):
        limit = min(round(0.1 * in_use[t - 1]), bench.REQUESTS * (bench.BEAMS - 1))
        assert pairs[t] <= limit
    assert 40 <= np.mean(pairs[1:]) <= 56, np.mean(pairs[1:])

    new_kv = []
    for i in range(LAYERS):
        qkv = host_bits(wl["qkv"][i]).reshape(rows, 3, 16, 64)
        new_kv.append((np.ascontiguousarray(qkv[:, 1]), np.ascontiguousarray(qkv[:, 2]),
                       as_f64(qkv[:, 0])))
    cross_want = [cross_oracle(wl, i) for i in range(LAYERS)]

    graphs, keep, outputs = bench.capture_steps(torch, wl, grouped=True, keep_outputs=True)
    assert len(graphs) == len(plans)
    # host mirror of the self-attention pools as the build left them (it launched every
    # step's graph once), V in logical order; the replays below start from there
    torch.cuda.synchronize()
    mirror = [[host_bits(L.self_attn.k_cache),
               host_bits(hip_attn.v_cache_logical(L.self_attn.v_cache))] for L in wl["layers"]]
    for t, plan in enumerate(plans):
        graphs[t].replay()
        for i in range(LAYERS):
            orc.copy_blocks(mirror[i], plan.copies)
            k, v, _ = new_kv[i]
            orc.reshape_and_cache(k, v, mirror[i][0], mirror[i][1],
                                  np.array(plan.slot_mapping, dtype=np.int64))
        if t not in CHECK_STEPS:
            continue
        torch.cuda.synchronize()
        print(f"[bench-workload] step {t}: {pairs[t]} copy pairs, contexts "
              f"{min(plan.context_lens)}..{max(plan.context_lens)}", flush=True)
        width = max(len(r) for r in plan.block_tables)
        table = np.zeros((rows, width), dtype=np.int32)
        for r, blocks in enumerate(plan.block_tables):
            table[r, : len(blocks)] = blocks
        lens = np.array(plan.context_lens, dtype=np.int32)
        for i, layer in enumerate(wl["layers"]):
            assert np.array_equal(host_bits(layer.self_attn.k_cache), mirror[i][0])
            assert np.array_equal(host_bits(hip_attn.v_cache_logical(layer.self_attn.v_cache)),
                                  mirror[i][1])
            self_out, cross_out = outputs[t][i]
            want = orc.paged_attention(new_kv[i][2], as_f64(mirror[i][0]), as_f64(mirror[i][1]),
                                       lens, table, 64**-0.5)
            got = as_f64(host_bits(self_out)).reshape(rows, 16, 64)
            np.testing.assert_allclose(got, want, **TOL)
            got = as_f64(host_bits(cross_out)).reshape(rows, 16, 64)
            np.testing.assert_allclose(got, cross_want[i], **TOL)
    del graphs, keep, outputs
