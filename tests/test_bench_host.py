"""bench.py's host-side pieces that decide what is timed (no GPU needed)."""

import bench


def test_timed_steps_cover_the_whole_schedule_whatever_the_count():
    """Any --steps walks the 128-step schedule from the first step to the last: whole
    passes in order, a shorter remainder at an even stride, no step replayed twice in a
    row (a repeat would read the blocks its predecessor just cached)."""
    for n in (1, 5, 20, 64, 127, 128, 129, 200, 256, 300):
        order = bench.schedule_order(n)
        assert len(order) == n
        assert all(0 <= t < bench.DECODE_STEPS for t in order)
        assert all(a != b for a, b in zip(order, order[1:]))
        # the first step and the schedule's end to within one stride
        assert order[0] == 0
        assert max(order) > bench.DECODE_STEPS - bench.DECODE_STEPS / min(n, 128) - 1
    assert bench.schedule_order(256) == list(range(128)) * 2
    assert bench.schedule_order(20)[:4] == [0, 6, 12, 19]
    full = bench.schedule_order(20)
    assert full[-1] >= 120  # the long-context end of the schedule is in the timed region


def test_cpu_baseline_threads_follow_affinity_and_environment(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    threads, host = bench.host_threads()
    assert threads == min(3, host["cores_in_affinity"]) and host["threads_used"] == threads
    monkeypatch.delenv("OMP_NUM_THREADS")
    threads, host = bench.host_threads()
    assert threads == host["cores_in_affinity"] and host["cpu_model"]
