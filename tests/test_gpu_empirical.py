"""The empirical single-tail model (hbf_device.cu:796-881) on the GPU against
the CPU oracle, bit-exact: burst runs of consecutive pages across tile
and run boundaries, saturation at 1023, reads and writes, bypass and
unsupported records in between, the hybrid sampler, split runs."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
import parity

pytestmark = pytest.mark.gpu

PROFILE = oracle_py.ROOT / "tests" / "golden" / "profiles" / "cd8p-vmem-p50.json"
BASE = 0x7E00_0000_0000
PAGE = 4096
RANGES = [(BASE, 64 << 20, 3), (BASE + (80 << 20), 16 << 20, 1)]
ORC_EMPIRICAL = 2


def burst_stream(n, seed):
    """Streaks of consecutive pages (lengths up to 1500, past the 1023 cap),
    repeated pages, jumps, writes, and records outside every range or
    crossing a page."""
    rng = np.random.default_rng(seed)
    rec = np.zeros((n, 4), np.uint64)
    i, t = 0, 0
    pages0 = (64 << 20) // PAGE
    while i < n:
        length = int(rng.choice([1, 2, 3, 7, 64, 300, 1100, 1500]))
        start = int(rng.integers(0, pages0 - length))
        op = 1 if rng.random() < 0.2 else 0
        for k in range(length):
            if i >= n:
                break
            page = start + k
            if rng.random() < 0.03:
                page = start + max(0, k - 1)  # same page again: the streak restarts
            addr = BASE + page * PAGE + int(rng.integers(0, 32)) * 128
            nbytes = 128
            r = rng.random()
            if r < 0.01:
                addr = BASE + (70 << 20) + k * 64  # outside every range: bypass
            elif r < 0.015:
                addr = BASE + page * PAGE + PAGE - 64  # crosses the page: unsupported
            t += int(rng.integers(0, 3000))
            rec[i] = (addr, nbytes, t, op)
            i += 1
    return rec


def make_pair(mode="fast", **opts):
    p = parity.Pair(PROFILE, RANGES, mode=mode, **opts)
    assert p.engine.options()["model"] == 1  # EMPIRICAL, chosen by the profile
    p.params.model = ORC_EMPIRICAL
    return p


def check_burst(p):
    st = p.engine.state()
    assert st["burst_state"] == p.ostate.s.burst_state
    assert st["sequence"] == p.ostate.s.modeled_sequence
    np.testing.assert_array_equal(st["channel_cursor"][:1], p.ostate.channel_cursor[:1])
    _, gc = p.engine.busy_totals()
    np.testing.assert_array_equal(gc[:1], p.ostate.channel_busy_total[:1])


@pytest.mark.parametrize("n,seed", [(1, 1), (37, 2), (4096, 3), (50_000, 4), (200_003, 5)])
def test_empirical_bit_exact(n, seed):
    rec = burst_stream(n, seed)
    p = make_pair()
    try:
        g, c = p.run(rec)
        parity.assert_same(g, c, f"empirical n={n}")
        check_burst(p)
        # a second run continues the burst state and the tail
        rec2 = burst_stream(n, seed + 100)
        rec2[:, 2] += rec[-1, 2]
        g2, c2 = p.run(rec2, base_ps=0)
        parity.assert_same(g2, c2, "second run")
        check_burst(p)
    finally:
        p.close()


def test_empirical_streak_across_runs_and_saturation():
    """One 3000-page streak split over three runs: runs reach the 1023 cap
    and keep it across run boundaries."""
    n = 3000
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = BASE + np.arange(n, dtype=np.uint64) * PAGE
    rec[:, 1] = 4096
    rec[:, 2] = np.arange(n, dtype=np.uint64) * 1000
    p = make_pair()
    try:
        for a, b in ((0, 700), (700, 1800), (1800, n)):
            g, c = p.run(rec[a:b])
            parity.assert_same(g, c, f"records {a}:{b}")
            check_burst(p)
        assert p.ostate.s.burst_state & 1023 == 1023
    finally:
        p.close()


def test_empirical_hybrid_sampling():
    rec = burst_stream(30_000, 9)
    p = make_pair(mode="hybrid")
    try:
        g, c = p.run(rec)
        parity.assert_same(g, c, "hybrid")
        assert c[2]["hybrid_sampled"] >= 1024  # the profile's warm-up requests
        check_burst(p)
    finally:
        p.close()
