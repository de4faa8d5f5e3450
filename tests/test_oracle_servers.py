"""MediaServers::issue (prefetch_model.cpp:22-50) in the oracle, pinned
against an independent min-heap simulation (Python's heapq standing in for
std::priority_queue<..., std::greater>), and the closed form the GPU kernel
uses for non-decreasing issue times: k interleaved Lindley chains,
c_i = max(now_i, c_{i-k}) + L."""
from __future__ import annotations

import heapq

import numpy as np
import pytest

import oracle_py


def heap_servers(now, k, latency):
    free = [0] * max(1, k)
    heapq.heapify(free)
    out = []
    for t in now:
        earliest = heapq.heappop(free)
        done = max(int(t), earliest) + latency
        heapq.heappush(free, done)
        out.append(done)
    return out


def oracle_servers(now, k, latency):
    now = np.ascontiguousarray(now, np.uint64)
    out = np.zeros(max(len(now), 1), np.uint64)
    oracle_py.lib().orc_media_servers(now.ctypes.data, len(now), k, latency, out.ctypes.data)
    return out[:len(now)].tolist()


def chains(now, k, latency):
    k = max(1, k)
    c = []
    for i, t in enumerate(now):
        prev = c[i - k] if i >= k else 0
        c.append(max(int(t), prev) + latency)
    return c


@pytest.mark.parametrize("k", [1, 2, 3, 7, 64, 1000])
@pytest.mark.parametrize("sorted_", [True, False])
def test_oracle_matches_heap(k, sorted_):
    rng = np.random.default_rng(k)
    now = rng.integers(0, 50_000, 3000)
    if sorted_:
        now = np.sort(now)
    assert oracle_servers(now, k, 700) == heap_servers(now, k, 700)


@pytest.mark.parametrize("k", [0, 1, 2, 5, 31, 500, 5000])
def test_chains_equal_heap_for_non_decreasing_issue(k):
    rng = np.random.default_rng(k + 1)
    # bursts of equal times, idle gaps, and stretches busier than k servers
    gaps = rng.choice([0, 0, 0, 1, 3, 50, 4000], 4000)
    now = np.cumsum(gaps)
    for latency in (0, 1, 997, 10**6):
        assert chains(now, k, latency) == heap_servers(now, k, latency)


def test_chains_differ_for_out_of_order_issue():
    """Why the GPU kernel rejects decreasing issue times."""
    now = [100, 0, 0]
    assert heap_servers(now, 2, 10) != chains(now, 2, 10)


GOLDEN_PREFETCH = None


def golden_prefetch():
    import json
    import pathlib
    global GOLDEN_PREFETCH
    if GOLDEN_PREFETCH is None:
        path = pathlib.Path(__file__).parent / "golden" / "ref_vectors.json"
        GOLDEN_PREFETCH = json.loads(path.read_text())["prefetch"]
    return GOLDEN_PREFETCH


def oracle_prefetch(pages, cfg):
    pages = np.ascontiguousarray(pages, np.uint64)
    stats = np.zeros(7, np.uint64)
    rc = oracle_py.lib().orc_simulate_prefetch(pages.ctypes.data, len(pages), *cfg,
                                               stats.ctypes.data)
    return rc, stats.tolist()


def test_prefetch_simulation_matches_reference_vectors():
    """The reference's compiled simulate_prefetch (MediaServers and the
    staging buffer inside it), policies None and NextPage: 80 streams."""
    cases = golden_prefetch()
    assert len(cases) == 80 and any(c["config"][3] > 1 for c in cases)
    for c in cases:
        assert c["ok"] == 1
        rc, stats = oracle_prefetch(c["pages"], c["config"])
        assert rc == 0 and stats == c["stats"], c["config"]


@pytest.mark.skipif(not oracle_py.ref_available(), reason="reference shim not built here")
def test_prefetch_simulation_live_against_reference():
    import sys
    import pathlib
    sys.path.insert(0, str(pathlib.Path(__file__).parent / "golden"))
    import make_golden
    ref = make_golden.bind(oracle_py.ref_lib())
    rng = np.random.default_rng(77)
    for _ in range(200):
        n = int(rng.integers(1, 3000))
        pages = make_golden.prefetch_stream(rng, n)
        cfg = [int(rng.integers(0, 2)), int(rng.integers(0, 4)), int(rng.integers(0, 100)),
               int(rng.integers(0, 64)), int(rng.integers(0, 50_000)), int(rng.integers(0, 5000))]
        stats = np.zeros(7, np.uint64)
        assert ref.ref_simulate_prefetch(pages.ctypes.data, n, cfg[0], 1.0, cfg[1], cfg[2],
                                         cfg[3], cfg[4], cfg[5], 1, stats.ctypes.data) == 1
        rc, mine = oracle_prefetch(pages, cfg)
        assert rc == 0 and mine == stats.tolist(), cfg
