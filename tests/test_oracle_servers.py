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
