"""The MQSim adapter's queue-depth admission and bandwidth cursor
(mqsim_online.cpp:266-376) over a fake media port, in the oracle.

Pinned three ways that do not share the oracle's event loop: the reference's
own queue-depth test (mqsim_queue_depth_test.cpp:73-124: a burst completes
every request, a shallow queue finishes later than a deep one, one slot
charges at least one read per request); the FIFO multi-server recursion
(admission = max(arrival, earliest completion among the queue_depth
requests in the device), a min-heap over requests in arrival order) with
the cursor taken in completion order; and closed forms (an unbounded queue
admits at arrival; one slot chains admission_k = max(arrival_k,
device_{k-1}))."""
from __future__ import annotations

import heapq

import numpy as np
import pytest

import oracle_py


def fifo_servers(arrival, nbytes, latency, depth, bandwidth):
    order = sorted(range(len(arrival)), key=lambda i: (int(arrival[i]), i))
    heap, adm, dev = [], {}, {}
    for i in order:
        t = int(arrival[i])
        if len(heap) == max(1, depth):
            t = max(t, heapq.heappop(heap))
        adm[i] = t
        dev[i] = t + int(latency[i])
        heapq.heappush(heap, dev[i])
    # completion callbacks in (media completion, admission order)
    rank = {i: r for r, i in enumerate(order)}
    cursor, done = 0, {}
    for i in sorted(dev, key=lambda i: (dev[i], adm[i], rank[i])):
        x = -(-int(nbytes[i]) * 10**9 // bandwidth)
        cursor = max(cursor, int(arrival[i])) + x
        done[i] = max(dev[i], cursor)
    n = len(arrival)
    return ([adm[i] for i in range(n)], [dev[i] for i in range(n)], [done[i] for i in range(n)])


def test_reference_queue_depth_properties():
    """A 32-request burst of 16 KiB reads at time 0 (the reference test's
    workload, with a fake port of the nominal read latency)."""
    read_ns, bw = 45_000, 32 * 10**9
    arrival = np.zeros(32, np.uint64)
    nbytes = np.full(32, 16384, np.uint64)
    _, _, shallow = oracle_py.mqsim_admission(arrival, nbytes, read_ns, 1, bw)
    _, _, deep = oracle_py.mqsim_admission(arrival, nbytes, read_ns, 32, bw)
    assert len(shallow) == len(deep) == 32
    assert shallow.max() > deep.max()
    assert shallow.max() >= 32 * read_ns


@pytest.mark.parametrize("seed", range(8))
def test_equals_fifo_multiserver_recursion(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 400))
    arrival = np.sort(rng.integers(0, 50 * n, n)).astype(np.uint64)
    if seed % 2:
        rng.shuffle(arrival)  # the adapter sorts staged requests itself
        arrival[rng.integers(0, n, n // 4)] = arrival[0]  # ties broken by index
    nbytes = (rng.integers(1, 64, n) * 512).astype(np.uint64)
    latency = rng.integers(1, 3000, n).astype(np.uint64)
    depth = int(rng.integers(0, 12))
    bw = int(rng.integers(10**9, 64 * 10**9))
    got = oracle_py.mqsim_admission(arrival, nbytes, latency, depth, bw)
    want = fifo_servers(arrival, nbytes, latency, depth, bw)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, np.array(w, np.uint64))


def test_closed_forms():
    rng = np.random.default_rng(3)
    n = 300
    arrival = np.sort(rng.integers(0, 20_000, n)).astype(np.uint64)
    nbytes = np.full(n, 4096, np.uint64)
    latency = rng.integers(1, 500, n).astype(np.uint64)
    adm, dev, _ = oracle_py.mqsim_admission(arrival, nbytes, latency, n, 10**10)
    np.testing.assert_array_equal(adm, arrival)
    np.testing.assert_array_equal(dev, arrival + latency)
    adm, dev, done = oracle_py.mqsim_admission(arrival, nbytes, latency, 1, 10**10)
    prev = 0
    for k in range(n):
        assert int(adm[k]) == max(int(arrival[k]), prev)
        prev = int(dev[k])
    # depth 0 behaves as 1 (std::max<size_t>(1, queue_depth))
    again = oracle_py.mqsim_admission(arrival, nbytes, latency, 0, 10**10)
    np.testing.assert_array_equal(again[2], done)
    with pytest.raises(ValueError):
        oracle_py.mqsim_admission(arrival, nbytes, latency, 1, 0)


# ---- the same loop with the engine as the media port (orc_engine_admission)

def _media_case(n, nbytes, gap, seed, flat=False):
    """The media bench's workload on the nominal profile: n requests of
    nbytes at random 16 KiB-aligned slots, arrivals i * gap ns, split at
    pages; returns (profile, params, table, count, records, first, arrival)."""
    from test_media_bench import NOMINAL, RANGE_BASE
    prof = oracle_py.load_profile(NOMINAL)
    opts = dict(flat_geometry=1, page_buffers=0, plane_contention=0,
                channel_bandwidth_bytes_per_s=1 << 60) if flat else {}
    params = oracle_py.engine_params(prof, **opts)
    cap = 1 << 30
    table, count = oracle_py.range_table([(RANGE_BASE, cap, 3)], prof["page_bytes"],
                                         prof["capacity_bytes"])
    rng = np.random.default_rng(seed)
    page = prof["page_bytes"]
    rec, first = [], [0]
    for i in range(n):
        addr = int(rng.integers(0, cap // nbytes)) * nbytes
        left = nbytes
        while left:
            piece = min(left, page - addr % page)
            rec.append((RANGE_BASE + addr, piece, 0, 0))
            addr += piece
            left -= piece
        first.append(len(rec))
    arrival = np.arange(n, dtype=np.uint64) * np.uint64(gap)
    return prof, params, table, count, np.array(rec, np.uint64), np.array(first, np.uint64), \
        arrival


def test_engine_port_unbounded_queue_is_one_engine_run():
    """Queue depth beyond the request count: every request dispatched at its
    arrival, so the device completions are one engine run of all pages
    issued at their arrivals."""
    prof, params, table, count, rec, first, arrival = _media_case(400, 32768, 30, 1)
    adm, dev, _ = oracle_py.engine_admission(params, table, count, rec, first, arrival,
                                             np.full(400, 32768, np.uint64), 1000,
                                             prof["aggregate_bandwidth_bytes_per_s"])
    np.testing.assert_array_equal(adm, arrival)
    issued = rec.copy()
    for k in range(400):
        issued[first[k]:first[k + 1], 2] = arrival[k] * np.uint64(1000)
    comp, _, _, _ = oracle_py.run(params, table, count, issued)
    want = [-(-int(comp[first[k]:first[k + 1]].max()) // 1000) for k in range(400)]
    np.testing.assert_array_equal(dev, np.array(want, np.uint64))


@pytest.mark.parametrize("depth", [1, 3, 32])
def test_engine_port_fixed_latency_is_the_fake_port_loop(depth):
    """A single plane without page register or contention, with a channel
    so fast that transfers never bind: every request's device time is its
    admission + tR, the fake media port of orc_mqsim_admission, whose loop the
    results must then equal exactly."""
    n = 300
    prof, params, table, count, rec, first, arrival = _media_case(n, 16384, 2000, 2, flat=True)
    nb = np.full(n, 16384, np.uint64)
    bw = prof["aggregate_bandwidth_bytes_per_s"]
    got = oracle_py.engine_admission(params, table, count, rec, first, arrival, nb, depth, bw)
    want = oracle_py.mqsim_admission(arrival, nb, prof["read_latency_ns"], depth, bw)
    for g, w_ in zip(got, want):
        np.testing.assert_array_equal(g, w_)


def test_engine_port_one_slot_chains_requests():
    """One slot: request k dispatches at max(arrival_k, device_{k-1}) and the
    engine times the requests one after another with its state carried."""
    n = 200
    prof, params, table, count, rec, first, arrival = _media_case(n, 16384, 500, 3)
    adm, dev, _ = oracle_py.engine_admission(params, table, count, rec, first, arrival,
                                             np.full(n, 16384, np.uint64), 1,
                                             prof["aggregate_bandwidth_bytes_per_s"])
    state = oracle_py.OracleState(params)
    prev = 0
    for k in range(n):
        t = max(int(arrival[k]), prev)
        assert int(adm[k]) == t
        pages = rec[first[k]:first[k + 1]].copy()
        pages[:, 2] = t * 1000
        comp, _, _, _ = oracle_py.run(params, table, count, pages, 0, state)
        prev = -(-int(comp.max()) // 1000)
        assert int(dev[k]) == prev
