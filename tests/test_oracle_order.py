"""Streams whose issue time goes back: the oracle serves every resource in
(issue time, stream position) order, the order in which the reference's
MQSim adapter serves staged arrivals (mqsim_online.cpp:269-289).  Pinned
without the oracle's own sort:

* running an unsorted stream equals running the same records permuted by
  numpy's stable argsort, results written back to stream positions
  (completions, status bytes, report, engine state and busy totals);
* on one plane and one channel, completions follow the Lindley / (max,+)
  recurrence evaluated over Python's `sorted` order of (issue, position);
* equal issue times keep stream order: which of two same-page reads hits the
  page register is decided by their positions;
* an issue-ordered stream is untouched by the order rule;
* the thermal-coupled run refuses demand records out of issue order."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
from hbfsim_amd import workloads as w

C0 = w.PROFILES / "c0.json"


def setup(profile=C0, ranges=None, **options):
    prof = oracle_py.load_profile(profile)
    params = oracle_py.engine_params(prof, **options)
    ranges = ranges or [(w.RANGE_BASE, 1 << 30, 3)]
    orng, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    return prof, params, orng, count


def shuffled_stream(n, seed, writes=100):
    s = w.config0(n=n, seed=seed, write_fraction_per_mille=writes)
    rec = s.records.copy()
    rng = np.random.default_rng(seed)
    # local disorder: pairs swapped, blocks moved back in time, exact ties
    idx = rng.integers(0, n - 1, n // 20)
    rec[idx, 2], rec[idx + 1, 2] = rec[idx + 1, 2].copy(), rec[idx, 2].copy()
    late = rng.integers(0, n, n // 50)
    rec[late, 2] //= np.uint64(2)
    tie = rng.integers(1, n, n // 50)
    rec[tie, 2] = rec[tie - 1, 2]
    rec[::97, 0] -= np.uint64(1 << 21)  # some bypass records
    return rec


@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("options", [dict(), dict(page_buffers=2), dict(plane_contention=0),
                                     dict(hybrid=True)])
def test_unsorted_equals_stable_argsort(threads, options):
    prof, params, orng, count = setup(**options)
    rec = shuffled_stream(30_000, 3)
    assert np.any(rec[1:, 2] < rec[:-1, 2])
    st_a = oracle_py.OracleState(params)
    comp, status, rep, _ = oracle_py.run(params, orng, count, rec, 777, st_a, threads=threads)
    order = np.argsort(rec[:, 2], kind="stable")
    st_b = oracle_py.OracleState(params)
    scomp, sstatus, srep, _ = oracle_py.run(params, orng, count, rec[order], 777, st_b,
                                            threads=threads)
    want_c = np.empty_like(scomp)
    want_c[order] = scomp
    want_s = np.empty_like(sstatus)
    want_s[order] = sstatus
    np.testing.assert_array_equal(comp, want_c)
    np.testing.assert_array_equal(status, want_s)
    assert rep == srep
    for k in ("plane_busy", "plane_tag", "channel_cursor", "plane_busy_total",
              "channel_busy_total"):
        np.testing.assert_array_equal(getattr(st_a, k), getattr(st_b, k), k)
    assert st_a.s.modeled_sequence == st_b.s.modeled_sequence


def test_single_resource_lindley_over_sorted_order():
    """One channel, one plane, no page register: completion =
    max(plane, channel) with plane' = max(plane, issue) + tR and channel' =
    max(channel, issue) + xfer, taken over (issue, position) order."""
    prof, params, orng, count = setup(flat_geometry=1, page_buffers=0)
    rng = np.random.default_rng(9)
    n = 400
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = np.uint64(w.RANGE_BASE) + rng.integers(0, 1 << 20, n).astype(np.uint64) * 128
    rec[:, 1] = 128
    rec[:, 2] = rng.integers(0, 50, n).astype(np.uint64) * 1000  # many ties, no order
    comp, _, _, _ = oracle_py.run(params, orng, count, rec)
    t_r = prof["read_latency_ns"] * 1000
    # transfer of 128 B at the aggregate bandwidth (one channel), ps, rounded up
    bw = prof["aggregate_bandwidth_bytes_per_s"]
    xfer = -(-128 * 10**12 // bw)
    plane = chan = 0
    want = [0] * n
    for i in sorted(range(n), key=lambda k: (int(rec[k, 2]), k)):
        issue = int(rec[i, 2])
        plane = max(plane, issue) + t_r
        chan = max(chan, issue) + xfer
        want[i] = max(plane, chan)
    np.testing.assert_array_equal(comp, np.array(want, np.uint64))


def test_ties_keep_stream_order():
    """Records A (t=10 ns), X (t=5 ns), B (t=10 ns) with A and B on one page:
    sorted (X, A, B), so B hits the page A opened, not the other way round."""
    prof, params, orng, count = setup()
    page = prof["page_bytes"]
    base = w.RANGE_BASE
    stride = params.channels * params.dies * params.planes * page  # same plane, other page
    rec = np.array([[base, 128, 10_000, 0],
                    [base + stride, 128, 5_000, 0],
                    [base + 256, 128, 10_000, 0]], np.uint64)
    _, status, rep, _ = oracle_py.run(params, orng, count, rec)
    assert rep["page_hits"] == 1
    assert status[2] & 4 and not status[0] & 4 and not status[1] & 4


def test_ordered_stream_unchanged():
    """Already issue-ordered (ties included): the same as the records taken
    one at a time in stream order, i.e. as several one-record runs."""
    prof, params, orng, count = setup()
    s = w.config0(n=3000, seed=4, write_fraction_per_mille=80)
    rec = s.records.copy()
    rec[1::3, 2] = rec[0::3, 2][: len(rec[1::3])]  # ties with the predecessor
    assert np.all(rec[1:, 2] >= rec[:-1, 2])
    comp, status, rep, _ = oracle_py.run(params, orng, count, rec)
    st = oracle_py.OracleState(params)
    one = [oracle_py.run(params, orng, count, rec[i:i + 1], 0, st) for i in range(len(rec))]
    np.testing.assert_array_equal(comp, np.concatenate([o[0] for o in one]))
    np.testing.assert_array_equal(status, np.concatenate([o[1] for o in one]))


def test_coupled_run_refuses_unsorted_demand():
    prof, params, orng, count = setup()
    rel = oracle_py.reliability(dict(w.C4_GRID, nx=8, ny=8, nz=8), dict(
        w.C4_RELIABILITY, regions_x=4, regions_y=2), params.dies)
    rec = w.config0(n=500, seed=2).records.copy()
    rec[[10, 400], 2] = rec[[400, 10], 2]
    assert np.any(rec[1:, 2] < rec[:-1, 2])
    temp = np.full(8 * 8 * 8, 318.15)
    age = np.zeros(params.channels * params.dies, np.uint64)
    t0, a0 = temp.copy(), age.copy()
    with pytest.raises(RuntimeError, match="failed: 1"):
        oracle_py.coupled_run(params, orng, count, rel, rec, temp, age)
    np.testing.assert_array_equal(temp, t0)
    np.testing.assert_array_equal(age, a0)
