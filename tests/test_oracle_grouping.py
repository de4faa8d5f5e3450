"""Warp grouping in the oracle (hbf_device.cu:1223-1231: lanes of one warp
instruction that passed validation and touch the same (range, page) share
the lowest lane's media request).

Pinned without the oracle's own grouping code: a grouped run must equal the
ungrouped run of the same stream with the joining records taken out (found
here from the ranges and the ungrouped run's classes), each joining record
taking its request's completion; on per-lane streams through the fast preset
the requests must follow the reference's own single-tail recurrence
(hbf_device.cu:895-910) written out directly."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
from hbfsim_amd import workloads

C0 = workloads.PROFILES / "c0.json"
PAGE = 16384
BASE = 0x5200_0000_0000


def grouping_ranges():
    # read-write, read-only, read-write; page-aligned bases with gaps
    return [(BASE, 64 * PAGE, 3), (BASE + 80 * PAGE, 32 * PAGE, 1),
            (BASE + 128 * PAGE, 48 * PAGE, 3)]


def warp_stream(seed: int, instrs: int, ranges, lanes: int = 32, t0: int = 0) -> np.ndarray:
    """Warp instructions of `lanes` records each (group id = instruction
    index + 1, one issue time): lanes read or write 32-256-byte pieces of one
    to three pages of a range, with some lanes bypassing, some crossing a
    page (unsupported) and some writing a read-only range; loose records
    with no group id in between."""
    rng = np.random.default_rng(seed)
    out = []
    t = t0
    gid = 1
    for _ in range(instrs):
        t += int(rng.integers(0, 4000))
        if rng.integers(0, 5) == 0:  # a loose record
            base, length, _ = ranges[int(rng.integers(0, len(ranges)))]
            out.append((base + int(rng.integers(0, length // 64)) * 64, 64, t, 0))
            continue
        base, length, _ = ranges[int(rng.integers(0, len(ranges)))]
        npages = int(rng.integers(1, 4))
        p0 = int(rng.integers(0, length // PAGE - npages + 1))
        size = int(rng.choice([32, 64, 128, 256]))
        op = int(rng.integers(0, 8) == 0)
        n = int(rng.integers(1, lanes + 1))
        for _ in range(n):
            k = int(rng.integers(0, 100))
            pg = p0 + int(rng.integers(0, npages))
            a = base + pg * PAGE + int(rng.integers(0, PAGE // size)) * size
            o = op
            if k < 4:
                a = 0x1000 + int(rng.integers(0, 1 << 16)) * 64   # bypass
            elif k < 7:
                a = base + pg * PAGE + PAGE - size // 2             # crosses a page
            elif k < 10:
                o = 1                                                # write
            out.append((a, size, t, o | (gid << 32)))
        gid += 1
    return np.array(out, dtype=np.uint64)


def keys(records: np.ndarray, ranges):
    """(range index, page within the range) of each record, -1 outside."""
    out = []
    for a, b, _, _ in records:
        a = int(a)
        k = (-1, -1)
        for r, (base, length, _) in enumerate(ranges):
            if base <= a < base + length:
                k = (r, (a - base) // PAGE)
        out.append(k)
    return out


def joiners(records: np.ndarray, modeled: np.ndarray, ranges) -> dict:
    """Joining record -> the record whose request it joins."""
    k = keys(records, ranges)
    group = (records[:, 3] >> np.uint64(32)).astype(np.int64)
    join = {}
    first = {}
    for i in range(len(records)):
        g = int(group[i])
        if g == 0 or i == 0 or group[i - 1] != g:
            first = {}
        if g == 0 or not modeled[i]:
            continue
        if k[i] in first:
            join[i] = first[k[i]]
        else:
            first[k[i]] = i
    return join


def run(records, grouping, ranges=None, **opts):
    ranges = ranges or grouping_ranges()
    prof = oracle_py.load_profile(C0)
    params = oracle_py.engine_params(prof, warp_grouping=grouping, **opts)
    table, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    return oracle_py.run(params, table, count, records)


@pytest.mark.parametrize("seed,opts", [(1, {}), (2, {"page_buffers": 0}),
                                       (3, {"plane_contention": 0}), (4, {"hybrid": True}),
                                       (5, {"transfer_page": 1})])
def test_grouped_equals_stream_without_joiners(seed, opts):
    ranges = grouping_ranges()
    rec = warp_stream(seed, 300, ranges)
    _, st0, _, _ = run(rec, 0, **opts)
    join = joiners(rec, (st0 & 3) == 0, ranges)
    assert len(join) > len(rec) // 4
    keep = np.array([i for i in range(len(rec)) if i not in join])
    c1, s1, r1, state1 = run(rec[keep], 0, **opts)
    c, s, r, state = run(rec, 1, **opts)
    np.testing.assert_array_equal(c[keep], c1)
    np.testing.assert_array_equal(s[keep], s1)
    jidx = np.array(sorted(join))
    lead = np.array([join[i] for i in jidx])
    np.testing.assert_array_equal(c[jidx], c[lead])
    assert (s[jidx] == 32).all()
    ops = rec[jidx, 3] & np.uint64(0xff)
    lat = (c[jidx] - rec[jidx, 2]).astype(object)
    assert r["grouped"] == len(jidx) and r1["grouped"] == 0
    assert r["records"] == r1["records"] + len(jidx)
    assert r["modeled"] == r1["modeled"] + len(jidx)
    assert r["reads"] == r1["reads"] + int((ops == 0).sum())
    assert r["writes"] == r1["writes"] + int((ops == 1).sum())
    for f in ("bypass", "unsupported", "page_hits", "programs", "hybrid_sampled",
              "service_sum_ps", "makespan_ps", "latency_max_ps"):
        assert r[f] == r1[f], f
    assert r["latency_sum_ps"] == r1["latency_sum_ps"] + int(sum(lat))
    assert state.s.modeled_sequence == state1.s.modeled_sequence
    np.testing.assert_array_equal(state.plane_busy, state1.plane_busy)
    np.testing.assert_array_equal(state.channel_cursor, state1.channel_cursor)
    np.testing.assert_array_equal(state.plane_tag, state1.plane_tag)


def test_group_ids_ignored_when_grouping_is_off():
    rec = warp_stream(7, 200, grouping_ranges())
    bare = rec.copy()
    bare[:, 3] &= np.uint64(0xff)
    a = run(rec, 0)
    b = run(bare, 0)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    assert a[2] == b[2]


def test_group_boundaries():
    """Adjacent instructions with different ids never share; the same id
    after a loose record starts a new group; a 64-record group is accepted,
    65 are refused, as is a group with two issue times."""
    base = BASE
    r = lambda a, t, g: (base + a, 64, t, g << 32)  # noqa: E731
    rec = np.array([r(0, 0, 1), r(64, 0, 1), r(128, 0, 2), r(192, 0, 2),
                    (base + 256, 64, 0, 0), r(320, 0, 2)], np.uint64)
    c, s, rep, _ = run(rec, 1)
    assert list(s & 32) == [0, 32, 0, 32, 0, 0] and rep["grouped"] == 2
    full = np.array([r(64 * k, 5, 9) for k in range(64)], np.uint64)
    c, s, rep, _ = run(full, 1)
    assert rep["grouped"] == 63 and (c == c[0]).all()
    over = np.array([r(64 * k, 5, 9) for k in range(65)], np.uint64)
    with pytest.raises(RuntimeError, match="6"):
        run(over, 1)
    run(over, 0)  # no groups without grouping
    mixed = full.copy()
    mixed[40, 2] += 1
    mixed[41:, 2] += 1
    with pytest.raises(RuntimeError, match="6"):
        run(mixed, 1)


def test_fast_preset_per_lane_streams_follow_reference_recurrence():
    """Per-lane streams (one record per active lane) through the fast
    preset: the requests, one per (instruction, page), follow the reference's
    single-tail recurrence, and every lane completes with its request."""
    from hbfsim_amd.engine import FAST_REFERENCE_OPTIONS
    nominal = oracle_py.ROOT / "tests" / "golden" / "profiles" / "nominal.json"
    prof = oracle_py.load_profile(nominal)
    ranges = [(workloads.RANGE_BASE, 1 << 26, 3)]
    rng = np.random.default_rng(9)
    out, t = [], 0
    for g in range(1, 400):
        t += int(rng.integers(0, 40)) * 1000
        page = int(rng.integers(0, (1 << 26) // 16384 - 2))
        op = int(rng.integers(0, 6) == 0)
        for lane in range(int(rng.integers(1, 33))):
            pg = page + int(rng.integers(0, 2))
            a = workloads.RANGE_BASE + pg * 16384 + int(rng.integers(0, 128)) * 128
            out.append((a, 128, t, op | (g << 32)))
    rec = np.array(out, np.uint64)
    params = oracle_py.engine_params(prof, warp_grouping=1, **FAST_REFERENCE_OPTIONS)
    table, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    comp, st, rep, _ = oracle_py.run(params, table, count, rec)
    xfer = -(-16384 * 10**9 // prof["aggregate_bandwidth_bytes_per_s"])
    tail = 0
    req = {}
    requests = 0
    for i, (a, _, issue, flags) in enumerate(rec):
        key = (int(flags) >> 32, (int(a) - workloads.RANGE_BASE) // 16384)
        if key in req:  # a lane of an earlier lane's request
            assert comp[i] == comp[req[key]] and st[i] == 32
            continue
        req[key] = i
        requests += 1
        arrival = int(issue) // 1000
        base = prof["program_latency_ns"] if int(flags) & 0xff else prof["read_latency_ns"]
        tail = max(tail, arrival) + xfer  # hbf_device.cu:895-910
        assert int(comp[i]) == max(arrival + base, tail) * 1000
    assert rep["modeled"] == len(rec) and rep["grouped"] == len(rec) - requests
