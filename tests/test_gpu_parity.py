"""HIP engine vs CPU oracle, bit-exact (integer ps), through the C ABI.

Covers config 0 (2^20 records, the reference-shaped synthetic trace), the
resolver's edge cases (bypass, straddle, page crossing, permission, zero
bytes, bad operation), writes that fill pages, page registers on and off,
plane contention on and off, whole-page transfers, ragged tile tails,
thousands of ranges (two-level range search), non-power-of-two geometry,
every allocation order family, hybrid sampling, and split runs that resume
from carried state.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

C0 = workloads.PROFILES / "c0.json"
C2 = workloads.PROFILES / "c2.json"


def mixed_stream(seed: int, n: int, ranges, page: int, write_per_mille: int = 200):
    """Records hitting every classification path, ordered by issue time."""
    rng = np.random.default_rng(seed)
    kinds = rng.integers(0, 100, n)
    rec = np.zeros((n, 4), np.uint64)
    ri = rng.integers(0, len(ranges), n)
    for i in range(n):
        base, length, perms = ranges[ri[i]]
        k = kinds[i]
        op = 1 if rng.integers(0, 1000) < write_per_mille else 0
        b = int(rng.choice([64, 128, 256, 512]))
        if k < 70:      # inside, within one page
            off = int(rng.integers(0, length // b)) * b
            a = base + off
        elif k < 76:    # same page as a recent record (page-register hits)
            a = int(rec[max(0, i - int(rng.integers(1, 4))), 0]) or base
            a -= a % b
            if not (base <= a < base + length):
                a = base
        elif k < 80:    # write that fills its page
            op = 1
            off = int(rng.integers(0, length // page)) * page + page - b
            a = base + off
        elif k < 84:    # bypass: far below every range
            a = 0x1000 + int(rng.integers(0, 1 << 20)) * 64
        elif k < 87:    # straddles into the range from below
            a = base - b // 2
        elif k < 90:    # crosses a page boundary inside the range
            a = base + page - b // 2
        elif k < 92:    # crosses the range end
            a = base + length - b // 2
        elif k < 94:    # zero bytes
            a, b = base, 0
        elif k < 96:    # invalid operation
            a, op = base, 2
        else:           # write attempt (unsupported when the range is read-only)
            a, op = base + int(rng.integers(0, length // b)) * b, 1
        rec[i] = (a, b, 0, op)
    gaps = rng.integers(0, 6000, n).astype(np.uint64)
    gaps[rng.integers(0, 100, n) < 10] = 0  # simultaneous issues
    rec[:, 2] = np.cumsum(gaps, dtype=np.uint64)
    return rec


def std_ranges(count=4, length=1 << 24, gap=1 << 22, page=16384, base=0x7000_0000_0000):
    out = []
    a = base
    for i in range(count):
        out.append((a, length, 1 if i % 3 == 2 else 3))
        a += length + gap + page * (i % 2)
    return out


def check(pair, rec, what, base_ps=0):
    g, c = pair.run(rec, base_ps)
    parity.assert_same(g, c, what)
    return g, c


def test_config0_full_stream():
    s = workloads.config0()
    p = parity.Pair(C0, s.ranges)
    try:
        (gcomp, _, grep), _ = check(p, s.records, "config0")
        assert grep["modeled"] == len(s.records)
        assert grep["makespan_ps"] > 80_000_000_000  # plane-saturated, ~82 ms
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("tile", [64, 128, 1024, 4096])
def test_config0_tiles(tile):
    s = workloads.config0(n=50_000 + 37, seed=5, write_fraction_per_mille=100)
    p = parity.Pair(C0, s.ranges, tile_records=tile)
    try:
        check(p, s.records, f"tile {tile}")
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("options", [
    dict(page_buffers=1, plane_contention=1),
    dict(page_buffers=0, plane_contention=1),
    dict(page_buffers=1, plane_contention=0),
    dict(page_buffers=0, plane_contention=0, transfer_page=1),
    dict(page_buffers=1, program_every_write=1),
    dict(xfer_quantum_ps=1000),
    dict(channel_bandwidth_bytes_per_s=12_345_678_901),
])
def test_mixed_edge_cases(options):
    ranges = std_ranges()
    rec = mixed_stream(11, 20_000, ranges, 16384)
    p = parity.Pair(C0, ranges, **options)
    try:
        (_, gst, grep), _ = check(p, rec, f"mixed {options}")
        assert grep["bypass"] > 0 and grep["unsupported"] > 0 and grep["writes"] > 0
        if options.get("page_buffers", 1):
            assert grep["page_hits"] > 0
        p.check_state()
    finally:
        p.close()


def test_split_runs_resume_exactly():
    ranges = std_ranges()
    rec = mixed_stream(3, 30_000, ranges, 16384)
    whole = parity.Pair(C0, ranges)
    split = parity.Pair(C0, ranges)
    try:
        (gw, _, _), _ = check(whole, rec, "whole")
        parts = []
        for lo, hi in [(0, 7), (7, 4100), (4100, 4101), (4101, 30_000)]:
            (g, _, _), _ = check(split, rec[lo:hi], f"part {lo}:{hi}")
            parts.append(g)
        np.testing.assert_array_equal(np.concatenate(parts), gw)
        split.check_state()
    finally:
        whole.close()
        split.close()


def test_state_checkpoint_round_trip():
    ranges = std_ranges()
    rec = mixed_stream(4, 10_000, ranges, 16384)
    a = parity.Pair(C0, ranges)
    b = parity.Pair(C0, ranges)
    try:
        check(a, rec[:5000], "first half")
        b.engine.set_state(a.engine.state())
        ga, _ = a.run(rec[5000:])
        gb, _ = b.run(rec[5000:])
        np.testing.assert_array_equal(ga[0], gb[0])
    finally:
        a.close()
        b.close()


def test_base_offset_and_empty_runs():
    s = workloads.config0(n=5000, seed=9)
    p = parity.Pair(C0, s.ranges)
    try:
        g, c = p.run(s.records[:0])
        assert g[2]["records"] == 0
        check(p, s.records[:1], "one record", base_ps=123_456_789)
        check(p, s.records[1:], "rest", base_ps=10**15)
        p.check_state()
    finally:
        p.close()


def test_many_ranges_two_level_search():
    page = 16384
    ranges = [(0x6000_0000_0000 + i * (3 * page), page * 2 - 4096 * (i % 3), 3)
              for i in range(3000)]
    rng = np.random.default_rng(21)
    n = 40_000
    rec = np.zeros((n, 4), np.uint64)
    pick = rng.integers(0, len(ranges), n)
    for i in range(n):
        base, length, _ = ranges[pick[i]]
        k = rng.integers(0, 10)
        if k < 8:
            rec[i, 0] = base + int(rng.integers(0, length // 128)) * 128
        elif k < 9:
            rec[i, 0] = base + length + 64  # in the gap: bypass
        else:
            rec[i, 0] = base - 64           # straddles from the gap below
        rec[i, 1] = 128
    rec[:, 2] = np.cumsum(rng.integers(0, 3000, n).astype(np.uint64))
    p = parity.Pair(C0, ranges)
    try:
        (_, _, grep), _ = check(p, rec, "3000 ranges")
        assert grep["bypass"] > 0 and grep["unsupported"] > 0
        p.check_state()
    finally:
        p.close()


SCHEMES = ["".join(o) for o in __import__("itertools").permutations("CWDP")]


@pytest.mark.parametrize("geometry", ["pow2", "mixed"])
@pytest.mark.parametrize("scheme", SCHEMES)
def test_allocation_orders(tmp_path, scheme, geometry):
    """All 24 channel/way/die/plane orders, with two ways per channel so
    that every axis has extent: power-of-two axes (shift and mask striping)
    and mixed-radix ones (division striping)."""
    prof = json.loads(C0.read_text())
    prof["plane_allocation_scheme"] = scheme
    ways = 2
    if geometry == "mixed":
        prof.update(channels=6, dies_per_channel=3, planes_per_die=2,
                    capacity_bytes=6 * 3 * 2 * 3 * 16384 * prof["pages_per_block"] * 64)
        ways = 3
    path = tmp_path / f"c0-{scheme}-{geometry}.json"
    path.write_text(json.dumps(prof))
    s = workloads.config0(n=30_000, seed=2)
    p = parity.Pair(path, s.ranges, ways=ways)
    try:
        check(p, s.records, f"{scheme} {geometry}")
        p.check_state()
    finally:
        p.close()


def test_non_power_of_two_geometry(tmp_path):
    prof = json.loads(C0.read_text())
    prof.update(channels=6, dies_per_channel=3, planes_per_die=2,
                capacity_bytes=16384 * 6 * 3 * 2 * 256 * 60,
                aggregate_bandwidth_bytes_per_s=192_000_000_000)
    path = tmp_path / "c0-npot.json"
    path.write_text(json.dumps(prof))
    s = workloads.config0(n=30_000, seed=3)
    p = parity.Pair(path, s.ranges)
    try:
        check(p, s.records, "6x3x2")
        p.check_state()
    finally:
        p.close()


def test_config2_geometry_sequential_expert_reads():
    """512 planes x 16 channels: sequential lines of several experts."""
    expert = 9_437_184
    ranges = [(0x5000_0000_0000 + i * expert, expert, 1) for i in range(8)]
    lines = expert // 128
    n = 4 * 8192
    rec = np.zeros((n, 4), np.uint64)
    j = np.arange(n, dtype=np.uint64)
    e = (j // np.uint64(8192)) * np.uint64(2)          # experts 0, 2, 4, 6
    rec[:, 0] = np.uint64(0x5000_0000_0000) + e * np.uint64(expert) + \
        (j % np.uint64(lines)) * np.uint64(128)
    rec[:, 1] = 128
    rec[:, 2] = (j // np.uint64(256)) * np.uint64(1000)
    p = parity.Pair(C2, ranges)
    try:
        (_, _, grep), _ = check(p, rec, "config2 shape")
        assert grep["page_hits"] > 0
        p.check_state()
    finally:
        p.close()


def test_hybrid_sampling_counts(tmp_path):
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=0.05, reference_warmup_requests=100)
    path = tmp_path / "c0-hybrid.json"
    path.write_text(json.dumps(prof))
    ranges = std_ranges()
    rec = mixed_stream(8, 20_000, ranges, 16384)
    p = parity.Pair(path, ranges, mode="hybrid")
    try:
        (_, _, grep), _ = check(p, rec, "hybrid")
        assert grep["hybrid_sampled"] > 100
        (_, _, grep2), _ = check(p, rec, "hybrid second run")
        stats = p.engine.stats()
        sampled = grep["hybrid_sampled"] + grep2["hybrid_sampled"]
        modeled = grep["modeled"] + grep2["modeled"]
        # context.cpp:1983-2004: the request counters count ring requests
        # (the sampled ones), fast_requests the fast-model resolutions
        assert stats["reference_requests"] == sampled
        assert stats["requests_submitted"] == stats["requests_completed"] == sampled
        assert stats["fast_requests"] == modeled - sampled
    finally:
        p.close()


def test_fast_reference_preset_matches_single_tail_recurrence():
    """HBF model degenerated to one channel, unserialised latency, whole-page
    transfers in whole ns: the reference's fast model (hbf_device.cu:895-910)."""
    from hbfsim_amd.engine import FAST_REFERENCE_OPTIONS
    nominal = oracle_py.ROOT / "tests" / "golden" / "profiles" / "nominal.json"
    prof = oracle_py.load_profile(nominal)
    base = 0x4000_0000_0000
    ranges = [(base, 1 << 28, 3)]
    rng = np.random.default_rng(7)
    n = 20_000
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = base + rng.integers(0, (1 << 28) // 64, n).astype(np.uint64) * np.uint64(64)
    rec[:, 1] = 64
    rec[:, 3] = (rng.integers(0, 10, n) == 0).astype(np.uint64)
    rec[:, 2] = np.cumsum(rng.integers(0, 40, n).astype(np.uint64)) * np.uint64(1000)
    p = parity.Pair(nominal, ranges, **FAST_REFERENCE_OPTIONS)
    try:
        (gcomp, _, grep), _ = check(p, rec, "fast preset")
        arrival = (rec[:, 2] // np.uint64(1000)).astype(np.uint64)
        ops = rec[:, 3].astype(np.uint32)
        sizes = np.full(n, prof["page_bytes"], np.uint32)
        tail = np.zeros(1, np.uint64)
        target = np.zeros(n, np.uint64)
        L = oracle_py.lib()
        modeled = L.orc_fast_model_scalar(
            oracle_py.addr(arrival), oracle_py.addr(ops), oracle_py.addr(sizes), n,
            prof["read_latency_ns"], prof["program_latency_ns"],
            prof["aggregate_bandwidth_bytes_per_s"], oracle_py.addr(tail),
            oracle_py.addr(target))
        np.testing.assert_array_equal(gcomp, target * np.uint64(1000))
        assert grep["service_sum_ps"] == modeled * 1000
    finally:
        p.close()


@pytest.mark.parametrize("gap_ps", [1_000, 40_000_000])
def test_sequential_writes_and_wide_steps(gap_ps):
    """Single-key steps whose values need 64 bits: page-filling sequential
    writes (tPROG = 200 us) and issue gaps beyond 2^30 ps inside a step,
    next to steps that take the 32-bit path."""
    base = 0x6100_0000_0000
    page = 16384
    ranges = [(base, 64 * page, 3)]
    n = 20_000
    j = np.arange(n, dtype=np.uint64)
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = np.uint64(base) + (j * np.uint64(128)) % np.uint64(64 * page)
    rec[:, 1] = 128
    rec[:, 3] = ((j // np.uint64(2048)) % np.uint64(2)).astype(np.uint64)  # read/write phases
    rec[:, 2] = j * np.uint64(gap_ps)
    p = parity.Pair(C0, ranges)
    try:
        (_, _, grep), _ = check(p, rec, f"sequential rw gap {gap_ps}")
        assert grep["programs"] > 0 and grep["page_hits"] > 0
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("options", [
    dict(), dict(plane_contention=0), dict(page_buffers=0), dict(tile_records=192),
    dict(tile_records=64, transfer_page=1),
])
def test_sequential_runs(tmp_path, options):
    """Streams of whole-wave sequential runs (the fast path) interleaved with
    steps that break the run conditions: a page boundary inside a step, a
    write, an out-of-order issue, a bypass record; hybrid sampling on."""
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=0.02, reference_warmup_requests=7)
    path = tmp_path / "c0-runs.json"
    path.write_text(json.dumps(prof))
    base = 0x6200_0000_0000
    page = 16384
    ranges = [(base, 256 * page, 3)]
    n = 64 * 400 + 17
    j = np.arange(n, dtype=np.uint64)
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = np.uint64(base) + (j * np.uint64(128) + np.uint64(64 * 128 * 3)) % \
        np.uint64(256 * page)
    rec[:, 1] = 128
    rec[:, 2] = (j // np.uint64(16)) * np.uint64(3000)
    rng = np.random.default_rng(5)
    breaks = rng.integers(0, n, 40)
    rec[breaks[:10], 3] = 1                          # writes
    rec[breaks[10:20], 0] = 0x1000                   # bypass
    rec[breaks[20:30], 2] = rec[breaks[20:30], 2] // np.uint64(2)  # issue out of order
    p = parity.Pair(path, ranges, mode="hybrid", **options)
    try:
        (_, _, grep), _ = check(p, rec, f"runs {options}")
        assert grep["hybrid_sampled"] > 0
        assert grep["page_hits"] > 0 or options.get("page_buffers", 1) == 0
        p.check_state()
    finally:
        p.close()
