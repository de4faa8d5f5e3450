"""Two page registers per plane (device_coalescer.cpp:134-168: a miss fills
the first empty slot, else slot 0) on the GPU against the CPU oracle,
bit-exact: from empty registers (every plane passes through its fill
events), from every partially filled state, across split runs, with the
resolver's edge cases and on the config-2 expert stream."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from hbfsim_amd import workloads
from test_gpu_parity import C0, C2, check, mixed_stream, std_ranges

pytestmark = pytest.mark.gpu

K2 = dict(page_buffers=2)


def test_k2_config0_from_empty():
    s = workloads.config0(n=300_000, seed=2)
    p = parity.Pair(C0, s.ranges, **K2)
    try:
        (_, _, grep), _ = check(p, s.records, "config0 K=2")
        p.check_state()
        assert grep["modeled"] == len(s.records)
    finally:
        p.close()


@pytest.mark.parametrize("options", [
    dict(plane_contention=1),
    dict(plane_contention=0),
    dict(program_every_write=1, transfer_page=1),
])
def test_k2_mixed_edge_cases(options):
    ranges = std_ranges()
    rec = mixed_stream(21, 30_000, ranges, 16384)
    p = parity.Pair(C0, ranges, **K2, **options)
    try:
        (_, _, grep), _ = check(p, rec, f"mixed K=2 {options}")
        assert grep["page_hits"] > 0 and grep["bypass"] > 0 and grep["unsupported"] > 0
        p.check_state()
    finally:
        p.close()


def alternating(n, seed, base, pages_per_plane=3, planes=64):
    """Each record reads one of a few pages of a plane: with two registers
    the second page stays buffered, so hits need both slots right."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, planes, n).astype(np.uint64)
    k = rng.choice(pages_per_plane, n, p=[0.5, 0.35, 0.15][:pages_per_plane]).astype(np.uint64)
    page = q + np.uint64(planes) * k * np.uint64(7)
    rec = np.zeros((n, 4), np.uint64)
    rec[:, 0] = np.uint64(base) + page * np.uint64(16384) + rng.integers(0, 128, n).astype(
        np.uint64) * np.uint64(128)
    rec[:, 1] = 128
    rec[:, 2] = np.cumsum(rng.integers(0, 4000, n).astype(np.uint64), dtype=np.uint64)
    return rec


def test_k2_alternating_pages_hit_more_than_one_register():
    base = workloads.RANGE_BASE
    ranges = [(base, 1 << 30, 1)]
    rec = alternating(100_000, 7, base)
    p2 = parity.Pair(C0, ranges, **K2)
    p1 = parity.Pair(C0, ranges)
    try:
        (_, _, r2), _ = check(p2, rec, "alternating K=2")
        (_, _, r1), _ = check(p1, rec, "alternating K=1")
        p2.check_state()
        assert r2["page_hits"] > r1["page_hits"]
    finally:
        p2.close()
        p1.close()


def test_k2_split_runs_resume_exactly():
    ranges = std_ranges()
    rec = mixed_stream(5, 40_000, ranges, 16384)
    whole = parity.Pair(C0, ranges, **K2)
    split = parity.Pair(C0, ranges, **K2)
    try:
        (gw, _, _), _ = check(whole, rec, "whole")
        parts = []
        for lo, hi in [(0, 3), (3, 64), (64, 5000), (5000, 5001), (5001, 40_000)]:
            (g, _, _), _ = check(split, rec[lo:hi], f"part {lo}:{hi}")
            parts.append(g)
            split.check_state()
        np.testing.assert_array_equal(np.concatenate(parts), gw)
    finally:
        whole.close()
        split.close()


def test_k2_from_every_partial_state():
    """Planes start in each register state: both empty, slot 0 only, slot 1
    only, both held (set through the checkpoint interface on both sides)."""
    base = workloads.RANGE_BASE
    ranges = [(base, 1 << 30, 1)]
    rec = alternating(60_000, 11, base)
    p = parity.Pair(C0, ranges, **K2)
    try:
        st = p.engine.state()
        tags = st["plane_tags"].reshape(-1, 2)
        rng = np.random.default_rng(3)
        for r in range(tags.shape[0]):
            kind = r % 4
            a = int(rng.integers(0, 64 * 21)) + 1  # page + 1
            b = int(rng.integers(0, 64 * 21)) + 1
            if b == a:
                b += 1
            tags[r] = {0: (0, 0), 1: (a, 0), 2: (0, b), 3: (a, b)}[kind]
        st["plane_tags"] = tags.reshape(-1)
        p.engine.set_state(st)
        p.ostate.plane_tag[:] = st["plane_tags"]
        check(p, rec, "partial states")
        p.check_state()
    finally:
        p.close()


def test_k2_config2_expert_stream_prefix():
    shape = workloads.QWEN3_30B_A3B
    sel = workloads.moe_selection(shape, 1)[0]
    seg = workloads.moe_segments(shape, sel)
    rec = workloads.segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                    shape.issuers, 0, 1 << 20)
    p = parity.Pair(C2, workloads.moe_ranges(shape), **K2)
    try:
        (_, _, grep), _ = check(p, rec, "config2 K=2")
        assert grep["page_hits"] == len(rec) - len(rec) * 128 // 16384
        p.check_state()
    finally:
        p.close()
