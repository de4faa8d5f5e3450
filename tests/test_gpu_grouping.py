"""Warp grouping on the GPU (k_lead, the summary and apply passes with
joining records left out, k_follow) against the oracle, bit for bit:
completions, statuses, reports and carried state, across tile and
k_lead-window boundaries, page-register and contention options, hybrid
sampling, the fast preset on per-lane streams, and refusals that leave the
state untouched."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from hbfsim_amd import _native as nat
from hbfsim_amd.engine import FAST_REFERENCE_OPTIONS
from test_oracle_grouping import C0, grouping_ranges, warp_stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,opts", [
    (1, {}), (2, {"page_buffers": 0}), (3, {"plane_contention": 0}),
    (4, {"transfer_page": 1}), (5, {"tile_records": 128}), (6, {"tile_records": 192}),
    (7, {"mode": "hybrid"})])
def test_grouped_parity(seed, opts):
    opts = dict(opts)
    mode = opts.pop("mode", "fast")
    ranges = grouping_ranges()
    pair = parity.Pair(C0, ranges, mode=mode, warp_grouping=1, **opts)
    try:
        t0 = 0
        for k in range(2):  # state carries from the first run to the second
            rec = warp_stream(seed * 10 + k, 400, ranges, t0=t0)
            t0 = int(rec[-1, 2]) + 1
            gpu, cpu = pair.run(rec)
            parity.assert_same(gpu, cpu, f"seed {seed} run {k}")
            assert gpu[2]["grouped"] > 0
        pair.check_state()
    finally:
        pair.close()


def test_grouped_parity_large():
    """~330K records: thousands of k_lead windows and tiles."""
    ranges = grouping_ranges()
    pair = parity.Pair(C0, ranges, warp_grouping=1)
    try:
        rec = warp_stream(77, 20_000, ranges, lanes=64)
        gpu, cpu = pair.run(rec)
        parity.assert_same(gpu, cpu, "large")
        assert gpu[2]["grouped"] > len(rec) // 3
        pair.check_state()
    finally:
        pair.close()


def test_fast_preset_per_lane():
    ranges = [(0x5400_0000_0000, 1 << 26, 3)]
    rng = np.random.default_rng(3)
    out, t = [], 0
    for g in range(1, 3000):
        t += int(rng.integers(0, 40)) * 1000
        page = int(rng.integers(0, (1 << 26) // 16384 - 2))
        for _ in range(int(rng.integers(1, 33))):
            a = ranges[0][0] + (page + int(rng.integers(0, 2))) * 16384 + \
                int(rng.integers(0, 128)) * 128
            out.append((a, 128, t, int(rng.integers(0, 6) == 0) | (g << 32)))
    rec = np.array(out, np.uint64)
    pair = parity.Pair(C0, ranges, warp_grouping=1, **FAST_REFERENCE_OPTIONS)
    try:
        gpu, cpu = pair.run(rec)
        parity.assert_same(gpu, cpu, "fast preset, per lane")
        assert gpu[2]["grouped"] > 0
    finally:
        pair.close()


def test_refused_groups_leave_state():
    import torch
    ranges = grouping_ranges()
    pair = parity.Pair(C0, ranges, warp_grouping=1)
    try:
        first = warp_stream(21, 200, ranges)
        gpu, cpu = pair.run(first)
        parity.assert_same(gpu, cpu, "before")
        t = int(first[-1, 2]) + 10
        over = np.array([(ranges[0][0] + 64 * k, 64, t, 5 << 32) for k in range(65)], np.uint64)
        mixed = over[:40].copy()
        mixed[20:, 2] += 1
        for bad in (over, mixed):
            with pytest.raises(nat.HbfSimError) as e:
                pair.engine.run(parity.to_device(bad),
                                torch.zeros(len(bad), dtype=torch.int64, device="cuda"))
            assert e.value.code == nat.HBFSIM_INVALID_ARGUMENT
        after = warp_stream(22, 200, ranges, t0=t)
        gpu, cpu = pair.run(after)
        parity.assert_same(gpu, cpu, "after the refusals")
        pair.check_state()
    finally:
        pair.close()


def test_unsupported_combinations_and_packed():
    import torch
    ranges = grouping_ranges()
    rec = warp_stream(31, 50, ranges)
    pair = parity.Pair(C0, ranges, warp_grouping=1, page_buffers=2)
    try:
        with pytest.raises(nat.HbfSimError) as e:
            pair.engine.run(parity.to_device(rec),
                            torch.zeros(len(rec), dtype=torch.int64, device="cuda"))
        assert e.value.code == nat.HBFSIM_UNSUPPORTED
    finally:
        pair.close()
    # packed records carry no group id: grouping changes nothing
    bare = rec.copy()
    bare[:, 3] &= np.uint64(0xff)
    pair = parity.Pair(C0, ranges, warp_grouping=1)
    try:
        gpu, cpu = pair.run_packed(bare)
        parity.assert_same(gpu, cpu, "packed")
        assert gpu[2]["grouped"] == 0
    finally:
        pair.close()
