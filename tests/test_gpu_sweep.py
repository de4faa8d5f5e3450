"""A seeded sweep of mixed streams through both record forms: linear
batches, contiguous groups and random records (config-0 style) interleaved
in random proportions, under random tile sizes and engine options, on both
profiles.  Every case must equal the oracle bit for bit (completions,
statuses, report) and leave the same engine state, and the packed run of a
case must equal its 32-byte run."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0, C2
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

OPTIONS = [dict(), dict(plane_contention=0), dict(transfer_page=1), dict(program_every_write=1)]


def mixed_stream(seed):
    rng = np.random.default_rng(seed)
    ranges = ranges_for(count=int(rng.integers(2, 9)), pages=int(rng.integers(40, 200)))
    parts = []
    for _ in range(int(rng.integers(2, 6))):
        kind = rng.integers(0, 3)
        if kind == 0:
            parts.append(linear_stream(int(rng.integers(0, 1 << 30)), int(rng.integers(1, 400)),
                                       ranges))
        elif kind == 1:
            parts.append(contiguous_stream(int(rng.integers(0, 1 << 30)),
                                           int(rng.integers(1, 60)), ranges))
        else:
            s = workloads.config0(n=int(rng.integers(1, 20_000)), seed=int(rng.integers(0, 1000)),
                                  write_fraction_per_mille=int(rng.integers(0, 300)))
            rec = s.records.copy()
            # re-aim the random lines at one of this case's ranges, keeping
            # their offsets modulo its length (line-aligned)
            r = ranges[int(rng.integers(0, len(ranges)))]
            off = (rec[:, 0] - np.uint64(workloads.RANGE_BASE)) % np.uint64(r[1])
            rec[:, 0] = np.uint64(r[0]) + off
            parts.append(rec)
    # each part continues the clock of the one before: the stream is in issue
    # order (streams that leave it are tested in test_gpu_order.py)
    return ranges, chain_clocks(*parts)


@pytest.mark.parametrize("seed", range(32))
def test_mixed_streams_both_forms(seed):
    rng = np.random.default_rng(1000 + seed)
    ranges, rec = mixed_stream(seed)
    profile = C0 if seed % 2 else C2
    opts = dict(OPTIONS[seed % len(OPTIONS)])
    tile = int(rng.choice([64 * 8, 64 * 64, 64 * 257, 0]))
    if tile:
        opts["tile_records"] = tile
    cut = int(rng.integers(0, len(rec) + 1))
    a = parity.Pair(profile, ranges, **opts)
    b = parity.Pair(profile, ranges, **opts)
    try:
        for lo, hi in [(0, cut), (cut, len(rec))]:
            ga, ca = a.run(rec[lo:hi], 1000 * seed)
            parity.assert_same(ga, ca, f"seed {seed} 32-byte part {lo}:{hi}")
            gb, cb = b.run_packed(rec[lo:hi], 1000 * seed)
            parity.assert_same(gb, cb, f"seed {seed} packed part {lo}:{hi}")
            np.testing.assert_array_equal(ga[0], gb[0])
            np.testing.assert_array_equal(ga[1], gb[1])
        a.check_state()
        b.check_state()
    finally:
        a.close()
        b.close()
