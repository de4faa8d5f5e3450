"""A seeded sweep over four profile geometries (configs 0, 2, 3 and 4: 64
to 1,024 planes), five option sets (among them no page register) and tile
sizes from one step to 257 steps: each case a mixed stream of linear,
contiguous, split and random parts through the packed records, every fourth
followed by a 32-byte run from the state the first left.  Small tiles give
runs of thousands of tiles (the four-wave summary form), the others the
few-tiles and LDS-bound forms; every case must equal the oracle bit for bit
and leave the same engine state."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_split import split_stream
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

PROFILES = {name: workloads.PROFILES / f"{name}.json" for name in ("c0", "c2", "c3", "c4")}
OPTIONS = [dict(), dict(plane_contention=0), dict(transfer_page=1), dict(program_every_write=1),
           dict(page_buffers=0)]
CASES = 50  # per profile


def mixed_stream(rng, ranges):
    parts = []
    for _ in range(int(rng.integers(2, 7))):
        kind = rng.integers(0, 4)
        seed = int(rng.integers(0, 1 << 30))
        if kind == 0:
            parts.append(linear_stream(seed, int(rng.integers(1, 600)), ranges))
        elif kind == 1:
            parts.append(contiguous_stream(seed, int(rng.integers(1, 80)), ranges))
        elif kind == 2:
            parts.append(split_stream(seed, int(rng.integers(1, 400)), ranges))
        else:
            s = workloads.config0(n=int(rng.integers(1, 120_000)), seed=seed % 1000,
                                  write_fraction_per_mille=int(rng.integers(0, 300)))
            rec = s.records.copy()
            # re-aim the random lines at one of the ranges (line-aligned offsets)
            r = ranges[int(rng.integers(0, len(ranges)))]
            off = (rec[:, 0] - np.uint64(workloads.RANGE_BASE)) % np.uint64(r[1])
            rec[:, 0] = np.uint64(r[0]) + off
            parts.append(rec)
    return chain_clocks(*parts)


@pytest.mark.parametrize("name", list(PROFILES))
def test_profile_sweep(name):
    ranges = ranges_for()
    for case in range(CASES):
        rng = np.random.default_rng([list(PROFILES).index(name), case])
        rec = mixed_stream(rng, ranges)
        opts = dict(OPTIONS[int(rng.integers(0, len(OPTIONS)))])
        tile = int(rng.choice([64, 64 * 3, 64 * 8, 64 * 64, 64 * 257, 0]))
        if tile:
            opts["tile_records"] = tile
        what = f"{name} case {case} {opts} n={len(rec)}"
        p = parity.Pair(PROFILES[name], ranges, **opts)
        try:
            base = int(rng.integers(0, 1 << 40))
            g, c = p.run_packed(rec, base)
            parity.assert_same(g, c, what)
            if case % 4 == 0:
                g2, c2 = p.run(rec, int(g[2]["makespan_ps"]))
                parity.assert_same(g2, c2, what + " (32-byte second run)")
            p.check_state()
        finally:
            p.close()
