"""The packed summary pass comes in three forms chosen per run: the
LDS-bound one (two waves per SIMD, 16 steps in flight) where the per-plane
state allows no more waves, the form for runs whose tiles fit one round of
three-wave slots (at most 3,072 tiles: three waves, eight steps), and the
four-wave form (three steps) for the rest; general steps look their plane and
channel up in an LDS stripe table where it costs no occupancy.  The forms
differ in speed only: runs on either side of the 3,072-tile boundary, and on
both geometries, must equal the oracle bit for bit.  So must runs on either
side of the carry chain's 4,096-tile boundary (one launch up to it, three
above)."""
from __future__ import annotations

import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0, C2
from test_gpu_split import split_stream
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

TILE = 256  # records per tile
FEW = 3 * 4 * 256  # tiles in one round of three-wave slots


def mixed(n, seed, side):
    """n records: random general steps with linear, grouped and split steps
    in between, in issue order."""
    head = workloads.config0(n=n // 2, seed=seed, write_fraction_per_mille=40).records
    tail = workloads.config0(n=n, seed=seed + 1, write_fraction_per_mille=40).records
    rec = chain_clocks(head, linear_stream(seed + 2, 400, side),
                       contiguous_stream(seed + 3, 60, side), split_stream(seed + 4, 300, side),
                       tail)
    return rec[:n]


@pytest.mark.parametrize("tiles", [FEW, FEW + 1], ids=["few-tiles form", "four-wave form"])
def test_summary_forms_at_the_tile_boundary(tiles):
    side = ranges_for()
    ranges = [(workloads.RANGE_BASE, 1 << 30, 3)] + side
    rec = mixed(tiles * TILE, 40 + tiles % 2, side)
    assert len(rec) == tiles * TILE
    p = parity.Pair(C0, ranges, tile_records=TILE)
    try:
        base = 0
        for k in range(2):  # the second run starts from the first one's state
            g, c = p.run_packed(rec, base_ps=base)
            parity.assert_same(g, c, f"{tiles} tiles, run {k}")
            base = int(g[2]["makespan_ps"])
        p.check_state()
    finally:
        p.close()


def test_summary_lds_bound_form_with_general_steps():
    """Config 2's 512-plane geometry: the LDS-bound summary form, without the
    stripe table, on the same kind of mixed stream."""
    side = ranges_for()
    ranges = [(workloads.RANGE_BASE, 1 << 30, 3)] + side
    rec = mixed(600 * TILE, 51, side)
    p = parity.Pair(C2, ranges, tile_records=TILE)
    try:
        g, c = p.run_packed(rec)
        parity.assert_same(g, c, "config 2 geometry, mixed stream")
        p.check_state()
    finally:
        p.close()


ONE_CARRY = 4096  # tiles up to which the carry chain is one launch


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("tiles", [ONE_CARRY, ONE_CARRY + 1],
                         ids=["one-launch carry", "three-launch carry"])
def test_carry_forms_at_the_tile_boundary(profile, tiles):
    side = ranges_for()
    ranges = [(workloads.RANGE_BASE, 1 << 30, 3)] + side
    rec = mixed(tiles * 64, 60 + tiles % 2, side)
    assert len(rec) == tiles * 64
    p = parity.Pair(profile, ranges, tile_records=64)
    try:
        base = 0
        for k in range(2):  # the second run starts from the first one's state
            g, c = p.run_packed(rec, base_ps=base)
            parity.assert_same(g, c, f"{profile.name}, {tiles} tiles, run {k}")
            base = int(g[2]["makespan_ps"])
        p.check_state()
    finally:
        p.close()
