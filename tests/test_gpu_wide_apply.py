"""The four-wave apply pass.  A run of at least 2^24 packed records on an
engine whose previous run had fewer page-register hits than an eighth of its
modeled records (a stream of general steps) takes the apply kernel built for
four waves per SIMD; any other run takes the three-wave one.  The form is a
matter of speed only: every completion, status, report and state word must
equal the oracle's either way, with linear, grouped and split steps mixed
into the general ones."""
from __future__ import annotations

import json

import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0
from test_gpu_split import split_stream
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

BIG = 1 << 24


def test_wide_apply_takes_over_on_general_streams():
    first = workloads.config0(n=BIG, seed=21, write_fraction_per_mille=50)
    second = workloads.config0(n=BIG, seed=22, write_fraction_per_mille=50)
    side = ranges_for()
    # general steps, then linear, grouped and split steps, then general again
    mixed = chain_clocks(second.records[: BIG // 2], linear_stream(5, 3000, side),
                         contiguous_stream(6, 400, side), split_stream(7, 2000, side),
                         second.records[BIG // 2:])
    linear = chain_clocks(linear_stream(8, 4000, side), contiguous_stream(9, 400, side))
    # tiles of 4,096 records: the large runs have more tiles than one round of
    # three-wave slots, so their summary pass is the four-wave form too
    p = parity.Pair(C0, first.ranges + side, tile_records=4096)
    try:
        # no earlier run: the three-wave form
        g, c = p.run_packed(first.records)
        parity.assert_same(g, c, "first general run")
        assert p.engine.apply_waves() == 3
        assert g[2]["page_hits"] * 8 < g[2]["modeled"]
        # the previous run was general: the four-wave form, mixed steps too
        g, c = p.run_packed(mixed, base_ps=int(g[2]["makespan_ps"]))
        parity.assert_same(g, c, "mixed run, four-wave apply")
        assert p.engine.apply_waves() == 4
        p.check_state()
        # a small run keeps the three-wave form whatever came before
        g, c = p.run_packed(linear, base_ps=int(g[2]["makespan_ps"]))
        parity.assert_same(g, c, "small linear run")
        assert p.engine.apply_waves() == 3
        p.check_state()
    finally:
        p.close()


def test_wide_apply_hybrid_sampling(tmp_path):
    """Hybrid mode (every modeled record through the reference sampler, rate
    1%, 1,000 warm-up requests) in both forms of the apply pass: sequence
    numbers carry across the runs."""
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=0.01, reference_warmup_requests=1000)
    path = tmp_path / "c0-hybrid-wide.json"
    path.write_text(json.dumps(prof))
    first = workloads.config0(n=BIG, seed=31)
    second = workloads.config0(n=BIG, seed=32, write_fraction_per_mille=30)
    p = parity.Pair(path, first.ranges, mode="hybrid")
    try:
        g, c = p.run_packed(first.records)
        parity.assert_same(g, c, "hybrid, three-wave apply")
        assert p.engine.apply_waves() == 3 and g[2]["hybrid_sampled"] > 0
        g, c = p.run_packed(second.records, base_ps=int(g[2]["makespan_ps"]))
        parity.assert_same(g, c, "hybrid, four-wave apply")
        assert p.engine.apply_waves() == 4
        p.check_state()
    finally:
        p.close()


def test_wide_apply_leaves_linear_streams_alone():
    """A large run after a run of mostly page-register hits stays on the
    three-wave form."""
    side = ranges_for()
    parts = [linear_stream(10 + k, 4000, side) for k in range(4)]
    linear = chain_clocks(*parts)
    reps = -(-BIG // len(linear))
    big = chain_clocks(*([linear] * reps))
    p = parity.Pair(C0, side)
    try:
        g, c = p.run_packed(linear)
        parity.assert_same(g, c, "linear warm-up")
        assert g[2]["page_hits"] * 8 >= g[2]["modeled"]
        g, c = p.run_packed(big, base_ps=int(g[2]["makespan_ps"]))
        parity.assert_same(g, c, "large linear run")
        assert p.engine.apply_waves() == 3
        p.check_state()
    finally:
        p.close()
