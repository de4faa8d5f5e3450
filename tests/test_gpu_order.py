"""Streams whose issue time goes back, on the GPU.  The engine serves every
resource in (issue time, stream position) order (the order of the
reference's MQSim adapter, mqsim_online.cpp:269-289): the summary pass
notices a record below its predecessor, the run leaves the engine state
untouched, and a copy sorted on the GPU is timed with results written back
to stream positions.  Checked bit for bit against the oracle and against
the same engine run on the records sorted by numpy's stable argsort, on
every pipeline (both record forms, linear batches and groups, hybrid
sampling, two page registers, warp grouping, the empirical model), plus the
entry points that refuse such streams without changing anything."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import _native as nat
from hbfsim_amd import engine as eng
from hbfsim_amd import workloads as w
from hbfsim_amd.engine import pack_records
from test_gpu_linear import contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0, C2

pytestmark = pytest.mark.gpu


def unordered_stream(seed):
    """Linear steps (some issued far back in time), contiguous groups and
    random records, each part on its own clock, so the issue time falls back
    between parts and inside them."""
    rng = np.random.default_rng(seed)
    ranges = ranges_for(count=4, pages=120)
    lin = linear_stream(seed, 500, ranges, kinds={"lin": 0.85, "late": 0.05, "write": 0.05,
                                                  "bypass": 0.05})
    grp = contiguous_stream(seed + 1, 80, ranges)
    s = w.config0(n=6000, seed=seed, write_fraction_per_mille=100)
    rnd = s.records.copy()
    r = ranges[int(rng.integers(0, 3))]
    rnd[:, 0] = np.uint64(r[0]) + (rnd[:, 0] - np.uint64(w.RANGE_BASE)) % np.uint64(r[1])
    rec = np.concatenate([lin, grp, rnd])
    assert np.any(rec[1:, 2] < rec[:-1, 2])
    return ranges, rec


def sorted_pair_run(pair, rec, packed, base_ps=0):
    """The engine on the records permuted by a stable argsort of issue time,
    results written back to stream positions."""
    order = np.argsort(rec[:, 2], kind="stable")
    g, _ = pair.run_packed(rec[order], base_ps) if packed else pair.run(rec[order], base_ps)
    comp = np.empty_like(g[0])
    comp[order] = g[0]
    st = np.empty_like(g[1])
    st[order] = g[1]
    return comp, st, g[2]


@pytest.mark.parametrize("seed,profile,options", [
    (1, C0, {}), (2, C2, {}), (3, C0, {"plane_contention": 0}), (4, C2, {"transfer_page": 1}),
    (5, C0, {"tile_records": 64 * 8}), (6, C2, {"tile_records": 64 * 64}),
    (7, C0, {"page_buffers": 0})])
def test_unordered_both_forms(seed, profile, options):
    ranges, rec = unordered_stream(seed)
    a = parity.Pair(profile, ranges, **options)
    b = parity.Pair(profile, ranges, **options)
    ref = parity.Pair(profile, ranges, **options)
    try:
        base = 1000 * seed
        ga, ca = a.run(rec, base)
        parity.assert_same(ga, ca, f"seed {seed} 32-byte")
        packed = options.get("page_buffers", 1) == 1  # packed runs keep one page register
        if packed:
            gb, cb = b.run_packed(rec, base)
            parity.assert_same(gb, cb, f"seed {seed} packed")
        else:
            gb, cb = b.run(rec, base)
        sc, ss, sr = sorted_pair_run(ref, rec, packed=packed, base_ps=base)
        np.testing.assert_array_equal(ga[0], sc)
        np.testing.assert_array_equal(ga[1], ss)
        assert ga[2] == sr
        # state carries into an ordered second run exactly as the oracle's
        rec2 = w.config0(n=3000, seed=seed + 50).records
        rec2[:, 0] = rec[:3000, 0]
        parity.assert_same(*a.run(rec2, int(ga[2]["makespan_ps"])), "second run")
        a.check_state()
        b.check_state()
        ref.check_state()
    finally:
        a.close()
        b.close()
        ref.close()


def test_unordered_hybrid_sequence_follows_sorted_order():
    """Hybrid sampling: sequence numbers are taken in (issue, position)
    order, so the sampled records are the sorted run's."""
    ranges, rec = unordered_stream(11)
    import json
    import tempfile
    import pathlib
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=0.05, reference_warmup_requests=40)
    path = pathlib.Path(tempfile.mkdtemp()) / "c0-hybrid.json"
    path.write_text(json.dumps(prof))
    p = parity.Pair(path, ranges, mode="hybrid")
    ref = parity.Pair(path, ranges, mode="hybrid")
    try:
        g, c = p.run(rec)
        parity.assert_same(g, c, "hybrid unordered")
        assert g[2]["hybrid_sampled"] > 40
        sc, ss, sr = sorted_pair_run(ref, rec, packed=False)
        np.testing.assert_array_equal(g[1], ss)
        assert g[2] == sr
        p.check_state()
    finally:
        p.close()
        ref.close()


def test_unordered_two_page_registers():
    ranges, rec = unordered_stream(12)
    p = parity.Pair(C0, ranges, page_buffers=2)
    try:
        g, c = p.run(rec)
        parity.assert_same(g, c, "K=2 unordered")
        assert g[2]["page_hits"] > 0
        p.check_state()
    finally:
        p.close()


def test_unordered_warp_grouping():
    """Warp groups in a stream that falls back: groups are checked on the
    stream as given and again once sorted, where records of equal issue time
    from the two halves meet.  With distinct group ids the sorted groups are
    valid and timed; with the ids reused, two groups of one id and two issue
    times end up side by side and both sides refuse the run."""
    from test_oracle_grouping import grouping_ranges, warp_stream
    ranges = grouping_ranges()
    a = warp_stream(21, 300, ranges)
    b = warp_stream(22, 300, ranges)  # its own clock from 0: falls back
    gid = b[:, 3] >> np.uint64(32)
    moved = b.copy()
    moved[:, 3] += np.where(gid != 0, np.uint64(10_000 << 32), np.uint64(0))
    p = parity.Pair(C0, ranges, warp_grouping=1)
    try:
        g, c = p.run(np.concatenate([a, moved]))
        parity.assert_same(g, c, "grouping unordered")
        assert g[2]["grouped"] > 0
        p.check_state()
        before = p.engine.state()
        import torch
        with pytest.raises(nat.HbfSimError) as err:
            p.engine.run(parity.to_device(np.concatenate([a, b])),
                         torch.zeros(len(a) + len(b), dtype=torch.int64, device="cuda"))
        assert err.value.code == nat.HBFSIM_INVALID_ARGUMENT
        with pytest.raises(RuntimeError, match="failed: 6"):
            oracle_py.run(p.params, p.ranges, p.count, np.concatenate([a, b]), 0, p.ostate)
        after = p.engine.state()
        for k in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(after[k], before[k], k)
        p.check_state()
    finally:
        p.close()


def test_unordered_empirical():
    from test_gpu_empirical import burst_stream, check_burst, make_pair
    a = burst_stream(20_000, 31)
    b = burst_stream(20_000, 32)
    rec = np.concatenate([a, b])  # the second stream's clock starts again
    p = make_pair()
    try:
        g, c = p.run(rec)
        parity.assert_same(g, c, "empirical unordered")
        check_burst(p)
    finally:
        p.close()


def test_ordered_ties_are_not_resorted():
    """Equal issue times in stream order are already in order: the run is a
    plain one (one engine pass), equal to the oracle."""
    s = w.config0(n=40_000, seed=8, write_fraction_per_mille=50)
    rec = s.records.copy()
    rec[1::2, 2] = rec[0::2, 2][: len(rec[1::2])]
    assert np.all(rec[1:, 2] >= rec[:-1, 2])
    p = parity.Pair(C0, s.ranges)
    try:
        parity.assert_same(*p.run(rec), "ties")
        p.check_state()
    finally:
        p.close()


def test_noalloc_refuses_unordered_untouched():
    import torch
    s = w.config0(n=20_000, seed=3)
    e = eng.Engine(str(C0))
    for base, length, perms in s.ranges:
        e.register(base, length, perms)
    try:
        d_rec = pack_records(torch.from_numpy(s.records.view(np.int64)).cuda())
        comp = torch.zeros(len(s.records), dtype=torch.int64, device="cuda")
        e.run_packed(d_rec, comp)  # the engine exists and holds state
        before, totals, report = e.state(), e.busy_totals(), e.report()
        bad = s.records.copy()
        bad[[100, 101], 2] = bad[[101, 100], 2]
        d_bad = pack_records(torch.from_numpy(bad.view(np.int64)).cuda())
        with pytest.raises(nat.HbfSimError) as err:
            e.run_packed_noalloc(d_bad, comp)
        assert err.value.code == nat.HBFSIM_INVALID_ARGUMENT
        after = e.state()
        for k in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(after[k], before[k], k)
        assert after["sequence"] == before["sequence"]
        for x, y in zip(e.busy_totals(), totals):
            np.testing.assert_array_equal(x, y)
        assert e.report() == report
    finally:
        e.close()


def coupled_setup():
    from test_gpu_thermal import c4_case, grid_kw
    import torch
    rec, ranges = c4_case(20_000)
    grid = grid_kw(nx=16, ny=8, nz=8, sweeps=3)
    opts = dict(w.C4_RELIABILITY, retention_ps=500_000)
    age0 = w.staggered_ages(64, opts["retention_ps"])
    t0 = np.linspace(318.0, 330.0, 16 * 8 * 8)
    return torch, rec, ranges, grid, opts, age0, t0


@pytest.mark.parametrize("case", ["unordered", "grouping", "two_registers"])
def test_coupled_refusals_leave_everything(case):
    """Refused before the grid, the ages or the engine change."""
    torch, rec, ranges, grid, opts, age0, t0 = coupled_setup()
    C4 = w.PROFILES / "c4.json"
    e = eng.Engine(str(C4))
    for base, length, perms in ranges:
        e.register(base, length, perms)
    th = eng.Thermal(**grid)
    try:
        if case == "unordered":
            rec = rec.copy()
            rec[[500, 9000], 2] = rec[[9000, 500], 2]  # records share issue times in fours
            assert np.any(rec[1:, 2] < rec[:-1, 2])
            want = nat.HBFSIM_INVALID_ARGUMENT
        elif case == "grouping":
            e.set_options(warp_grouping=1)
            want = nat.HBFSIM_UNSUPPORTED
        else:
            e.set_options(page_buffers=2)
            want = nat.HBFSIM_UNSUPPORTED
        d_rec = torch.from_numpy(np.ascontiguousarray(rec).view(np.int64)).cuda()
        d_comp = torch.zeros(len(rec), dtype=torch.int64, device="cuda")
        d_temp = torch.from_numpy(t0.copy()).cuda()
        age = age0.copy()
        before = e.state()
        with pytest.raises(nat.HbfSimError) as err:
            e.run_coupled(th, opts, d_rec, d_comp, d_temp, age)
        torch.cuda.synchronize()
        assert err.value.code == want
        np.testing.assert_array_equal(d_temp.cpu().numpy(), t0)
        np.testing.assert_array_equal(age, age0)
        after = e.state()
        for k in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(after[k], before[k], k)
    finally:
        th.close()
        e.close()
