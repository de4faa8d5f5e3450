"""The EQ3 grid stencil and the thermal-coupled run on the GPU against the
CPU oracle.  Temperatures are compared for exact equality (the kernel
performs the oracle's IEEE operation sequence), which is stricter than the
1e-4 K relative bar; everything derived from them (hotspots, throttle
levels, refresh decisions, completions) is compared exactly."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
from hbfsim_amd import engine as eng
from hbfsim_amd import workloads as w

pytestmark = pytest.mark.gpu

f = oracle_py.addr
C4 = w.PROFILES / "c4.json"


def grid_kw(**kw):
    g = dict(w.C4_GRID)
    g.update(kw)
    return g


@pytest.mark.parametrize("shape,sweeps,steps", [
    ((64, 64, 8), 4, 3), ((7, 5, 3), 1, 2), ((7, 5, 3), 3, 1), ((33, 17, 1), 2, 4),
    ((1, 1, 4), 4, 2), ((40, 24, 16), 2, 1), ((130, 3, 2), 8, 1),
    # big enough for the 1,024-thread tiles (interiors of 24-50 cells, ragged
    # last tiles at every edge)
    ((400, 400, 8), 4, 3), ((390, 410, 6), 3, 2), ((512, 300, 4), 8, 1),
    ((1000, 700, 2), 1, 2),
    # at least 2^21 cells with 1-4 sweeps: the marching stencil (64-column
    # strips walked along y in segments; ragged last strips and segments,
    # 1 to 16 layers)
    ((1030, 260, 8), 4, 3), ((2048, 128, 8), 3, 2), ((700, 3000, 1), 2, 2),
    ((520, 260, 16), 4, 2), ((300, 1200, 6), 1, 3), ((129, 2100, 8), 4, 1),
    ((1100, 1000, 2), 4, 2),
    # odd pass counts of 3 (three two-step passes; two and a single step):
    # the passes route through a second scratch buffer and the last writes
    # the caller's array
    ((1030, 260, 8), 4, 6), ((700, 3000, 1), 2, 5),
    # 5-8 sweeps march with up to 8 layers (48-54 written columns per strip)
    ((600, 900, 4), 5, 1), ((700, 3000, 1), 6, 2), ((520, 520, 8), 7, 1),
    ((1030, 260, 8), 8, 2)])
def test_thermal_step_bit_exact(oracle, shape, sweeps, steps):
    import torch
    nx, ny, nz = shape
    n = nx * ny * nz
    g = grid_kw(nx=nx, ny=ny, nz=nz, sweeps=sweeps)
    rng = np.random.default_rng(nx * 7 + nz)
    t0 = rng.uniform(318.0, 340.0, n)
    power = rng.uniform(0.0, 0.05, n)
    th = eng.Thermal(**g)
    try:
        t = torch.from_numpy(t0.copy()).cuda()
        p = torch.from_numpy(power).cuda()
        th.step(p, t, steps)
        got = t.cpu().numpy()
    finally:
        th.close()
    want = t0.copy()
    for _ in range(steps):
        assert oracle.orc_thermal_grid_step(nx, ny, nz, g["capacity_j_per_k"], g["gx_w_per_k"],
                                            g["gy_w_per_k"], g["gz_w_per_k"], g["top_g_w_per_k"],
                                            g["ambient_k"], g["dt_s"], f(power), f(want), -1.0,
                                            sweeps) == sweeps
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape,sweeps", [((1030, 260, 8), 4), ((400, 400, 8), 4)])
def test_thermal_steps_across_calls(oracle, shape, sweeps):
    """One grid object stepped by two calls with different power arrays and
    odd and even step counts (the marching kernel keeps its launch geometry
    from the first call; the tiles rebuild theirs), against the oracle."""
    import torch
    nx, ny, nz = shape
    n = nx * ny * nz
    g = grid_kw(nx=nx, ny=ny, nz=nz, sweeps=sweeps)
    rng = np.random.default_rng(nx + ny)
    t0 = rng.uniform(318.0, 340.0, n)
    powers = [rng.uniform(0.0, 0.05, n), rng.uniform(0.0, 0.02, n)]
    th = eng.Thermal(**g)
    try:
        t = torch.from_numpy(t0.copy()).cuda()
        for p, steps in zip(powers, (3, 2)):
            th.step(torch.from_numpy(p).cuda(), t, steps)
        got = t.cpu().numpy()
    finally:
        th.close()
    want = t0.copy()
    for p, steps in zip(powers, (3, 2)):
        for _ in range(steps):
            oracle.orc_thermal_grid_step(nx, ny, nz, g["capacity_j_per_k"], g["gx_w_per_k"],
                                         g["gy_w_per_k"], g["gz_w_per_k"], g["top_g_w_per_k"],
                                         g["ambient_k"], g["dt_s"], f(p), f(want), -1.0, sweeps)
    np.testing.assert_array_equal(got, want)


def test_thermal_step_is_the_implicit_solve(oracle):
    """Six sweeps at the config-4 stiffness reach the dense backward-Euler
    solution (pinned to the compiled reference thermal.cpp) to 1e-12."""
    import torch
    nx, ny, nz = 12, 10, 8
    n = nx * ny * nz
    g = grid_kw(nx=nx, ny=ny, nz=nz, sweeps=6)
    rng = np.random.default_rng(11)
    t0 = rng.uniform(318.0, 330.0, n)
    power = rng.uniform(0.0, 0.2, n)
    th = eng.Thermal(**g)
    t = torch.from_numpy(t0.copy()).cuda()
    th.step(torch.from_numpy(power).cuda(), t, 1)
    got = t.cpu().numpy()
    th.close()
    ea, eb, eg = [], [], []
    for z in range(nz):
        for y in range(ny):
            for x in range(nx):
                i = (z * ny + y) * nx + x
                for ok, j, gg in ((x + 1 < nx, i + 1, g["gx_w_per_k"]),
                                  (y + 1 < ny, i + nx, g["gy_w_per_k"]),
                                  (z + 1 < nz, i + nx * ny, g["gz_w_per_k"])):
                    if ok:
                        ea.append(i), eb.append(j), eg.append(gg)
    ea, eb, eg = (np.array(ea, np.uint32), np.array(eb, np.uint32), np.array(eg))
    gb = np.array([g["top_g_w_per_k"] if i // (nx * ny) == nz - 1 else 0.0 for i in range(n)])
    dense = t0.copy()
    assert oracle.orc_thermal_dense_step(
        n, f(np.full(n, g["capacity_j_per_k"])), f(gb), f(np.full(n, g["ambient_k"])),
        f(np.zeros(n)), len(ea), f(ea), f(eb), f(eg), g["dt_s"], f(power * g["dt_s"]),
        f(dense)) == 0
    np.testing.assert_allclose(got, dense, rtol=1e-12)


def c4_case(n_records, layers=2):
    shape = w.OLMOE
    seg = w.c4_segments(shape, 1)
    seg = seg[: (n_records + shape.lines_per_expert - 1) // shape.lines_per_expert]
    rec = w.segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                            shape.issuers, 0, n_records)
    ranges = [(shape.expert_base(l_, e), shape.expert_bytes, 1)
              for l_ in range(layers) for e in range(shape.experts)]
    return rec, ranges


def run_pair(rec, ranges, grid, opts, age0, t0):
    import torch
    prof = oracle_py.load_profile(C4)
    params = oracle_py.engine_params(prof)
    orng, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    rel = oracle_py.reliability(grid, opts, params.dies)
    o_temp, o_age = t0.copy(), age0.copy()
    o_comp, o_rep, o_trace, o_state = oracle_py.coupled_run(params, orng, count, rel, rec,
                                                            o_temp, o_age)
    e = eng.Engine(str(C4))
    for base, length, perms in ranges:
        e.register(base, length, perms)
    th = eng.Thermal(**grid)
    try:
        d_rec = torch.from_numpy(np.ascontiguousarray(rec).view(np.int64)).cuda()
        d_comp = torch.empty(len(rec), dtype=torch.int64, device="cuda")
        d_temp = torch.from_numpy(t0.copy()).cuda()
        g_age = age0.copy()
        g_rep, g_erep = e.run_coupled(th, opts, d_rec, d_comp, d_temp, g_age)
        torch.cuda.synchronize()
        trace = th.trace()
        got = dict(comp=d_comp.cpu().numpy().view(np.uint64), temp=d_temp.cpu().numpy(),
                   age=g_age, rep=g_rep, erep=g_erep, trace=trace, state=e.state())
    finally:
        th.close()
        e.close()
    want = dict(comp=o_comp, temp=o_temp, age=o_age, rep=o_rep, trace=o_trace, state=o_state)
    return got, want


def assert_coupled_equal(got, want):
    t, u = got["trace"], want["trace"]
    assert t["windows"] == u["windows"] and t["dies"] == u["dies"]
    np.testing.assert_array_equal(t["hot"], u["hot"])
    np.testing.assert_array_equal(t["level"], u["level"])
    np.testing.assert_array_equal(t["refresh"], u["refresh"])
    np.testing.assert_array_equal(got["temp"], want["temp"])
    np.testing.assert_array_equal(got["age"], want["age"])
    np.testing.assert_array_equal(got["comp"], want["comp"])
    for k, v in want["rep"].items():
        assert got["rep"][k] == v, k
    s = want["state"]
    np.testing.assert_array_equal(got["state"]["plane_busy"], s.plane_busy)
    np.testing.assert_array_equal(got["state"]["channel_cursor"], s.channel_cursor)


def test_coupled_run_matches_oracle():
    """Reduced grid, strong heating: throttling (light and severe),
    deferral, and Arrhenius-derated refreshes all occur; every per-window
    decision, the final grid and every completion match the oracle."""
    rec, ranges = c4_case(200_000)
    grid = grid_kw(nx=16, ny=8, nz=8, sweeps=3)
    opts = dict(w.C4_RELIABILITY, access_energy_j=4e-7, retention_ps=500_000, light_k=320.0,
                severe_k=324.0, shutdown_k=340.0, hysteresis_k=0.5, action_delay_ps=1_000_000,
                min_dwell_ps=3_000_000, light_gap_ps=500)
    age0 = w.staggered_ages(64, opts["retention_ps"])
    t0 = np.full(16 * 8 * 8, 318.15)
    got, want = run_pair(rec, ranges, grid, opts, age0, t0)
    rep = want["rep"]
    assert rep["refreshes"] > 0 and rep["deferred"] > 0
    assert rep["level_windows"][1] > 0 and rep["level_windows"][2] > 0
    assert_coupled_equal(got, want)


@pytest.mark.parametrize("windows", [300, 1301])
def test_coupled_run_full_grid_prefix(windows):
    """The config-4 grid and parameters on the first 300 (one launch per
    window) or 1,301 windows of the config-4 trace (five replays of the
    chain's 256-window captured chunk, then 21 windows launched one by one,
    an odd count that ends in the scratch buffer)."""
    n = windows * 4000  # 4 lines per ns issued -> one window per 1 us
    rec, ranges = c4_case(n, layers=3)
    opts = dict(w.C4_RELIABILITY)
    age0 = w.staggered_ages(64, opts["retention_ps"])
    t0 = np.full(64 * 64 * 8, 318.15)
    got, want = run_pair(rec, ranges, dict(w.C4_GRID), opts, age0, t0)
    assert want["rep"]["windows"] == windows
    assert want["rep"]["refreshes"] > 0
    assert_coupled_equal(got, want)


def test_coupled_run_whole_config4():
    """The benchmarked config-4 run in full: the first 1e8 records of the
    OLMoE trace on all 1,024 expert ranges, the 64x64x8 grid stepped through
    all 25,000 windows with the config-4 reliability parameters from the
    ambient grid and staggered ages.  Every window's hotspots, levels and
    refresh flags, the final grid and ages, every demand completion, the
    report and the engine state equal the oracle's."""
    shape = w.OLMOE
    seg = w.c4_segments(shape, 2)
    d_rec = w.gpu_segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                  shape.issuers)[: w.C4_ACCESSES]
    rec = d_rec.cpu().numpy().view(np.uint64)
    del d_rec
    opts = dict(w.C4_RELIABILITY)
    age0 = w.staggered_ages(64, opts["retention_ps"])
    t0 = np.full(64 * 64 * 8, w.C4_GRID["ambient_k"])
    got, want = run_pair(rec, w.moe_ranges(shape), dict(w.C4_GRID), opts, age0, t0)
    rep = want["rep"]
    assert rep["windows"] == 25_000 and rep["demand_modeled"] == w.C4_ACCESSES
    assert rep["refreshes"] > 1000 and rep["deferred"] > 0
    assert rep["level_windows"][1] > 0 and rep["level_windows"][2] > 0
    assert_coupled_equal(got, want)


def test_coupled_without_events_is_the_plain_run():
    import torch
    rec, ranges = c4_case(100_000)
    opts = dict(w.C4_RELIABILITY, retention_ps=1 << 62, light_k=1e9, severe_k=1e9,
                shutdown_k=1e9)
    grid = grid_kw(nx=16, ny=8, nz=8, sweeps=2)
    d_rec = torch.from_numpy(np.ascontiguousarray(rec).view(np.int64)).cuda()
    out = []
    for coupled in (True, False):
        e = eng.Engine(str(C4))
        for base, length, perms in ranges:
            e.register(base, length, perms)
        comp = torch.empty(len(rec), dtype=torch.int64, device="cuda")
        if coupled:
            th = eng.Thermal(**grid)
            temp = torch.full((16 * 8 * 8,), 318.15, dtype=torch.float64, device="cuda")
            rep, erep = e.run_coupled(th, opts, d_rec, comp, temp, np.zeros(64, np.uint64))
            th.close()
            assert rep["refreshes"] == 0 and rep["deferred"] == 0
        else:
            erep = e.run(d_rec, comp)
        torch.cuda.synchronize()
        out.append((comp.cpu().numpy(), erep))
        e.close()
    np.testing.assert_array_equal(out[0][0], out[1][0])
    assert out[0][1] == out[1][1]


def test_thermal_rejects_bad_shapes():
    with pytest.raises(eng.nat.HbfSimError):
        eng.Thermal(**grid_kw(sweeps=0))
    with pytest.raises(eng.nat.HbfSimError):
        eng.Thermal(**grid_kw(sweeps=9))
    with pytest.raises(eng.nat.HbfSimError):
        eng.Thermal(**grid_kw(nz=64, sweeps=8))
    # no tile holds 12 layers at 8 sweeps, and the marching kernel takes at
    # most 8 layers at 5-8 sweeps
    with pytest.raises(eng.nat.HbfSimError):
        eng.Thermal(**grid_kw(nx=1024, ny=1024, nz=12, sweeps=8))
