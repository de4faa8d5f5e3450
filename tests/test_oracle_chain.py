"""Multi-window pins of the oracle's thermal-coupled chain
(orc_reliability_chain, orc_coupled_run) by checks that do not reuse the
oracle's own decision code:

* isolated cells (no conductance): every die's temperature follows the closed
  form T' = T + P dt / C, so the whole trace -- ages, refresh flags, the heat
  a refresh adds to the next window -- is computed here by hand from the
  Arrhenius law (reliability.py:17-23) and the age rule (reliability.py:93-108,
  cpu_service.cpp:169-217: age grows by window x AF(hotspot at the window's
  start), a refresh is due at the retention period and restarts the age);
* a coupled grid over 24 windows with refreshes: every window is replayed
  through the dense backward-Euler solve (pinned to the compiled thermal.cpp)
  with power rebuilt from the counts and the chain's refresh flags, and the
  flags and ages are then recomputed from the replayed hotspots;
* the coupled run's composition (counts -> chain -> admission -> refresh
  records -> merge -> engine) restated in Python around the engine."""
from __future__ import annotations

import ctypes
import math

import numpy as np

import oracle_py
from test_oracle_reliability import GRID, OPTS, grid_edges

f = oracle_py.addr
KB = 8.62e-5


def af(t, ea=1.04, tref=358.15):
    return math.exp(ea / KB * (1.0 / tref - 1.0 / t))


def bin_of(t):
    """1/16-K bins from 200 K, clamped to [0, 4095]."""
    if not t >= 200.0:
        return 0
    return min(4095, int((t - 200.0) * 16.0))


def table_entry(t, window_ps):
    """Retention credit of a window spent at hotspot t: window x AF at the
    centre of t's bin, rounded to the nearest ps (half away from zero)."""
    b = bin_of(t)
    v = window_ps * af(200.0 + (b + 0.5) / 16.0)
    return int(math.floor(v + 0.5))


def run_chain(oracle, rel, counts, temp, age, ndie):
    windows = counts.shape[0]
    ctl = oracle_py.OrcControl(0, oracle_py.NO_PENDING, 0, 0)
    hot = np.zeros((windows + 1) * ndie)
    level = np.zeros(windows, np.uint8)
    refresh = np.zeros(windows * ndie, np.uint8)
    c = np.ascontiguousarray(counts, np.uint32)
    assert oracle.orc_reliability_chain(ctypes.byref(rel), f(c), windows, f(temp), f(age),
                                        ctypes.byref(ctl), f(hot), f(level), f(refresh)) == 0
    return hot.reshape(windows + 1, ndie), level, refresh.reshape(windows, ndie)


def test_isolated_cells_trace_by_hand(oracle):
    """Four dies of four cells each, no conductance: T' = T + P dt / C per
    cell.  Each access adds 0.25 K and each refresh 3 K to its die (E / (C *
    cells)), and every temperature sits at a bin centre so rounding never
    moves a bin.  Retention 3 us at 1-us windows."""
    grid = dict(nx=4, ny=2, nz=2, sweeps=3, capacity_j_per_k=1e-6, gx_w_per_k=0.0,
                gy_w_per_k=0.0, gz_w_per_k=0.0, top_g_w_per_k=0.0, ambient_k=318.15,
                dt_s=1e-6)
    cells = 4  # (4 / 2) x (2 / 1) x (2 / 2)
    opts = dict(OPTS, regions_x=2, regions_y=1, static_power_w=0.0,
                access_energy_j=0.25 * 1e-6 * cells, refresh_energy_j=3.0 * 1e-6 * cells,
                retention_ps=3_000_000)
    rel = oracle_py.reliability(grid, opts, 2)
    ndie = 4
    centre = lambda b: 200.0 + (b + 0.5) / 16.0  # noqa: E731
    t_die = [centre(2530), centre(2850), centre(2464), centre(2530)]  # ~358, 378, 354, 358 K
    age0 = [0, 0, 0, 3_000_000]
    counts = np.array([[0, 0, 0, 0],
                       [4, 0, 0, 0],
                       [0, 0, 8, 0],
                       [0, 0, 0, 0],
                       [0, 1, 0, 0],
                       [0, 0, 0, 0]], np.uint32)
    windows = counts.shape[0]

    # the trace by hand
    want_hot = np.zeros((windows + 1, ndie))
    want_ref = np.zeros((windows, ndie), np.uint8)
    want_age_after = np.zeros((windows, ndie), np.uint64)
    t = list(t_die)
    a = list(age0)
    want_hot[0] = t
    for w in range(windows):
        for d in range(ndie):
            if w > 0:
                a[d] += table_entry(want_hot[w][d], 1_000_000)
            if a[d] >= 3_000_000:
                want_ref[w][d] = 1
                a[d] = 0
            want_age_after[w][d] = a[d]
        for d in range(ndie):
            t[d] = t[d] + 0.25 * int(counts[w][d]) + 3.0 * int(want_ref[w][d])
        want_hot[w + 1] = t
    # every hotspot sits at a bin centre (no rounding can move a bin)
    frac = (want_hot - 200.0) * 16.0 - np.floor((want_hot - 200.0) * 16.0)
    assert np.all(np.abs(frac - 0.5) < 1e-6)
    # the hand trace exercises what the rule must get right
    assert want_ref[0].tolist() == [0, 0, 0, 1]        # due at issue -> window 0
    assert want_ref[:, 1].sum() >= 4                    # hot die refreshes often
    assert want_ref[:, 2].sum() >= 1 and want_ref[:3, 2].sum() == 0  # cool die ages slowly

    def initial():
        # cell order x fastest; die = region(x // 2) * 2 + z
        tt = np.zeros(16)
        for z in range(2):
            for y in range(2):
                for x in range(4):
                    tt[(z * 2 + y) * 4 + x] = t_die[(x // 2) * 2 + z]
        return tt, np.array(age0, np.uint64)

    temp, age = initial()
    hot, level, refresh = run_chain(oracle, rel, counts, temp, age, ndie)
    np.testing.assert_array_equal(refresh, want_ref)
    np.testing.assert_allclose(hot, want_hot, rtol=1e-13)
    assert age.tolist() == want_age_after[-1].tolist()
    assert level.tolist() == [0] * windows
    # ages after each prefix of windows, from runs over the prefixes
    for w in range(1, windows + 1):
        tp, ap = initial()
        run_chain(oracle, rel, counts[:w], tp, ap, ndie)
        assert ap.tolist() == want_age_after[w - 1].tolist(), w
    # a refresh in window w raises the die by 3 K at window w + 1, on top of
    # the accesses (E_refresh / dt / cells of power for one window)
    for w in range(windows):
        for d in range(ndie):
            rise = hot[w + 1][d] - hot[w][d]
            assert abs(rise - (0.25 * counts[w][d] + 3.0 * refresh[w][d])) < 1e-9


def build_power(nx, ny, nz, regions_x, regions_y, dies, static_w, pa, pr, counts_w, ref_w):
    rw, rh, lpd = nx // regions_x, ny // regions_y, nz // dies
    p = np.zeros(nx * ny * nz)
    for z in range(nz):
        for y in range(ny):
            for x in range(nx):
                d = ((y // rh) * regions_x + x // rw) * dies + z // lpd
                p[(z * ny + y) * nx + x] = static_w + counts_w[d] * pa + ref_w[d] * pr
    return p


def die_max(t, nx, ny, nz, regions_x, regions_y, dies):
    rw, rh, lpd = nx // regions_x, ny // regions_y, nz // dies
    out = np.zeros(regions_x * regions_y * dies)
    for z in range(nz):
        for y in range(ny):
            for x in range(nx):
                d = ((y // rh) * regions_x + x // rw) * dies + z // lpd
                out[d] = max(out[d], t[(z * ny + y) * nx + x])
    return out


def test_chain_replayed_through_the_dense_solve(oracle):
    """24 windows of an 8x4x4 grid (2 regions x 2 dies) with a retention
    period short enough for repeated refreshes.  Each window is replayed
    through the dense backward-Euler solve with power rebuilt from the counts
    and the chain's refresh flags; every hotspot row agrees at 1e-12.  The
    flags and final ages are then recomputed from the replayed hotspots with
    this file's own retention arithmetic."""
    nx, ny, nz, dies, rx, ry = 8, 4, 4, 2, 2, 1
    ndie = rx * ry * dies
    n = nx * ny * nz
    cells = (nx // rx) * (ny // ry) * (nz // dies)
    opts = dict(OPTS, regions_x=rx, regions_y=ry, access_energy_j=4e-8,
                refresh_energy_j=2e-5, retention_ps=2_600_000)
    rel = oracle_py.reliability(GRID, opts, dies)
    windows = 24
    rng = np.random.default_rng(11)
    counts = rng.integers(0, 400, (windows, ndie)).astype(np.uint32)
    t0 = rng.uniform(330.0, 372.0, n)
    age0 = np.array([0, 1_000_000, 2_500_000, 2_600_000], np.uint64)
    temp, age = t0.copy(), age0.copy()
    hot, level, refresh = run_chain(oracle, rel, counts, temp, age, ndie)
    assert refresh.sum() >= 8 and refresh[:, 0].sum() >= 2  # repeated refreshes of a die

    dt, C = GRID["dt_s"], GRID["capacity_j_per_k"]
    pa = (opts["access_energy_j"] / dt) / cells
    pr = (opts["refresh_energy_j"] / dt) / cells
    ea, eb, eg = grid_edges(nx, ny, nz, GRID["gx_w_per_k"], GRID["gy_w_per_k"],
                            GRID["gz_w_per_k"])
    gb = np.array([GRID["top_g_w_per_k"] if i // (nx * ny) == nz - 1 else 0.0
                   for i in range(n)])
    tb = np.full(n, GRID["ambient_k"])
    cap = np.full(n, C)
    zero = np.zeros(n)
    t = t0.copy()
    np.testing.assert_array_equal(hot[0], die_max(t, nx, ny, nz, rx, ry, dies))
    for w in range(windows):
        power = build_power(nx, ny, nz, rx, ry, dies, opts["static_power_w"], pa, pr,
                            counts[w], refresh[w])
        assert oracle.orc_thermal_dense_step(n, f(cap), f(gb), f(tb), f(zero), len(ea), f(ea),
                                             f(eb), f(eg), dt, f(power * dt), f(t)) == 0
        np.testing.assert_allclose(hot[w + 1], die_max(t, nx, ny, nz, rx, ry, dies),
                                   rtol=1e-12, err_msg=f"window {w}")
    np.testing.assert_allclose(temp, t, rtol=1e-12)

    # decisions from the replayed hotspots: between two refreshes of a die the
    # credits stay below the period, and the flagged window reaches it
    a = [int(v) for v in age0]
    for w in range(windows):
        for d in range(ndie):
            if w > 0:
                a[d] += table_entry(hot[w][d], opts["window_ps"])
            due = a[d] >= opts["retention_ps"]
            assert bool(refresh[w][d]) == due, (w, d, a[d])
            if due:
                a[d] = 0
    assert age.tolist() == a


def py_defer(level, window_ps, t, limit):
    w = t // window_ps
    if w >= len(level) or level[w] < limit:
        return t
    w += 1
    while w < len(level) and level[w] >= limit:
        w += 1
    return w * window_ps


def test_coupled_run_is_its_composition(oracle):
    """orc_coupled_run on a 200,000-record slice of the config-4 trace with
    a short retention period and low throttle thresholds equals, completion
    for completion: demand admitted past severe/shutdown windows and spaced
    by the light gap, refresh records of each flagged die (its k-th refresh
    on plane k % P, row k / P, held past shutdown windows) merged ahead of
    demand at equal times, the engine over the merged stream, and latencies
    from the original issue.  Admission, placement and merge are restated
    here in Python; the chain and the engine are pinned on their own."""
    from test_oracle_reliability import c4_small_case
    prof, ranges, rec = c4_small_case(200_000)
    p = oracle_py.engine_params(prof)
    orng, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    grid = dict(GRID, nx=8, ny=4, nz=8, sweeps=2)
    opts = dict(OPTS, regions_x=4, regions_y=2, access_energy_j=2e-7, retention_ps=500_000,
                light_k=320.0, severe_k=325.0, shutdown_k=327.0, hysteresis_k=0.5,
                action_delay_ps=1_000_000, min_dwell_ps=2_000_000, light_gap_ps=500)
    rel = oracle_py.reliability(grid, opts, p.dies)
    temp = np.full(8 * 4 * 8, 318.15)
    age = np.zeros(64, np.uint64)
    comp, rep, trace, st = oracle_py.coupled_run(p, orng, count, rel, rec, temp.copy(),
                                                 age.copy())
    level = trace["level"].tolist()
    flags = trace["refresh"]
    W, ndie = flags.shape
    wp = opts["window_ps"]
    assert rep["refreshes"] > 0 and rep["deferred"] > 0
    assert 3 in level and 1 in level  # shutdown and light windows both occur

    # admission (cpu_service.cpp:256-285)
    admit, gate = [], 0
    for t in rec[:, 2].tolist():
        e = py_defer(level, wp, t, 2)
        we = e // wp
        gap = opts["light_gap_ps"] if we < W and level[we] == 1 else 0
        a = max(e, gate)
        admit.append(a)
        gate = a + gap
    # refresh records: die d = (c * ways + way) * dies + die-in-channel
    sizes = [p.channels, p.ways, p.dies, p.planes]
    order = list(p.order)
    div, stride = [0] * 4, 1
    for ax in order:
        div[ax] = stride
        stride *= sizes[ax]
    rows = max(1, p.media_pages // stride)
    ordinal = [0] * ndie
    extra = []
    for w in range(W):
        for d in range(ndie):
            if not flags[w][d]:
                continue
            q, dd = d // p.dies, d % p.dies
            k = ordinal[d]
            ordinal[d] += 1
            coord = [q // p.ways, q % p.ways, dd, k % p.planes]
            page = ((k // p.planes) % rows) * stride + sum(c * div[ax]
                                                           for ax, c in enumerate(coord))
            extra.append((page, 2 * prof["page_bytes"], py_defer(level, wp, w * wp, 3),
                          0x102))
    assert len(extra) == rep["refreshes"]
    # merge: refreshes first at equal times
    merged, pos, j = [], [], 0
    for i in range(len(rec)):
        while j < len(extra) and extra[j][2] <= admit[i]:
            merged.append(extra[j])
            j += 1
        pos.append(len(merged))
        merged.append((int(rec[i, 0]), int(rec[i, 1]), admit[i], int(rec[i, 3])))
    merged.extend(extra[j:])
    m = np.array(merged, np.uint64)
    q = oracle_py.engine_params(prof)
    q.media_records = 1
    mcomp, mst, erep, st2 = oracle_py.run(q, orng, count, m)
    got = mcomp[np.array(pos)]
    np.testing.assert_array_equal(comp, got)
    lat = got.astype(object) - rec[:, 2].astype(object)
    modeled = (mst[np.array(pos)] & 3) == 0
    assert rep["demand_modeled"] == int(modeled.sum())
    assert rep["latency_sum_ps"] == int(sum(lat[modeled]))
    assert rep["latency_max_ps"] == int(max(lat[modeled]))
    assert rep["makespan_ps"] == erep["makespan_ps"]
    assert rep["deferred"] == int(sum(1 for a, t in zip(admit, rec[:, 2].tolist()) if a > t))
    np.testing.assert_array_equal(st.plane_busy_total, st2.plane_busy_total)
