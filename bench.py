"""Benchmark of the HBF access-timing engine on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--config c2|c0|c1|c3|c4|thermal|general|hybrid|link]

A step is one pass of the timing engine over one batch of access records
resident in HBM (one decode step of the workload); engine state carries from
step to step and each step's issue times start at the previous step's
makespan.  Prints one JSON line with the modeled accesses/s, the roofline of
the dominant kernel (HIP-event timed on the engine's stream) and the CPU
oracle's rate on a bounded sample of the same stream, timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
PEAK_FP64_TFLOPS = 78.6  # MI355X dense FP64 (vector / matrix)
# EQ3 Jacobi update per cell and sweep: 6 neighbour products, 7 additions
# (the six terms and the ambient term onto the right-hand side) and the
# product with 1 / den
THERMAL_FLOPS_PER_CELL_SWEEP = 14
# Algorithmic bytes per access: the record in + the 8-B completion out, 40 B
# with 32-byte records and 24 B with packed 16-byte ones (the roofline of
# each form is its own; the two are never mixed).  The same bytes split over
# the two per-record kernels: the summary pass reads each record, the apply
# pass writes each completion (linear steps replay from the summary pass's
# step descriptors, not from the records).
RECORD_BYTES = {"packed": 16, "32": 32}


def kernel_bytes(records: str, apply_rereads: bool = False) -> dict:
    """Algorithmic bytes per access of the two per-record kernels.  The apply
    pass writes the 8-B completion; it re-reads the record too where steps
    are replayed from their records (streams without linear steps, such as
    random ones), and replays linear steps from the summary pass's step
    descriptors otherwise."""
    return {"k_summary": RECORD_BYTES[records],
            "k_apply": 8 + (RECORD_BYTES[records] if apply_rereads else 0)}


def profile_kernel_us(summary: str, kernel: str) -> float | None:
    """Average duration (us) of `kernel` in a committed kernel-trace summary
    under profiles/ (rocprofv3 --kernel-trace --stats, one line per kernel);
    of several instantiations, the one launched most often (the timed steps'
    form: a warm-up run may take another)."""
    import re
    path = ROOT / "profiles" / summary
    if not path.exists():
        return None
    best = None
    for line in path.read_text().splitlines():
        m = re.match(r"(\S+?(?:<[^>]*>)?)\s+(\d+)\s+([\d.]+)\s", line)
        if m and not line.startswith("#") and (m.group(1) == kernel or
                                               m.group(1).startswith(kernel + "<")):
            if best is None or int(m.group(2)) > best[0]:
                best = (int(m.group(2)), float(m.group(3)))
    return None if best is None else best[1]


def roofline_from_profile(summary: str, kernel: str, bytes_per_launch: float) -> dict | None:
    """The same roofline recomputed from a committed kernel summary: the
    algorithmic bytes of one launch over the profile's average duration."""
    us = profile_kernel_us(summary, kernel)
    if us is None:
        return None
    gbps = bytes_per_launch / (us / 1e6) / 1e9
    return {"source": f"profiles/{summary}", "kernel_avg_us": us, "achieved": gbps,
            "frac": gbps / PEAK_HBM_GBPS}


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--batches", type=int, default=None,
                    help="distinct decode-step batches generated for config c2 (default: one "
                         "per warm-up and timed step, at most 12; steps beyond reuse them "
                         "in turn)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="budget for the CPU-oracle baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--records", choices=("packed", "32"), default="packed",
                    help="record form in HBM: packed 16-byte records (hbf_record16) or "
                         "32-byte ones (hbf_record32); packing runs before the timed region")
    ap.add_argument("--no-compare", action="store_true",
                    help="with packed records, skip timing the same steps from 32-byte ones")
    ap.add_argument("--no-extra", action="store_true",
                    help="config c2: skip the read/write ceilings and the general-path, "
                         "hybrid, UCIe-link, config-4, EQ3-stencil and config 0/1/3 sub-lines")
    ap.add_argument("--c4-records", type=int, default=None,
                    help="config c4: time only this prefix of the trace (fewer windows; "
                         "below 512 windows the chain launches window by window, which "
                         "counter runs need)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first fill and copy 2 GiB (known HBM bytes) so that counter runs "
                         "can calibrate FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


def copy_probe() -> None:
    """A plain fill (2 GiB written) and copy (2 GiB read + 2 GiB written)
    outside the timed region: the reference kernels for HBM counters."""
    import torch
    n = (1 << 31) // 4
    src = torch.empty(n, dtype=torch.float32, device="cuda")
    src.fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def gpu_random_stream(n: int, seed: int):
    """A config-0-shaped stream of n records generated on the GPU: uniform
    random 128-B reads in the 1 GiB range at workloads.RANGE_BASE, issue gaps
    exponential with a mean of 2 ns (whole ps), seeded."""
    import torch
    from hbfsim_amd import workloads
    g = torch.Generator(device="cuda").manual_seed(seed)
    rec = torch.empty((n, 4), dtype=torch.int64, device="cuda")
    rec[:, 0] = torch.randint(0, (1 << 30) // 128, (n,), generator=g, device="cuda") * 128 + \
        workloads.RANGE_BASE
    rec[:, 1] = 128
    gaps = torch.empty(n, dtype=torch.float64, device="cuda").exponential_(1 / 2000.0, generator=g)
    rec[:, 2] = torch.cumsum(gaps.round_().to(torch.int64), 0)
    rec[:, 3] = 0
    del gaps
    torch.cuda.synchronize()
    return rec


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def committed_traffic(summary: str, kernel: str, units: int) -> tuple[float | None, str | None]:
    """HBM bytes per launch of `kernel` for `units` records (or cells), from
    a committed counter summary under profiles/ (two rocprofv3 passes,
    FETCH_SIZE and WRITE_SIZE, each calibrated against a 2 GiB copy).
    Counters cannot be read from inside the timed run, so the figure is the
    measured bytes per unit of that profile scaled to this launch."""
    path = ROOT / "profiles" / summary
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        parts = line.split()
        if parts and parts[0] == kernel and not line.startswith("#"):
            return float(parts[-1]) * units, f"profiles/{summary}"
    return None, None


def build_workload(name: str, steps: int, batches: int = 6):
    """Returns (profile, ranges, list of per-step record arrays on the GPU,
    description, host sample) of config 2: `batches` distinct decode steps
    generated on the GPU (step k of the run uses batch k mod batches)."""
    import torch
    from hbfsim_amd import workloads

    if name == "c2":
        shape = workloads.QWEN3_30B_A3B
        sel = workloads.moe_selection(shape, batches)
        out = []
        for k in range(batches):
            seg = workloads.moe_segments(shape, sel[k])
            out.append(workloads.gpu_segment_records(seg, shape.lines_per_expert, shape.line,
                                                     shape.gap_ps, shape.issuers))
            log(f"generated step {k}: {out[-1].shape[0]} records")
        torch.cuda.synchronize()
        sample = out[0][: 1 << 25].cpu().numpy().view(np.uint64)
        desc = {"workload": "config2: Qwen3-30B-A3B MoE decode, 48 layers x 128 experts "
                            "(9,437,184 B bf16 each) on HBF, 32 tokens/step top-8 Zipf(1.1) "
                            "deduplicated, 128-B lines from 256 wavefronts every 64 ns",
                "records_per_step": int(np.mean([b.shape[0] for b in out])),
                "distinct_steps": batches, "profile": "c2.json (16 ch x 8 die x 4 plane)",
                "ranges": len(workloads.moe_ranges(shape))}
        return (workloads.PROFILES / "c2.json", workloads.moe_ranges(shape), out, desc, sample)

    raise SystemExit(f"unknown config {name}")


def cpu_baseline(profile, ranges, host_records: np.ndarray, budget_s: float,
                 **options) -> dict:
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_py

    prof = oracle_py.load_profile(profile)
    params = oracle_py.engine_params(prof, **options)
    orng, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])

    def timed(threads: int, seconds: float) -> tuple[float, int, float]:
        state = oracle_py.OracleState(params)
        done, base = 0, 0
        t0 = time.perf_counter()
        while True:
            _, _, rep, _ = oracle_py.run(params, orng, count, host_records, base, state,
                                         threads=threads)
            base = rep["makespan_ps"]
            done += len(host_records)
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
        return done / dt, done, dt

    value, done, dt = timed(1, budget_s)
    out = {"value": value, "unit": "accesses/s", "cores": 1, "kind": "port",
           "sample": f"{done} records: the first {len(host_records)} records of step 0, "
                     f"replayed {done // len(host_records)}x with carried state, "
                     f"single-threaded oracle ({dt:.1f} s)"}
    # the same sample on the host's cores (the oracle's OpenMP split: tiles
    # summarised in parallel, composed in order), at most the box's share of 16
    threads = max(1, min(16, os.cpu_count() or 1))
    if threads > 1:
        pv, pdone, pdt = timed(threads, budget_s / 2)
        out["parallel"] = {"value": pv, "unit": "accesses/s", "cores": threads,
                           "sample": f"{pdone} records, the same sample ({pdt:.1f} s)"}
    out["host"] = {"nproc": os.cpu_count(), "cpu": host_cpu()}
    return out


def host_cpu() -> str:
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def bench_c4(args) -> dict:
    """Config 4: the OLMoE trace (1e8 accesses) through the thermal-coupled
    run.  A step is one whole coupled run from the initial state: access
    counts, the 64x64x8 grid stepped every simulated microsecond with
    refresh and throttle decisions, admission, refresh merge, engine."""
    import torch
    from hbfsim_amd import engine, workloads as w

    shape = w.OLMOE
    seg = w.c4_segments(shape, 2)
    limit = getattr(args, "c4_records", None) or w.C4_ACCESSES
    rec = w.gpu_segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                shape.issuers)[: min(limit, w.C4_ACCESSES)]
    ranges = w.moe_ranges(shape)
    e = engine.Engine(str(w.PROFILES / "c4.json"))
    for base, length, perms in ranges:
        e.register(base, length, perms)
    th = engine.Thermal(**w.C4_GRID)
    cells = th.cells
    comp = torch.empty(rec.shape[0], dtype=torch.int64, device="cuda")
    temp = torch.empty(cells, dtype=torch.float64, device="cuda")
    age0 = w.staggered_ages(64, w.C4_RELIABILITY["retention_ps"])
    stream = torch.cuda.current_stream()

    def step():
        e.reset()
        temp.fill_(w.C4_GRID["ambient_k"])
        age = age0.copy()
        return e.run_coupled(th, w.C4_RELIABILITY, rec, comp, temp, age, stream)

    log(f"c4: {rec.shape[0]} records, warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    phases = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rep, erep = step()
        for k, v in th.coupled_ms().items():
            phases[k] = phases.get(k, 0.0) + v / args.steps
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    windows = rep["windows"]
    per_window_ms = phases["thermal_chain"] / max(1, windows)
    # one window moves each cell's temperature in and out (8 + 8 B; the power
    # map comes from the per-die counts on chip): 16 B per cell per launch
    thermal_gbps = 16 * cells / (per_window_ms / 1e3) / 1e9
    n = int(rec.shape[0])
    engine_gbps = (RECORD_BYTES["32"] + 8) * (n + rep["refreshes"]) / (phases["engine"] / 1e3) / 1e9
    dominant = max(("thermal_chain", "engine"), key=lambda k: phases[k])
    traffic = committed_traffic("coupled_traffic_config4.txt", "k_thermal_window", cells)[0]
    roof = ({"bound": "latency (a chain of dependent one-window launches; priced against hbm)",
             "kernel": "k_thermal_window", "achieved": thermal_gbps,
             "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": thermal_gbps / PEAK_HBM_GBPS,
             "traffic": traffic, "traffic_source": "profiles/coupled_traffic_config4.txt",
             "algorithmic": f"16 B per cell per window (temperature read and written) x {cells} "
                            f"cells per launch, one launch per window",
             "kernel_ms": per_window_ms,
             "from_profile": roofline_from_profile("coupled_kernels_config4.txt",
                                                   "k_thermal_window", 16 * cells)}
            if dominant == "thermal_chain" else
            {"bound": "hbm", "kernel": "engine (k_summary + k_carry + k_apply)",
             "achieved": engine_gbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
             "frac": engine_gbps / PEAK_HBM_GBPS, "traffic": None})
    roof["phases_ms"] = phases
    out = {
        "metric": "modeled HBF accesses/sec on 1 MI355X",
        "value": rep["demand_modeled"] * args.steps / dt,
        "unit": "accesses/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": dt / args.steps * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u64+f64", "data": "synthetic",
        "config": {"workload": "config4: OLMoE-shaped decode trace (16 layers x 64 experts, "
                               "top-8 of 32 tokens, Zipf(1.1) seed 3) truncated at 1e8 "
                               "accesses, thermal-coupled: 64x64x8 EQ3 grid stepped every "
                               "1 us, Arrhenius-derated refresh, hysteresis throttling",
                   "records_per_step": n, "profile": "c4.json (8 ch x 8 die x 2 plane)",
                   "windows": windows, "refreshes": rep["refreshes"],
                   "level_windows": rep["level_windows"], "deferred": rep["deferred"],
                   "peak_k": rep["peak_k"], "makespan_ps": rep["makespan_ps"]},
        "roofline": roof,
    }
    if not args.no_cpu:
        log("cpu baseline (coupled oracle)")
        out["cpu_baseline"] = cpu_baseline_c4(rec, ranges, args.cpu_seconds)
    th.close()
    e.close()
    return out


def cpu_baseline_c4(rec, ranges, budget_s: float) -> dict:
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_py
    from hbfsim_amd import workloads as w

    prof = oracle_py.load_profile(w.PROFILES / "c4.json")
    params = oracle_py.engine_params(prof)
    orng, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
    rel = oracle_py.reliability(w.C4_GRID, w.C4_RELIABILITY, params.dies)
    sample = rec[: 1_000_000].cpu().numpy().view(np.uint64)
    oracle_py.lib().orc_set_threads(1)  # single-threaded, as `cores` states
    done, t0 = 0, time.perf_counter()
    while True:
        temp = np.full(64 * 64 * 8, w.C4_GRID["ambient_k"])
        age = w.staggered_ages(64, w.C4_RELIABILITY["retention_ps"])
        oracle_py.coupled_run(params, orng, count, rel, sample, temp, age)
        done += len(sample)
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "accesses/s", "cores": 1, "kind": "port",
            "sample": f"the first {len(sample)} records of the config-4 trace (250 windows of "
                      f"the 64x64x8 grid), coupled run from the initial state, repeated "
                      f"{done // len(sample)}x, single-threaded oracle ({dt:.1f} s)"}


def bench_thermal(args) -> dict:
    """The EQ3 stencil alone on a large grid (2048 x 2048 x 8 cells, 4 sweeps
    per step, constant power): cell-sweeps per second."""
    import torch
    from hbfsim_amd import engine, workloads as w

    g = dict(w.C4_GRID, nx=2048, ny=2048)
    th = engine.Thermal(**g)
    cells = th.cells
    gen = torch.Generator(device="cuda").manual_seed(7)
    power = torch.rand(cells, dtype=torch.float64, device="cuda", generator=gen) * 0.01
    temp = torch.full((cells,), g["ambient_k"], dtype=torch.float64, device="cuda")
    steps_per_call = 10
    th.step(power, temp, steps_per_call * max(1, args.warmup))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    kms = 0.0
    for _ in range(args.steps):
        th.step(power, temp, steps_per_call)
        kms += th.last_ms() / args.steps
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # a launch of the marching kernel makes two steps (same power) when the
    # sweeps allow; the profile's launches are these passes
    per_launch = steps_per_call / th.last_launches()
    launch_ms = kms * per_launch
    sweeps = cells * g["sweeps"]
    value = sweeps * steps_per_call * args.steps / dt
    # HBM bytes one launch must move, however many steps it fuses: T and P
    # read once, T written once (24 B per cell); the sweeps and the fused
    # steps stay on chip
    achieved = 24 * cells / (launch_ms / 1e3) / 1e9
    # FP64: per cell and sweep six neighbour products and their sums, the
    # ambient and right-hand-side terms and the scaling by 1 / den
    flops = THERMAL_FLOPS_PER_CELL_SWEEP * sweeps * per_launch
    tflops = flops / (launch_ms / 1e3) / 1e12
    traffic = committed_traffic("thermal_traffic_grid2048.txt", "k_thermal_march", cells)[0]
    out = {
        "metric": "EQ3 thermal grid cell-sweeps/sec on 1 MI355X", "value": value,
        "unit": "cell-sweeps/s", "n_gpus": 1, "steps": args.steps * steps_per_call,
        "warmup": args.warmup * steps_per_call, "ms_per_step": dt / args.steps / steps_per_call * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": "EQ3 grid 2048 x 2048 x 8 cells, 4 Jacobi sweeps per backward-"
                               "Euler step, config-4 conductances, random power"},
        "roofline": {"bound": "lds (LDS-staged sweeps; below both the HBM and the FP64 peak)",
                     "kernel": "k_thermal_march",
                     "algorithmic": f"24 B per cell per launch (T and P read once, T written "
                                    f"once; {per_launch:g} steps of {g['sweeps']} sweeps fused "
                                    f"on chip) x {cells} cells",
                     "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS,
                     "traffic": traffic, "traffic_source": "profiles/thermal_traffic_grid2048.txt",
                     "traffic_gbps": traffic / (launch_ms / 1e3) / 1e9 if traffic else None,
                     "traffic_frac": traffic / (launch_ms / 1e3) / 1e9 / PEAK_HBM_GBPS
                     if traffic else None,
                     "fp64": {"flops_per_cell_sweep": THERMAL_FLOPS_PER_CELL_SWEEP,
                              "achieved_tflops": tflops, "peak_tflops": PEAK_FP64_TFLOPS,
                              "frac": tflops / PEAK_FP64_TFLOPS},
                     "kernel_ms": launch_ms, "steps_per_launch": per_launch, "step_ms": kms,
                     "from_profile": roofline_from_profile("thermal_kernel_grid2048.txt",
                                                           "k_thermal_march", 24 * cells)},
    }
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT / "tests"))
        import oracle_py
        L = oracle_py.lib()
        nx, ny, nz = 256, 256, 8
        p = np.random.default_rng(7).uniform(0, 0.01, nx * ny * nz)
        t = np.full(nx * ny * nz, g["ambient_k"])
        done, c0 = 0, time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds:
            L.orc_thermal_grid_step(nx, ny, nz, g["capacity_j_per_k"], g["gx_w_per_k"],
                                    g["gy_w_per_k"], g["gz_w_per_k"], g["top_g_w_per_k"],
                                    g["ambient_k"], g["dt_s"], p.ctypes.data, t.ctypes.data,
                                    -1.0, 4)
            done += nx * ny * nz * 4
        out["cpu_baseline"] = {"value": done / (time.perf_counter() - c0),
                               "unit": "cell-sweeps/s", "cores": 1, "kind": "port",
                               "sample": "256 x 256 x 8 grid, 4 sweeps per step, "
                                         "single-threaded oracle"}
    th.close()
    return out


def sub_line(engine, profile, ranges, batches, records, args, what: str, mode="fast",
             apply_rereads: bool = False, kernels_summary: str | None = None,
             traffic_summary: str | None = None) -> dict:
    """One more workload timed like the main line (same step count), with
    its own roofline for the dominant per-record kernel, the same roofline
    recomputed from the committed kernel summary it cites, and the HBM
    traffic of that summary's counter companion."""
    value, dt, kms, streamed, apply_waves = time_steps(engine, profile, ranges, batches, records,
                                                       args, mode)
    names = ["k_summary", "k_carry", "k_apply"]
    kb = kernel_bytes(records, apply_rereads)
    dominant = 0 if kms[0] >= kms[2] else 2
    per_launch = streamed / args.steps
    achieved = kb[names[dominant]] * per_launch / (kms[dominant] / 1e3) / 1e9
    algo = RECORD_BYTES[records] + 8
    roof = {"bound": "hbm", "kernel": names[dominant],
            "algorithmic": f"{kb[names[dominant]]} B per access x {int(per_launch)} accesses "
                           f"per launch",
            "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBPS,
            "kernel_ms": {nm: float(v) for nm, v in zip(names, kms)},
            "apply_bytes_per_access": kb["k_apply"],
            "apply_waves_per_simd": apply_waves,
            "algorithmic_bytes_per_access": algo,
            "pipeline_frac": value * algo / 1e9 / PEAK_HBM_GBPS}
    if kernels_summary is not None:
        roof["from_profile"] = roofline_from_profile(kernels_summary, names[dominant],
                                                     kb[names[dominant]] * per_launch)
        if kms[dominant] < 0.1:
            roof["timing_note"] = ("a kernel of tens of microseconds: the HIP-event interval "
                                   "around it holds its dispatch too (2.5-5 us more than the "
                                   "kernel trace's duration on config 0)")
    if traffic_summary is not None:
        traffic, src = committed_traffic(traffic_summary, names[dominant], int(per_launch))
        roof["traffic"], roof["traffic_source"] = traffic, src
    return {"workload": what, "value": value, "unit": "accesses/s",
            "ms_per_step": dt / args.steps * 1e3,
            "records": "packed 16-byte records" if records == "packed" else "32-byte records",
            "roofline": roof}


def config_workload(name: str, batches: int = 2):
    """Configs 0, 1 and 3 as the engine times them (packed records on the
    GPU): (profile, ranges, packed batches, description, host sample of the
    first step for the CPU baseline, whether the apply pass re-reads records).
    Config 0: the 2^20-record stream (random: every step replayed from its
    records).  Config 1: TinyLlama-1.1B decode steps (17.2M records each).
    Config 3: full-size paged-KV decode steps (1.17e9 records each)."""
    import torch
    from hbfsim_amd import engine, workloads as w
    if name == "c0":
        s = w.config0()
        rec = torch.from_numpy(s.records.view(np.int64)).cuda()
        desc = {"workload": "config0: 2^20 uniform 128-B reads in one 1 GiB range, Poisson "
                            "issue gaps of mean 2 ns, seed 0; the same stream each step",
                "records_per_step": len(s.records), "profile": "c0.json (8 ch x 4 die x 2 plane)"}
        return (s.profile, s.ranges, [engine.pack_records(rec)], desc, s.records, True)
    if name == "c1":
        shape = w.TINYLLAMA
        spans = w.dense_spans(shape)
        rec = w.gpu_span_records(*spans, shape.line, shape.gap_ps, shape.issuers)
        sample = rec[: 1 << 22].cpu().numpy().view(np.uint64)
        desc = {"workload": "config1: TinyLlama-1.1B decode, 22 layers, every matrix and norm "
                            "read in 128-B lines by 256 wavefronts; the same step each time",
                "records_per_step": int(rec.shape[0]), "profile": "c0.json",
                "ranges": len(w.dense_ranges(shape))}
        out = [engine.pack_records(rec)]
        del rec
        torch.cuda.empty_cache()
        return (w.PROFILES / "c0.json", w.dense_ranges(shape), out, desc, sample, False)
    if name == "c3":
        shape = w.PAGED_KV
        tables = shape.tables()
        out, sample, n = [], None, 0
        for step in range(batches):
            spans = w.kv_spans(shape, step, tables)
            rec = w.gpu_span_records(*spans, shape.line, shape.gap_ps, shape.issuers)
            if sample is None:
                sample = rec[: 1 << 22].cpu().numpy().view(np.uint64)
            n = int(rec.shape[0])
            out.append(engine.pack_records(rec))
            del rec
            torch.cuda.empty_cache()
            log(f"config 3 step {step}: {n} records")
        desc = {"workload": "config3: paged KV cache on HBF, 32 layers x 8 KV heads x 128 dim "
                            "bf16, 16-token pages, 64 sequences of 1,024-32,768 tokens (seed 2); "
                            "each step reads every page and appends one token per sequence and "
                            "layer (page-fill programs at tPROG 200 us)",
                "records_per_step": n, "distinct_steps": batches, "profile": "c3.json",
                "ranges": len(w.kv_ranges(shape))}
        return (w.PROFILES / "c3.json", w.kv_ranges(shape), out, desc, sample, False)
    raise SystemExit(f"unknown config {name}")


def bench_config(engine_mod, name: str, args, cpu_seconds: float) -> dict:
    """A config line: whole steps of config 0, 1 or 3 with the dominant
    kernel's roofline (and the same recomputed from the committed summary it
    cites) and the CPU oracle on a bounded sample of the same stream."""
    import torch
    profile, ranges, batches, desc, sample, rereads = config_workload(name)
    line = sub_line(engine_mod, profile, ranges, batches, "packed", args, desc["workload"],
                    apply_rereads=rereads,
                    kernels_summary=f"engine_kernels_config{name[1:]}_packed.txt",
                    traffic_summary=f"engine_traffic_config{name[1:]}_packed.txt")
    line["config"] = desc
    del batches
    torch.cuda.empty_cache()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(profile, ranges, sample, cpu_seconds)
        line["cpu_baseline"]["speedup"] = {
            "vs_1_core": line["value"] / line["cpu_baseline"]["value"],
            "vs_all_cores": line["value"] / line["cpu_baseline"]["parallel"]["value"]
            if line["cpu_baseline"].get("parallel") else None}
    return line


def bench_general(engine, args) -> dict:
    """The general per-record path at scale: 2^28 config-0-shaped random
    records (no linear steps: every record decodes, groups and folds on its
    own), packed, on the config-0 profile."""
    from hbfsim_amd import workloads
    n = 1 << 28
    batches, sample = [], None
    for k in range(2):
        b = gpu_random_stream(n, 11 + k)
        if k == 0:
            sample = b[: 1 << 22].cpu().numpy().view(np.uint64)
        batches.append(engine.pack_records(b))
        del b
    profile = workloads.PROFILES / "c0.json"
    ranges = [(workloads.RANGE_BASE, 1 << 30, 3)]
    line = sub_line(engine, profile, ranges, batches, "packed", args,
                    "config0-shaped random stream: 2^28 uniform 128-B reads in 1 GiB, exponential "
                    "gaps mean 2 ns, 8 ch x 4 die x 2 plane, 2 distinct batches",
                    apply_rereads=True, kernels_summary="engine_kernels_general.txt",
                    traffic_summary="engine_traffic_general.txt")
    del batches
    if not getattr(args, "no_cpu", True):
        line["cpu_baseline"] = sub_cpu_baseline(line, profile, ranges, sample, args)
    return line


def sub_cpu_baseline(line: dict, profile, ranges, sample: np.ndarray, args, **options) -> dict:
    """The CPU oracle on a bounded sample of a sub-line's stream (a few
    seconds), with the line's speedup over it."""
    cb = cpu_baseline(profile, ranges, sample, min(3.0, args.cpu_seconds / 2), **options)
    cb["speedup"] = {"vs_1_core": line["value"] / cb["value"],
                     "vs_all_cores": line["value"] / cb["parallel"]["value"]
                     if cb.get("parallel") else None}
    return cb


def bench_hybrid(engine, batches, args, packed=None) -> dict:
    """Config 2 in hybrid mode (context mode 2): every modeled record passes
    the reference sampler (rate 1%, 1,000 warm-up requests); the apply pass
    folds linear steps and samples each of their records (the range id the
    sampler's key needs is kept beside each step descriptor).  Packed records
    (packed before the timed region)."""
    import tempfile
    from hbfsim_amd import workloads
    prof = json.loads((workloads.PROFILES / "c2.json").read_text())
    prof.update(reference_sample_rate=0.01, reference_warmup_requests=1000)
    path = pathlib.Path(tempfile.mkdtemp(prefix="hbf-bench-")) / "c2-hybrid.json"
    path.write_text(json.dumps(prof))
    shape = workloads.QWEN3_30B_A3B
    if packed is None:
        packed = [engine.pack_records(b) for b in batches]
    line = sub_line(engine, path, workloads.moe_ranges(shape), packed, "packed", args,
                    "config2 with hybrid sampling (rate 0.01, warm-up 1,000), packed records",
                    mode="hybrid", kernels_summary="engine_kernels_config2_hybrid.txt")
    if not getattr(args, "no_cpu", True):
        sample = batches[0][: 1 << 22].cpu().numpy().view(np.uint64)
        line["cpu_baseline"] = sub_cpu_baseline(line, path, workloads.moe_ranges(shape), sample,
                                                args, hybrid=True)
    return line


def link_workload(links: int, per_link: int, seed: int = 5):
    """Synthetic UCIe traffic: per link, `per_link` reads, each an AR request
    (exponential gaps, mean 3 ns) and its R return 300 ns later, merged in
    ready order.  Returns host arrays (first, ready_ns, direction)."""
    rng = np.random.default_rng(seed)
    gaps = rng.exponential(3.0, (links, per_link)).astype(np.uint64) + 1
    ar = np.cumsum(gaps, axis=1, dtype=np.uint64)
    ready = np.concatenate([ar, ar + 300], axis=1)
    direction = np.concatenate([np.zeros_like(ar, np.uint8), np.ones_like(ar, np.uint8)], axis=1)
    order = np.argsort(ready, axis=1, kind="stable")
    ready = np.take_along_axis(ready, order, axis=1).reshape(-1)
    direction = np.take_along_axis(direction, order, axis=1).reshape(-1)
    first = np.arange(links + 1, dtype=np.uint64) * np.uint64(2 * per_link)
    return first, ready, direction


def bench_link(args, links: int = 1 << 17, per_link: int = 256) -> dict:
    """The UCIe Streaming / AoU link stage (hbfsim_amd_link_run): `links`
    independent links, each carrying `per_link` reads through the reference
    LinkProfile defaults; one step is one run of every link to quiescence.
    The kernel runs one link per lane, an event loop whose steps depend on
    each other, so it is bound by load latency rather than HBM bandwidth;
    the roofline prices its algorithmic bytes (ready 8 + direction 1 in,
    delivery 8 out = 17 B per message) against HBM all the same."""
    import torch
    from hbfsim_amd import _native as nat
    from hbfsim_amd import link as lk
    first, ready, direction = link_workload(links, per_link)
    n = len(ready)
    t_first = torch.from_numpy(first.view(np.int64)).cuda()
    t_ready = torch.from_numpy(ready.view(np.int64)).cuda()
    t_dir = torch.from_numpy(direction).cuda()
    prof = lk.link_profile()
    stream = torch.cuda.current_stream()
    # outputs allocated once, outside the timed calls (each call synchronises
    # its stream; nothing is copied to the host inside the timed region)
    delivered = torch.zeros(n, dtype=torch.int64, device="cuda")
    counters = torch.zeros((links, 2, len(nat.LINK_COUNTER_FIELDS)), dtype=torch.int64,
                           device="cuda")
    for _ in range(max(1, args.warmup)):
        lk.run_into(prof, t_first, t_ready, t_dir, delivered, counters, stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        lk.run_into(prof, t_first, t_ready, t_dir, delivered, counters, stream)
    e1.record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    achieved = 17 * n / (ms / 1e3) / 1e9
    # the same bytes over the committed kernel trace's two kernels per call
    us = [profile_kernel_us("link_kernels.txt", k) for k in ("k_link", "k_link_split")]
    from_profile = None
    if None not in us:
        gbps = 17 * n / (sum(us) / 1e6) / 1e9
        from_profile = {"source": "profiles/link_kernels.txt", "kernel_avg_us": sum(us),
                        "achieved": gbps, "frac": gbps / PEAK_HBM_GBPS}
    counters = counters.cpu().numpy().view(np.uint64)
    # two lanes per link, 64-lane waves; the small LDS form (4 admitted
    # messages and 4 flit slots per direction, 6 KiB per wave) leaves room
    # for 7 waves per SIMD (71 VGPRs), so all of them are resident at once
    simds = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    waves = (2 * links + 63) // 64
    out = {"workload": f"{links} links x {per_link} reads (AR + R each, AR gaps exp mean 3 ns, "
                       f"R 300 ns later), reference LinkProfile defaults (16 GT/s, AR 12 / R 56 "
                       f"granule credits, 4 accepted per direction)",
           "value": n * args.steps / dt, "unit": "messages/s", "ms_per_step": dt / args.steps * 1e3,
           "occupancy": {"waves": waves, "simds": simds, "waves_per_simd": waves / simds,
                         "kernel_form": "k_link<4, 4> (LDS rings, 6 KiB per wave)",
                         "resident_waves_per_simd_max": 7},
           "roofline": {"bound": "latency (dependent event loop per link direction; priced "
                                 "against hbm)", "kernel": "k_link (with k_link_split)",
                        "algorithmic": f"17 B per message x {n} messages per launch",
                        "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                        "frac": achieved / PEAK_HBM_GBPS, "call_ms": ms,
                        "messages_per_s_per_call": n / (ms / 1e3),
                        "from_profile": from_profile},
           "flits": int(counters[:, :, 0].sum())}
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT / "tests"))
        import oracle_py
        op = oracle_py.link_profile(gt=16, ar=12, r=56, max_accepted=4)
        budget = min(5.0, args.cpu_seconds)
        done, k, c0 = 0, 0, time.perf_counter()
        while time.perf_counter() - c0 < budget and k < links:
            b, e = int(first[k]), int(first[k + 1])
            got, _ = oracle_py.link_scenario(op, direction[b:e], ready[b:e])
            if k < 64:
                assert np.array_equal(got, delivered[b:e].cpu().numpy().view(np.uint64)), k
            done += e - b
            k += 1
        cdt = time.perf_counter() - c0
        out["cpu_baseline"] = {"value": done / cdt, "unit": "messages/s", "cores": 1,
                               "kind": "port",
                               "sample": f"the first {k} links of the same workload through the "
                                         f"oracle's StreamingLink restatement ({cdt:.1f} s); the "
                                         f"first 64 checked equal to the GPU's deliveries"}
    return out


def scalar_floor(budget_s: float) -> dict:
    """The reference's own per-access fast model (the single-tail recurrence
    of hbf_device.cu:895-910, oracle orc_fast_model_scalar) on config 0's
    2^20 records, single-threaded: the like-for-like CPU floor."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_py
    from hbfsim_amd import workloads
    s = workloads.config0()
    arrival = np.ascontiguousarray(s.records[:, 2] // 1000, np.uint64)
    op = np.zeros(len(arrival), np.uint32)
    nbytes = np.full(len(arrival), 16384, np.uint32)
    target = np.zeros(len(arrival), np.uint64)
    prof = oracle_py.load_profile(workloads.PROFILES / "c0.json")
    L = oracle_py.lib()
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        tail = np.zeros(1, np.uint64)
        L.orc_fast_model_scalar(arrival.ctypes.data, op.ctypes.data, nbytes.ctypes.data,
                                len(arrival), prof["read_latency_ns"], prof["program_latency_ns"],
                                prof["aggregate_bandwidth_bytes_per_s"], tail.ctypes.data,
                                target.ctypes.data)
        done += len(arrival)
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "accesses/s", "cores": 1, "kind": "port",
            "sample": f"config 0 (2^20 records, whole-page 16 KiB transfers) through the "
                      f"single-tail fast model, repeated {done // len(arrival)}x ({dt:.1f} s)"}


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this engine runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from hbfsim_amd import engine

    if args.copy_probe:
        copy_probe()
    if args.config == "link":
        print(json.dumps(bench_link(args)), flush=True)
        return
    if args.config in ("c4", "thermal"):
        out = bench_c4(args) if args.config == "c4" else bench_thermal(args)
        print(json.dumps(out), flush=True)
        return
    if args.config in ("general", "hybrid"):
        if args.config == "general":
            line = bench_general(engine, args)
        else:
            # the same decode steps as the default run's hybrid sub-line
            nb = args.batches or max(1, min(args.steps + args.warmup, 12))
            batches = build_workload("c2", args.steps, nb)[2]
            line = bench_hybrid(engine, batches, args)
        out = {"metric": "modeled HBF accesses/sec on 1 MI355X", "value": line["value"],
               "unit": "accesses/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": line["ms_per_step"], "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "u64", "data": "synthetic",
               "config": {"workload": line["workload"], "records": line["records"]},
               "roofline": line["roofline"]}
        if "cpu_baseline" in line:
            out["cpu_baseline"] = line["cpu_baseline"]
        print(json.dumps(out), flush=True)
        return
    if args.config in ("c0", "c1", "c3"):
        line = bench_config(engine, args.config, args, args.cpu_seconds)
        out = {"metric": "modeled HBF accesses/sec on 1 MI355X", "value": line["value"],
               "unit": "accesses/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": line["ms_per_step"], "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "u64", "data": "synthetic",
               "config": dict(line["config"], records=line["records"]),
               "roofline": line["roofline"]}
        if "cpu_baseline" in line:
            out["cpu_baseline"] = line["cpu_baseline"]
        print(json.dumps(out), flush=True)
        return

    if args.batches is None:
        args.batches = max(1, min(args.steps + args.warmup, 12))
    profile, ranges, batches, desc, host_records = build_workload(args.config, args.steps,
                                                                  args.batches)
    records = args.records
    timed = batches
    if records == "packed":
        try:
            timed = [engine.pack_records(b) for b in batches]
        except ValueError as err:
            log(f"{err}: timing 32-byte records")
            records = "32"
    desc = dict(desc, records=("packed 16-byte records (hbf_record16)" if records == "packed"
                               else "32-byte records (hbf_record32)"))
    value, dt, avg_ms, accesses, _ = time_steps(engine, profile, ranges, timed, records, args)
    other = None
    if records == "packed" and not args.no_compare:
        # the same steps from 32-byte records, for comparison (its own roofline)
        v32, dt32, ms32, _, _ = time_steps(engine, profile, ranges, batches, "32", args)
        other = {"records": "32-byte records (hbf_record32)", "value": v32,
                 "ms_per_step": dt32 / args.steps * 1e3, "algorithmic_bytes_per_access": 40,
                 "pipeline_frac": v32 * 40 / 1e9 / PEAK_HBM_GBPS,
                 "kernel_ms": {nm: float(v) for nm, v in
                               zip(["k_summary", "k_carry", "k_apply"], ms32)}}
    algo = RECORD_BYTES[records] + 8
    kb = kernel_bytes(records)
    names = ["k_summary", "k_carry", "k_apply"]
    # the dominant per-record kernel (the carry chain works per tile and resource)
    dominant = 0 if avg_ms[0] >= avg_ms[2] else 2
    per_launch = accesses / args.steps
    achieved = kb[names[dominant]] * per_launch / (avg_ms[dominant] / 1e3) / 1e9
    summary = ("engine_traffic_config2_packed.txt" if records == "packed"
               else "engine_traffic_config2.txt")
    kernels_summary = ("engine_kernels_config2_packed.txt" if records == "packed"
                       else "engine_kernels_config2.txt")
    traffic, traffic_src = committed_traffic(summary, names[dominant], int(per_launch))
    out = {
        "metric": "modeled HBF accesses/sec on 1 MI355X",
        "value": value,
        "unit": "accesses/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": desc,
        "roofline": {"bound": "hbm", "kernel": names[dominant],
                     "algorithmic": f"{kb[names[dominant]]} B per access x "
                                    f"{int(per_launch)} accesses per launch",
                     "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel_ms": {nm: float(v) for nm, v in zip(names, avg_ms)},
                     "algorithmic_bytes_per_access": algo,
                     "pipeline_frac": value * algo / 1e9 / PEAK_HBM_GBPS,
                     "from_profile": roofline_from_profile(
                         kernels_summary, names[dominant], kb[names[dominant]] * per_launch)},
    }
    if other is not None:
        out["records32"] = other
    if args.config == "c2" and not args.no_extra:
        log("read / write ceilings")
        probe = engine.probe_bandwidth()
        out["stream_probe"] = probe
        # k_summary only reads (its records), k_apply only writes (completions):
        # each against the ceiling of its own access pattern
        out["roofline"]["measured_read_gbps"] = probe["read_gbps"]
        out["roofline"]["frac_of_measured_read"] = (
            kb["k_summary"] * per_launch / (avg_ms[0] / 1e3) / 1e9 / probe["read_gbps"])
        out["roofline"]["measured_write_gbps"] = probe["write_gbps"]
        out["roofline"]["k_apply_frac_of_measured_write"] = (
            kb["k_apply"] * per_launch / (avg_ms[2] / 1e3) / 1e9 / probe["write_gbps"])
        log("general path: random stream")
        out["general"] = bench_general(engine, args)
        log("hybrid mode")
        out["hybrid"] = bench_hybrid(engine, batches, args,
                                     packed=timed if records == "packed" else None)
        log("ucie link")
        out["link"] = bench_link(args)
    if not args.no_cpu:
        log("cpu baseline")
        cb = cpu_baseline(profile, ranges, host_records, args.cpu_seconds)
        cb["scalar_fast_model"] = scalar_floor(min(3.0, args.cpu_seconds))
        # the speedup over the CPU oracle, on the host's single core and on its cores together
        cb["speedup"] = {"vs_1_core": value / cb["value"],
                         "vs_all_cores": value / cb["parallel"]["value"]
                         if cb.get("parallel") else None}
        out["cpu_baseline"] = cb
    if args.config == "c2" and not args.no_extra:
        del batches, timed
        import torch
        torch.cuda.empty_cache()
        log("config 4")
        c4 = bench_c4(argparse.Namespace(steps=2, warmup=1, no_cpu=args.no_cpu,
                                         cpu_seconds=args.cpu_seconds / 2))
        out["config4"] = {k: c4[k] for k in ("value", "unit", "ms_per_step", "steps", "warmup",
                                              "dtype", "config", "roofline", "cpu_baseline")
                          if k in c4}
        log("eq3 stencil, 2048 x 2048 x 8")
        th = bench_thermal(argparse.Namespace(steps=3, warmup=1, no_cpu=args.no_cpu,
                                              cpu_seconds=min(3.0, args.cpu_seconds)))
        out["thermal"] = {k: th[k] for k in ("metric", "value", "unit", "ms_per_step", "steps",
                                             "warmup", "dtype", "config", "roofline",
                                             "cpu_baseline") if k in th}
        # configs 0, 1 and 3 at their own sizes, each with its own roofline and
        # CPU baseline
        for name in ("c0", "c1", "c3"):
            log(f"config {name[1:]}")
            out[f"config{name[1:]}"] = bench_config(
                engine, name, argparse.Namespace(steps=args.steps, warmup=args.warmup,
                                                 no_cpu=args.no_cpu),
                min(3.0, args.cpu_seconds / 2))
            torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)


def time_steps(engine, profile, ranges, batches, records, args, mode="fast"):
    """Warm-up steps, then exactly `args.steps` timed steps of one engine
    (bracketed by device synchronisation); returns (modeled accesses/s,
    seconds, average per-kernel ms, records streamed, waves per SIMD of the
    last step's apply kernel)."""
    import torch
    e = engine.Engine(str(profile), mode=mode)
    for base, length, perms in ranges:
        e.register(base, length, perms)
    run = e.run_packed if records == "packed" else e.run
    n = max(int(b.shape[0]) for b in batches)
    comp = torch.empty(n, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    base_ps = 0
    log(f"warmup {args.warmup} steps of {n} records ({records})")
    for k in range(args.warmup):
        rep = run(batches[k % len(batches)], comp, None, base_ps, stream)
        base_ps = rep["makespan_ps"]
    torch.cuda.synchronize()
    kernel_ms = np.zeros(3)
    records_seen, modeled = 0, 0
    log(f"timing {args.steps} steps ({records})")
    t0 = time.perf_counter()
    for k in range(args.steps):
        rep = run(batches[k % len(batches)], comp, None, base_ps, stream)
        base_ps = rep["makespan_ps"]
        records_seen += rep["records"]
        modeled += rep["modeled"]
        kernel_ms += np.array(e.kernel_ms()[:3])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # the apply kernel's form in the last timed step (waves per SIMD it was built for)
    apply_waves = e.apply_waves()
    e.close()
    # the metric counts modeled accesses; the kernels stream every record
    return modeled / dt, dt, kernel_ms / args.steps, records_seen, apply_waves


if __name__ == "__main__":
    main()
