"""Test-side ctypes binding of the CPU oracle (oracle/liboracle.so).

Test infrastructure only: the oracle is the checker the HIP engine is
compared against, never part of the product path.
"""
from __future__ import annotations

import ctypes
import json
import math
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
LIB = ORACLE_DIR / "liboracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libhbfref.so"

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64


class OrcRange(ctypes.Structure):
    _fields_ = [("base", _U64), ("length", _U64), ("file_offset", _U64), ("range_id", _U32),
                ("mode", _U32), ("permissions", _U32), ("cache_policy", _U32),
                ("stream_id", _U32), ("flags", _U32), ("page_bytes", _U64),
                ("reserved1", _U64)]


class OrcMedia(ctypes.Structure):
    _fields_ = [("logical_address", _U64), ("bytes", _U32), ("valid", _U32)]


class OrcEmpirical(ctypes.Structure):
    _fields_ = [("flags", _U32), ("point_count", _U32), ("pages", _U32 * 6),
                ("cumulative_ns", _U64 * 6), ("program_latency_ns", _U64)]


class OrcParams(ctypes.Structure):
    _fields_ = [("model", _U32), ("channels", _U32), ("ways", _U32), ("dies", _U32),
                ("planes", _U32), ("order", _U32 * 4), ("page_shift", _U32),
                ("page_buffers", _U32), ("plane_contention", _U32), ("transfer_page", _U32),
                ("program_every_write", _U32), ("hybrid", _U32), ("hybrid_warmup", _U32),
                ("hybrid_threshold", _U64), ("read_ps", _U64), ("program_ps", _U64),
                ("xfer_num", _U64), ("xfer_den", _U64), ("xfer_quantum", _U64),
                ("empirical", OrcEmpirical), ("media_pages", _U64), ("media_records", _U32),
                ("warp_grouping", _U32)]


class OrcState(ctypes.Structure):
    _fields_ = [("plane_busy", _P), ("plane_tag", _P), ("channel_cursor", _P),
                ("plane_busy_total", _P), ("channel_busy_total", _P), ("burst_state", _U64),
                ("modeled_sequence", _U64)]


REPORT_FIELDS = ("records", "modeled", "bypass", "unsupported", "reads", "writes", "page_hits",
                 "programs", "hybrid_sampled", "makespan_ps", "latency_sum_lo",
                 "latency_sum_hi", "latency_max_ps", "service_sum_ps", "grouped")


class OrcReport(ctypes.Structure):
    _fields_ = [(name, _U64) for name in REPORT_FIELDS]

    def as_dict(self) -> dict:
        d = {name: int(getattr(self, name)) for name in REPORT_FIELDS}
        d["latency_sum_ps"] = d["latency_sum_lo"] | (d["latency_sum_hi"] << 64)
        return d


class OrcTraceEvent(ctypes.Structure):
    _fields_ = [("logical_address", _U64), ("bytes", _U64), ("page_bytes", _U32),
                ("operation", _U32)]


_D = ctypes.c_double


class OrcReliability(ctypes.Structure):
    _fields_ = [("nx", _U32), ("ny", _U32), ("nz", _U32), ("sweeps", _U32), ("capacity", _D),
                ("gx", _D), ("gy", _D), ("gz", _D), ("gb", _D), ("ambient_k", _D), ("dt_s", _D),
                ("window_ps", _U64), ("regions_x", _U32), ("regions_y", _U32), ("dies", _U32),
                ("policy", _U32), ("static_w", _D), ("access_energy_j", _D),
                ("refresh_energy_j", _D), ("activation_ev", _D), ("reference_k", _D),
                ("retention_ps", _U64), ("light_k", _D), ("severe_k", _D), ("shutdown_k", _D),
                ("hysteresis_k", _D), ("action_delay_ps", _U64), ("min_dwell_ps", _U64),
                ("light_gap_ps", _U64)]


class OrcControl(ctypes.Structure):
    _fields_ = [("applied", _U32), ("pending", _U32), ("pending_at_ps", _U64),
                ("last_change_ps", _U64)]


NO_PENDING = 4


class OrcCoupledReport(ctypes.Structure):
    _fields_ = [("windows", _U64), ("refreshes", _U64), ("deferred", _U64),
                ("level_windows", _U64 * 4), ("demand_modeled", _U64), ("latency_sum_lo", _U64),
                ("latency_sum_hi", _U64), ("latency_max_ps", _U64), ("makespan_ps", _U64),
                ("peak_k", _D)]

    def as_dict(self) -> dict:
        d = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            d[name] = [int(x) for x in v] if name == "level_windows" else (
                float(v) if name == "peak_k" else int(v))
        d["latency_sum_ps"] = d["latency_sum_lo"] | (d["latency_sum_hi"] << 64)
        return d


AF_BINS = 4096

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        sig = {
            "orc_fast_hash": (_U64, [_U64]),
            "orc_hybrid_reference_sample": (ctypes.c_int, [_U64, _U32, _U64, _U64]),
            "orc_sample_threshold": (_U64, [ctypes.c_double]),
            "orc_fast_transfer_ns": (_U64, [_U32, _U64]),
            "orc_fast_service_ns": (_U64, [_U64, _U32, _U64]),
            "orc_saturating_add": (_U64, [_U64, _U64]),
            "orc_saturating_multiply": (_U64, [_U64, _U32]),
            "orc_find_range_index": (_U32, [_P, _U32, _U64]),
            "orc_access_supported": (ctypes.c_int, [_P, _U64, _U32, _U32]),
            "orc_range_overlaps": (ctypes.c_int, [_P, _U64, _U32]),
            "orc_span_touches_any_range": (ctypes.c_int, [_P, _U32, _U64, _U32]),
            "orc_media_descriptor": (OrcMedia, [_P, _U64, _U32, _U32]),
            "orc_classify": (_U32, [_P, _U32, _U64, _U64, _U32, _P]),
            "orc_ceiling_scaled_delta": (_U64, [_U64, _U32, _U32]),
            "orc_empirical_cumulative_ns": (_U64, [_P, _P, _U32, _U32]),
            "orc_empirical_service_ns": (_U64, [_P, _P, _U32, _U32]),
            "orc_update_empirical_burst": (ctypes.c_int, [_U64, _U64, _U32, _P, _P]),
            "orc_empirical_control_valid": (ctypes.c_int, [_P]),
            "orc_empirical_request_service": (ctypes.c_int, [_P, _U64, _U64, _U32, _P, _P, _P]),
            "orc_range_table_create": (_P, [_U64, _U64]),
            "orc_range_table_destroy": (None, [_P]),
            "orc_range_table_add": (ctypes.c_int, [_P, _U64, _U64, _U32, _U32, _U32, _U32]),
            "orc_range_table_remove": (ctypes.c_int, [_P, _U64]),
            "orc_range_table_lookup": (ctypes.c_int, [_P, _U64, _U32, _P]),
            "orc_stripe": (_U64, [_U64, _P, _P, _P]),
            "orc_parse_scheme": (ctypes.c_int, [ctypes.c_char_p, _P]),
            "orc_hbf_media_lpa": (_U64, [_U64, _U32, _U32]),
            "orc_hbf_cold_read_bank": (None, [_U64, _U32, _U32, _U32, _P, _P, _P, _P]),
            "orc_engine_run": (ctypes.c_int, [_P, _P, _U32, _P, ctypes.c_size_t, _U64, _P, _P,
                                              _P, _P]),
            "orc_engine_run_parallel": (ctypes.c_int, [_P, _P, _U32, _P, ctypes.c_size_t, _U64,
                                                       _P, _P, _P, _P, ctypes.c_int]),
            "orc_fast_model_scalar": (_U64, [_P, _P, _P, ctypes.c_size_t, _U64, _U64, _U64, _P,
                                             _P]),
            "orc_trace_timing_fast": (ctypes.c_int, [_P, ctypes.c_size_t, _U64, _U64, _U64, _U64,
                                                     _U64, _P, _P, _P]),
            "orc_bandwidth_cursor": (_U64, [_P, _U64, _U64, _U64, _U64]),
            "orc_pagebuf_sequence": (None, [_P, ctypes.c_size_t, _U32, _P]),
            "orc_media_servers": (None, [_P, ctypes.c_size_t, _U32, _U64, _P]),
            "orc_mqsim_admission": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t, _U32, _U64,
                                                   _P, _P, _P]),
            "orc_engine_admission": (ctypes.c_int, [_P, _P, _U32, _P, _P, ctypes.c_size_t, _P,
                                                    _P, _U32, _U64, _P, _P, _P, _P]),
            "orc_simulate_prefetch": (ctypes.c_int, [_P, ctypes.c_size_t, _U32, _U32, _U32,
                                                     _U32, _U64, _U64, _P]),
            "orc_sampler_run": (ctypes.c_int, [_U32, ctypes.c_double, _U64, _P, _P,
                                               ctypes.c_size_t, _P]),
            "orc_calibrate": (ctypes.c_long, [_P, _P, ctypes.c_size_t, _P]),
            "orc_thermal_dense_step": (ctypes.c_int, [ctypes.c_size_t, _P, _P, _P, _P,
                                                      ctypes.c_size_t, _P, _P, _P,
                                                      ctypes.c_double, _P, _P]),
            "orc_thermal_grid_step": (ctypes.c_int, [_U32, _U32, _U32, ctypes.c_double,
                                                     ctypes.c_double, ctypes.c_double,
                                                     ctypes.c_double, ctypes.c_double,
                                                     ctypes.c_double, ctypes.c_double, _P, _P,
                                                     ctypes.c_double, ctypes.c_int]),
            "orc_arrhenius": (ctypes.c_double, [ctypes.c_double, ctypes.c_double,
                                                ctypes.c_double]),
            "orc_retention_table": (None, [_D, _D, _U64, _P]),
            "orc_retention_bin": (_U32, [_D]),
            "orc_control_step": (_U32, [_P, _P, _U64, _D]),
            "orc_reliability_chain": (ctypes.c_int, [_P, _P, _U64, _P, _P, _P, _P, _P, _P]),
            "orc_defer": (_U64, [_P, _U64, _U64, _U64, _U32]),
            "orc_admit": (None, [_P, _U64, _U64, _U64, _P, ctypes.c_size_t, _P]),
            "orc_refresh_records": (ctypes.c_size_t, [_P, _P, _P, _U64, _U64, _P, _P]),
            "orc_merge_records": (None, [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, _P]),
            "orc_window_counts": (ctypes.c_int, [_P, _P, _U32, _P, ctypes.c_size_t, _U64, _U64,
                                                 _P]),
            "orc_set_threads": (None, [ctypes.c_int]),
            "orc_get_threads": (ctypes.c_int, []),
            "orc_coupled_run": (ctypes.c_int, [_P, _P, _U32, _P, _P, ctypes.c_size_t, _P, _P, _P,
                                               _P, _P, _P, _P, _P, _U64]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ref_available() -> bool:
    """Whether the compiled reference shim was built here.  Checks the file
    only, so collecting tests never loads the shim."""
    return REF_LIB.exists()


def ref_lib() -> ctypes.CDLL | None:
    """The compiled reference shim, when it was built in this container."""
    if not ref_available():
        return None
    return ctypes.CDLL(str(REF_LIB))


def addr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------------------
# hybrid sampler and calibrator (calibrator.cpp:67-138)

CALIBRATION_DTYPE = np.dtype([("operation", "<u4"), ("bytes", "<u4"), ("queue_bucket", "<u4"),
                              ("locality_bucket", "<u4"), ("count", "<u8"), ("mean_ns", "<u8"),
                              ("p50_ns", "<u8"), ("p95_ns", "<u8"), ("p99_ns", "<u8"),
                              ("log_mean", "<f8"), ("log_sigma", "<f8")])


def mqsim_admission(arrival, nbytes, latency, queue_depth: int, bandwidth: int):
    """orc_mqsim_admission: (admission, media completion, bounded completion)
    per request, in ns."""
    arrival = np.ascontiguousarray(arrival, np.uint64)
    nbytes = np.ascontiguousarray(nbytes, np.uint64)
    latency = np.ascontiguousarray(np.broadcast_to(np.asarray(latency, np.uint64),
                                                   arrival.shape))
    n = len(arrival)
    out = [np.zeros(max(n, 1), np.uint64) for _ in range(3)]
    rc = lib().orc_mqsim_admission(addr(arrival), addr(nbytes), addr(latency), n, queue_depth,
                                   bandwidth, addr(out[0]), addr(out[1]), addr(out[2]))
    if rc != 0:
        raise ValueError("bandwidth 0 or too many requests")
    return tuple(o[:n] for o in out)


def engine_admission(params: OrcParams, ranges, count: int, records: np.ndarray,
                     first: np.ndarray, arrival_ns, nbytes, queue_depth: int, bandwidth: int,
                     state: "OracleState | None" = None):
    """orc_engine_admission: the adapter's admission and cursor with the engine
    as the media port.  records: every request's pages (32-byte records),
    request k = records[first[k]:first[k + 1]].  Returns (admission, device
    completion, bounded completion) per request, in ns."""
    rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
    first = np.ascontiguousarray(first, np.uint64)
    arrival = np.ascontiguousarray(arrival_ns, np.uint64)
    nbytes = np.ascontiguousarray(nbytes, np.uint64)
    n = len(arrival)
    if state is None:
        state = OracleState(params)
    out = [np.zeros(max(n, 1), np.uint64) for _ in range(3)]
    rc = lib().orc_engine_admission(ctypes.byref(params), ranges, count, addr(rec), addr(first),
                                    n, addr(arrival), addr(nbytes), queue_depth, bandwidth,
                                    ctypes.byref(state.s), addr(out[0]), addr(out[1]),
                                    addr(out[2]))
    if rc != 0:
        raise RuntimeError(f"oracle admission failed: {rc}")
    return tuple(o[:n] for o in out)


def sampler_run(warmup, rate, seed, access, sequence) -> np.ndarray:
    """flags[i] = HybridSampler(warmup, rate, seed).reference(sequence[i],
    access[i]) in order; access is (n, 4) u32.  ValueError for a bad rate."""
    access = np.ascontiguousarray(access, np.uint32).reshape(-1, 4)
    sequence = np.ascontiguousarray(sequence, np.uint64)
    flags = np.zeros(len(access), np.uint8)
    rc = lib().orc_sampler_run(warmup, rate, seed, addr(access), addr(sequence), len(access),
                               addr(flags))
    if rc == 1:
        raise ValueError("sample_rate must be in [0, 1]")
    assert rc == 0
    return flags


def calibrate(access, latency) -> np.ndarray:
    """Calibrator estimates of every observed class, in class order."""
    access = np.ascontiguousarray(access, np.uint32).reshape(-1, 4)
    latency = np.ascontiguousarray(latency, np.uint64)
    rows = np.zeros(max(len(access), 1), CALIBRATION_DTYPE)
    n = lib().orc_calibrate(addr(access), addr(latency), len(access), addr(rows))
    if n < 0:
        raise ValueError("latency_ns must be positive")
    return rows[:n]


# ---------------------------------------------------------------------------
# engine parameters, derived independently of the product's C++ code


def load_profile(path) -> dict:
    return json.loads(pathlib.Path(path).read_text())


def engine_params(profile: dict, page_buffers=1, plane_contention=1, transfer_page=0,
                  program_every_write=0, flat_geometry=0, ways=1, xfer_quantum_ps=1,
                  channel_bandwidth_bytes_per_s=0, hybrid=False, model=0,
                  warp_grouping=0) -> OrcParams:
    p = OrcParams()
    p.model = model
    p.warp_grouping = warp_grouping
    if flat_geometry:
        p.channels = p.ways = p.dies = p.planes = 1
    else:
        p.channels = profile["channels"]
        p.ways = ways
        p.dies = profile["dies_per_channel"]
        p.planes = profile["planes_per_die"]
    scheme = profile.get("plane_allocation_scheme", "CWDP")
    axis = {"C": 0, "W": 1, "D": 2, "P": 3}
    for i, ch in enumerate(scheme):
        p.order[i] = axis[ch]
    p.page_shift = int(math.log2(profile["page_bytes"]))
    p.page_buffers = page_buffers
    p.plane_contention = plane_contention
    p.transfer_page = transfer_page
    p.program_every_write = program_every_write
    p.hybrid = 1 if hybrid else 0
    p.hybrid_warmup = profile["reference_warmup_requests"]
    p.hybrid_threshold = lib().orc_sample_threshold(profile["reference_sample_rate"])
    p.read_ps = profile["read_latency_ns"] * 1000
    p.program_ps = profile["program_latency_ns"] * 1000
    q = xfer_quantum_ps or 1
    if channel_bandwidth_bytes_per_s:
        num, den = 10**12, channel_bandwidth_bytes_per_s * q
    else:
        num, den = 10**12 * p.channels, profile["aggregate_bandwidth_bytes_per_s"] * q
    g = math.gcd(num, den)
    p.xfer_num, p.xfer_den, p.xfer_quantum = num // g, den // g, q
    p.media_pages = profile["capacity_bytes"] // profile["page_bytes"]
    if "empirical_vmem" in profile:
        e = profile["empirical_vmem"]
        p.empirical.flags = 1
        p.empirical.point_count = 6
        for i, pt in enumerate(e["read_curve"]):
            p.empirical.pages[i] = pt["pages"]
            p.empirical.cumulative_ns[i] = pt["cumulative_ns"]
        p.empirical.program_latency_ns = profile["program_latency_ns"]
    return p


class OracleState:
    def __init__(self, params: OrcParams):
        planes = params.channels * params.ways * params.dies * params.planes
        self.plane_busy = np.zeros(planes, np.uint64)
        self.plane_tag = np.zeros(planes * 2, np.uint64)
        self.channel_cursor = np.zeros(params.channels, np.uint64)
        self.plane_busy_total = np.zeros(planes, np.uint64)
        self.channel_busy_total = np.zeros(params.channels, np.uint64)
        self.s = OrcState(addr(self.plane_busy), addr(self.plane_tag),
                          addr(self.channel_cursor), addr(self.plane_busy_total),
                          addr(self.channel_busy_total), 0, 0)


def range_table(ranges, page_bytes: int, capacity: int) -> list[OrcRange]:
    """Registers (base, length, permissions) in order through the oracle's
    restatement of RangeTable::add; returns the sorted records."""
    L = lib()
    t = L.orc_range_table_create(page_bytes, capacity)
    try:
        for base, length, perms in ranges:
            rc = L.orc_range_table_add(t, base, length, 1, perms, 0, 0)
            if rc != 0:
                raise ValueError(f"oracle range add failed: {rc}")
        class _T(ctypes.Structure):
            _fields_ = [("records", ctypes.POINTER(OrcRange)), ("count", _U32),
                        ("next_range_id", _U32), ("next_file_offset", _U64),
                        ("page_bytes", _U64), ("media_capacity", _U64)]
        tt = ctypes.cast(t, ctypes.POINTER(_T)).contents
        out = (OrcRange * max(1, tt.count))()
        ctypes.memmove(out, tt.records, ctypes.sizeof(OrcRange) * tt.count)
        return out, tt.count
    finally:
        L.orc_range_table_destroy(t)


def run(params: OrcParams, ranges, count: int, records: np.ndarray, base_ps: int = 0,
        state: OracleState | None = None, threads: int = 1):
    rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
    n = rec.shape[0]
    if state is None:
        state = OracleState(params)
    comp = np.zeros(n, np.uint64)
    st = np.zeros(n, np.uint8)
    rep = OrcReport()
    if threads > 1:
        rc = lib().orc_engine_run_parallel(ctypes.byref(params), ranges, count, addr(rec), n,
                                           base_ps, ctypes.byref(state.s), addr(comp), addr(st),
                                           ctypes.byref(rep), threads)
    else:
        rc = lib().orc_engine_run(ctypes.byref(params), ranges, count, addr(rec), n, base_ps,
                                  ctypes.byref(state.s), addr(comp), addr(st),
                                  ctypes.byref(rep))
    if rc != 0:
        raise RuntimeError(f"oracle engine failed: {rc}")
    return comp, st, rep.as_dict(), state


# ---------------------------------------------------------------------------
# thermal-coupled reliability


def reliability(grid: dict, options: dict, dies: int) -> OrcReliability:
    """orc_reliability from the keyword sets the product API takes (grid:
    nx, ny, nz, sweeps, capacity_j_per_k, g*_w_per_k, top_g_w_per_k,
    ambient_k, dt_s; options: the hbfsim_amd_reliability_options fields)."""
    r = OrcReliability()
    r.nx, r.ny, r.nz = grid["nx"], grid["ny"], grid["nz"]
    r.sweeps = grid.get("sweeps", 4)
    r.capacity = grid["capacity_j_per_k"]
    r.gx, r.gy, r.gz = grid["gx_w_per_k"], grid["gy_w_per_k"], grid["gz_w_per_k"]
    r.gb, r.ambient_k, r.dt_s = grid["top_g_w_per_k"], grid["ambient_k"], grid["dt_s"]
    r.window_ps = options["window_ps"]
    r.regions_x, r.regions_y, r.dies = options["regions_x"], options["regions_y"], dies
    r.policy = options.get("policy", 1)
    r.static_w = options.get("static_power_w", 0.0)
    r.access_energy_j = options.get("access_energy_j", 0.0)
    r.refresh_energy_j = options.get("refresh_energy_j", 0.0)
    r.activation_ev = options.get("activation_energy_ev", 0.0)
    r.reference_k = options.get("reference_k", 358.15)
    r.retention_ps = options.get("retention_ps", 0)
    r.light_k, r.severe_k = options.get("light_k", 0.0), options.get("severe_k", 0.0)
    r.shutdown_k, r.hysteresis_k = options.get("shutdown_k", 0.0), options.get("hysteresis_k", 0.0)
    r.action_delay_ps = options.get("action_delay_ps", 0)
    r.min_dwell_ps = options.get("min_dwell_ps", 0)
    r.light_gap_ps = options.get("light_gap_ps", 0)
    return r


def coupled_run(params: OrcParams, ranges, count: int, rel: OrcReliability,
                records: np.ndarray, temperature: np.ndarray, age: np.ndarray,
                state: OracleState | None = None):
    """orc_coupled_run; temperature and age are updated in place.  Returns
    (completion, report, trace dict, state)."""
    rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
    n = rec.shape[0]
    if state is None:
        state = OracleState(params)
    windows = int(rec[:, 2].max()) // rel.window_ps + 1 if n else 0
    dies = params.channels * params.ways * params.dies
    comp = np.zeros(max(n, 1), np.uint64)
    hot = np.zeros((windows + 1) * dies, np.float64)
    level = np.zeros(max(windows, 1), np.uint8)
    refresh = np.zeros(max(windows * dies, 1), np.uint8)
    rep = OrcCoupledReport()
    assert temperature.dtype == np.float64 and age.dtype == np.uint64
    rc = lib().orc_coupled_run(ctypes.byref(params), ranges, count, ctypes.byref(rel), addr(rec),
                               n, addr(temperature), addr(age), ctypes.byref(state.s),
                               addr(comp), ctypes.byref(rep), addr(hot), addr(level),
                               addr(refresh), windows)
    if rc != 0:
        raise RuntimeError(f"oracle coupled run failed: {rc}")
    trace = {"windows": windows, "dies": dies, "hot": hot.reshape(windows + 1, dies),
             "level": level[:windows], "refresh": refresh[: windows * dies].reshape(windows, dies)}
    return comp[:n], rep.as_dict(), trace, state


# ---------------------------------------------------------------------------
# UCIe Streaming / AoU link (oracle/ucie_link.c)


class OrcLinkProfile(ctypes.Structure):
    _fields_ = [("gt_per_second", _U32), ("initial_ar_granules", _U32),
                ("initial_r_granules", _U32), ("max_accepted", _U32), ("propagation_ns", _U64)]


LINK_COUNTER_FIELDS = ("flits", "wire_bytes", "ucie_header_bytes", "crc_position_bytes",
                       "aou_header_bytes", "aou_message_bytes", "unused_message_bytes",
                       "credit_only_flits", "accounting_saturated")


class OrcLinkCounters(ctypes.Structure):
    _fields_ = [(f, _U64) for f in LINK_COUNTER_FIELDS]

    def as_dict(self) -> dict:
        return {f: int(getattr(self, f)) for f in LINK_COUNTER_FIELDS}


class OrcLinkFragment(ctypes.Structure):
    _fields_ = [("request_id", _U64), ("flit_granule", _U32), ("message_granule", _U32),
                ("granules", _U32), ("msg_start", ctypes.c_uint8), ("msg_end", ctypes.c_uint8),
                ("pad", ctypes.c_uint8 * 2)]


class OrcLinkFlit(ctypes.Structure):
    _fields_ = [("direction", _U32), ("nfrag", _U32), ("start_ns", _U64),
                ("delivered_ns", _U64), ("message_granules", _U32), ("grant_granules", _U32),
                ("credit_only", _U32), ("pad", _U32), ("frag", OrcLinkFragment * 48)]


class OrcLinkDelivery(ctypes.Structure):
    _fields_ = [("direction", _U32), ("pad", _U32), ("request_id", _U64),
                ("delivered_ns", _U64)]


REQUEST, RETURN = 0, 1


def _link_lib() -> ctypes.CDLL:
    L = lib()
    if not getattr(L, "_link_bound", False):
        sig = {
            "orc_link_profile_valid": (ctypes.c_int, [_P]),
            "orc_link_serialization_ns": (_U64, [_P]),
            "orc_link_legal_grant": (_U32, [_U32]),
            "orc_link_create": (_P, [_P]),
            "orc_link_destroy": (None, [_P]),
            "orc_link_enqueue": (ctypes.c_int, [_P, _U32, _U64, _U64]),
            "orc_link_consume": (ctypes.c_int, [_P, _U32, _U64, _U64]),
            "orc_link_next_event": (ctypes.c_int, [_P, _P]),
            "orc_link_step": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P]),
            "orc_link_now": (_U64, [_P]),
            "orc_link_credits": (_U32, [_P, _U32]),
            "orc_link_counters_of": (ctypes.POINTER(OrcLinkCounters), [_P, _U32]),
            "orc_link_flit_count": (ctypes.c_size_t, [_P]),
            "orc_link_flit_at": (ctypes.POINTER(OrcLinkFlit), [_P, ctypes.c_size_t]),
            "orc_link_scenario": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t, _P, _P, _P]),
            "orc_link_scenario_traced": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t, _P, _P, _P,
                                                        _P, ctypes.c_size_t, _P, _P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        L._link_bound = True
    return L


def link_profile(gt=16, ar=128, r=128, max_accepted=128, propagation_ns=0) -> OrcLinkProfile:
    return OrcLinkProfile(gt, ar, r, max_accepted, propagation_ns)


class LinkError(Exception):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: code {code}")
        self.code = code


class Link:
    """The oracle's StreamingLink (object API of src/ucie/link.cpp)."""

    def __init__(self, profile: OrcLinkProfile):
        self._L = _link_lib()
        self.profile = profile
        self.h = self._L.orc_link_create(ctypes.byref(profile))
        if not self.h:
            raise ValueError("invalid link profile")

    def close(self):
        if self.h:
            self._L.orc_link_destroy(self.h)
            self.h = None

    def enqueue(self, direction, request_id, ready_ns):
        rc = self._L.orc_link_enqueue(self.h, direction, request_id, ready_ns)
        if rc:
            raise LinkError(rc, "enqueue")

    def consume(self, direction, request_id, at):
        rc = self._L.orc_link_consume(self.h, direction, request_id, at)
        if rc:
            raise LinkError(rc, "consume")

    def next_event_ns(self):
        t = ctypes.c_uint64()
        return int(t.value) if self._L.orc_link_next_event(self.h, ctypes.byref(t)) else None

    def step(self):
        out = (OrcLinkDelivery * 64)()
        k = ctypes.c_size_t()
        rc = self._L.orc_link_step(self.h, out, 64, ctypes.byref(k))
        if rc:
            raise LinkError(rc, "step")
        return [(int(out[i].direction), int(out[i].request_id), int(out[i].delivered_ns))
                for i in range(k.value)]

    def now(self):
        return int(self._L.orc_link_now(self.h))

    def credits(self, direction):
        return int(self._L.orc_link_credits(self.h, direction))

    def counters(self, direction) -> dict:
        return self._L.orc_link_counters_of(self.h, direction).contents.as_dict()

    def flits(self) -> list:
        return [flit_dict(self._L.orc_link_flit_at(self.h, i).contents)
                for i in range(self._L.orc_link_flit_count(self.h))]


def flit_dict(f) -> dict:
    """An orc_link_flit as a dict (FlitRecord's fields, link.hpp:22-38)."""
    return {"direction": f.direction, "start_ns": f.start_ns,
            "delivered_ns": f.delivered_ns, "message_granules": f.message_granules,
            "grant_granules": f.grant_granules, "credit_only": bool(f.credit_only),
            "fragments": [dict(request_id=f.frag[k].request_id,
                               flit_granule=f.frag[k].flit_granule,
                               message_granule=f.frag[k].message_granule,
                               granules=f.frag[k].granules,
                               msg_start=bool(f.frag[k].msg_start),
                               msg_end=bool(f.frag[k].msg_end))
                          for k in range(f.nfrag)]}


def link_scenario(profile: OrcLinkProfile, direction, ready, delay=(0, 0)):
    """orc_link_scenario: one link's messages (direction, ready_ns) through
    the caller that admits in order and consumes each delivery delay[dir]
    later.  Returns (delivered_ns[n], [request counters, return counters])."""
    direction = np.ascontiguousarray(direction, np.uint32)
    ready = np.ascontiguousarray(ready, np.uint64)
    n = len(ready)
    delivered = np.zeros(max(n, 1), np.uint64)
    counters = (OrcLinkCounters * 2)()
    d = (_U64 * 2)(*delay)
    rc = _link_lib().orc_link_scenario(ctypes.byref(profile), addr(direction), addr(ready), n, d,
                                       addr(delivered), counters)
    if rc:
        raise LinkError(rc, "scenario")
    return delivered[:n], [counters[0].as_dict(), counters[1].as_dict()]


def link_scenario_traced(profile: OrcLinkProfile, direction, ready, delay=(0, 0), cap=4096):
    """link_scenario that also returns the link's flit records (the first
    4096, in emission order) and how many were not recorded."""
    direction = np.ascontiguousarray(direction, np.uint32)
    ready = np.ascontiguousarray(ready, np.uint64)
    n = len(ready)
    delivered = np.zeros(max(n, 1), np.uint64)
    counters = (OrcLinkCounters * 2)()
    flits = (OrcLinkFlit * cap)()
    nflits = ctypes.c_size_t(0)
    dropped = _U64(0)
    d = (_U64 * 2)(*delay)
    rc = _link_lib().orc_link_scenario_traced(ctypes.byref(profile), addr(direction), addr(ready),
                                              n, d, addr(delivered), counters, flits, cap,
                                              ctypes.byref(nflits), ctypes.byref(dropped))
    if rc:
        raise LinkError(rc, "scenario")
    return (delivered[:n], [counters[0].as_dict(), counters[1].as_dict()],
            [flit_dict(flits[i]) for i in range(nflits.value)], int(dropped.value))
