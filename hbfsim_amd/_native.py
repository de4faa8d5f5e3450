"""ctypes binding of libhbfsim_amd.so (the C ABI in include/hbfsim_amd.h).

The library is loaded from this package directory.  There is no fallback:
when it is missing, loading raises, because every timing result must come
from the HIP engine.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libhbfsim_amd.so"

HBFSIM_OK = 0
HBFSIM_INVALID_ARGUMENT = 1
HBFSIM_IO_ERROR = 2
HBFSIM_CUDA_ERROR = 3
HBFSIM_TIMEOUT = 4
HBFSIM_UNSUPPORTED = 5
HBFSIM_DAEMON_LOST = 6

HBFSIM_RANGE_MODE_TIMING = 1
HBFSIM_RANGE_MODE_CAPACITY = 2
HBFSIM_RANGE_READ = 1
HBFSIM_RANGE_WRITE = 2
HBFSIM_RANGE_READ_WRITE = 3
HBFSIM_MODEL_REFERENCE = 0
HBFSIM_MODEL_FAST = 1
HBFSIM_MODEL_HYBRID = 2

MODEL_HBF = 0
MODEL_EMPIRICAL = 1

STATUS_MODELED = 0
STATUS_BYPASS = 1
STATUS_UNSUPPORTED = 2
STATUS_PAGE_HIT = 4
STATUS_HYBRID = 8
STATUS_PROGRAMMED = 16


class Options(ctypes.Structure):
    _fields_ = [("profile_path", ctypes.c_char_p), ("report_dir", ctypes.c_char_p),
                ("mode", ctypes.c_uint32), ("ring_capacity", ctypes.c_uint32),
                ("request_timeout_ns", ctypes.c_uint64)]


class RangeOptions(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_uint32), ("permissions", ctypes.c_uint32),
                ("cache_policy", ctypes.c_uint32), ("stream_id", ctypes.c_uint32)]


class Stats(ctypes.Structure):
    _fields_ = [("requests_submitted", ctypes.c_uint64), ("requests_completed", ctypes.c_uint64),
                ("fast_requests", ctypes.c_uint64), ("reference_requests", ctypes.c_uint64),
                ("fast_modeled_ns", ctypes.c_uint64)]


class CapacityStats(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("version", ctypes.c_uint32),
                ("enabled", ctypes.c_uint32), ("reserved0", ctypes.c_uint32)] + [
                   (name, ctypes.c_uint64) for name in (
                       "page_bytes", "vmm_granularity", "pool_allocated_bytes",
                       "logical_frame_count", "service_resolve_calls", "service_resident_hits",
                       "service_reclaimed_hits", "service_misses",
                       "successful_backing_read_pages", "successful_backing_read_bytes",
                       "successful_h2d_fill_pages", "successful_h2d_fill_bytes",
                       "successful_resolve_evictions", "service_ready_results",
                       "successful_d2h_readback_pages", "successful_d2h_readback_bytes",
                       "successful_backing_write_pages", "successful_backing_write_bytes")]


class VllmOptions(ctypes.Structure):
    _fields_ = [("profile_path", ctypes.c_char_p), ("report_dir", ctypes.c_char_p),
                ("ring_capacity", ctypes.c_uint32), ("timing_model", ctypes.c_uint32),
                ("request_timeout_ns", ctypes.c_uint64)]


class EngineOptions(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("model", ctypes.c_uint32),
                ("page_buffers", ctypes.c_uint32), ("plane_contention", ctypes.c_uint32),
                ("transfer_page", ctypes.c_uint32), ("program_every_write", ctypes.c_uint32),
                ("flat_geometry", ctypes.c_uint32), ("ways", ctypes.c_uint32),
                ("xfer_quantum_ps", ctypes.c_uint64),
                ("channel_bandwidth_bytes_per_s", ctypes.c_uint64),
                ("tile_records", ctypes.c_uint32), ("warp_grouping", ctypes.c_uint32)]


class Range(ctypes.Structure):
    _fields_ = [("base", ctypes.c_uint64), ("length", ctypes.c_uint64),
                ("file_offset", ctypes.c_uint64), ("range_id", ctypes.c_uint32),
                ("mode", ctypes.c_uint32), ("permissions", ctypes.c_uint32),
                ("stream_id", ctypes.c_uint32), ("page_bytes", ctypes.c_uint64)]


REPORT_FIELDS = ("records", "modeled", "bypass", "unsupported", "reads", "writes", "page_hits",
                 "programs", "hybrid_sampled", "makespan_ps", "latency_sum_lo",
                 "latency_sum_hi", "latency_max_ps", "service_sum_ps", "grouped")


class Report(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in REPORT_FIELDS]

    def as_dict(self) -> dict:
        d = {name: int(getattr(self, name)) for name in REPORT_FIELDS}
        d["latency_sum_ps"] = d["latency_sum_lo"] | (d["latency_sum_hi"] << 64)
        return d


class ThermalGrid(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("nx", ctypes.c_uint32),
                ("ny", ctypes.c_uint32), ("nz", ctypes.c_uint32), ("sweeps", ctypes.c_uint32),
                ("reserved0", ctypes.c_uint32), ("capacity_j_per_k", ctypes.c_double),
                ("gx_w_per_k", ctypes.c_double), ("gy_w_per_k", ctypes.c_double),
                ("gz_w_per_k", ctypes.c_double), ("top_g_w_per_k", ctypes.c_double),
                ("ambient_k", ctypes.c_double), ("dt_s", ctypes.c_double)]


RELIABILITY_FIELDS = [("struct_size", ctypes.c_uint32), ("policy", ctypes.c_uint32),
                      ("regions_x", ctypes.c_uint32), ("regions_y", ctypes.c_uint32),
                      ("window_ps", ctypes.c_uint64), ("static_power_w", ctypes.c_double),
                      ("access_energy_j", ctypes.c_double), ("refresh_energy_j", ctypes.c_double),
                      ("activation_energy_ev", ctypes.c_double), ("reference_k", ctypes.c_double),
                      ("retention_ps", ctypes.c_uint64), ("light_k", ctypes.c_double),
                      ("severe_k", ctypes.c_double), ("shutdown_k", ctypes.c_double),
                      ("hysteresis_k", ctypes.c_double), ("action_delay_ps", ctypes.c_uint64),
                      ("min_dwell_ps", ctypes.c_uint64), ("light_gap_ps", ctypes.c_uint64)]


class ReliabilityOptions(ctypes.Structure):
    _fields_ = RELIABILITY_FIELDS


COUPLED_FIELDS = ("windows", "refreshes", "deferred", "level_windows", "demand_modeled",
                  "latency_sum_lo", "latency_sum_hi", "latency_max_ps", "makespan_ps", "peak_k")


class CoupledReport(ctypes.Structure):
    _fields_ = [("windows", ctypes.c_uint64), ("refreshes", ctypes.c_uint64),
                ("deferred", ctypes.c_uint64), ("level_windows", ctypes.c_uint64 * 4),
                ("demand_modeled", ctypes.c_uint64), ("latency_sum_lo", ctypes.c_uint64),
                ("latency_sum_hi", ctypes.c_uint64), ("latency_max_ps", ctypes.c_uint64),
                ("makespan_ps", ctypes.c_uint64), ("peak_k", ctypes.c_double)]

    def as_dict(self) -> dict:
        d = {}
        for name in COUPLED_FIELDS:
            v = getattr(self, name)
            d[name] = [int(x) for x in v] if name == "level_windows" else (
                float(v) if name == "peak_k" else int(v))
        d["latency_sum_ps"] = d["latency_sum_lo"] | (d["latency_sum_hi"] << 64)
        return d


class LinkProfile(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("gt_per_second", ctypes.c_uint32),
                ("initial_ar_granules", ctypes.c_uint32), ("initial_r_granules", ctypes.c_uint32),
                ("max_accepted", ctypes.c_uint32), ("reserved0", ctypes.c_uint32),
                ("propagation_ns", ctypes.c_uint64), ("consume_delay_ns", ctypes.c_uint64 * 2)]


LINK_COUNTER_FIELDS = ("flits", "wire_bytes", "ucie_header_bytes", "crc_position_bytes",
                       "aou_header_bytes", "aou_message_bytes", "unused_message_bytes",
                       "credit_only_flits", "accounting_saturated")

# hbfsim_amd_link_fragment / hbfsim_amd_link_flit as numpy record layouts
LINK_FRAGMENT_DTYPE = np.dtype([("request_id", np.uint64), ("flit_granule", np.uint32),
                                ("message_granule", np.uint32), ("granules", np.uint32),
                                ("msg_start", np.uint8), ("msg_end", np.uint8),
                                ("reserved", np.uint8, 2)])
LINK_FLIT_DTYPE = np.dtype([("start_ns", np.uint64), ("delivered_ns", np.uint64),
                            ("step", np.uint64),
                            ("direction", np.uint32), ("message_granules", np.uint32),
                            ("grant_granules", np.uint32), ("credit_only", np.uint32),
                            ("fragments", np.uint32), ("reserved", np.uint32),
                            ("fragment", LINK_FRAGMENT_DTYPE, 16)])


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_INT = ctypes.c_int

# name -> (restype, argtypes); one entry per function in include/hbfsim_amd.h
SIGNATURES = {
    "hbfsim_abi_version": (_U32, []),
    "hbfsim_context_create": (_INT, [ctypes.POINTER(Options), ctypes.POINTER(_P)]),
    "hbfsim_register_device": (_INT, [_P, _P, _SZ, ctypes.POINTER(RangeOptions)]),
    "hbfsim_map_file": (_INT, [_P, ctypes.c_char_p, _U64, _SZ, ctypes.POINTER(RangeOptions),
                               ctypes.POINTER(_P)]),
    "hbfsim_flush": (_INT, [_P]),
    "hbfsim_get_stats": (_INT, [_P, ctypes.POINTER(Stats)]),
    "hbfsim_get_capacity_stats_v1": (_INT, [_P, ctypes.POINTER(CapacityStats)]),
    "hbfsim_unregister": (_INT, [_P, _P]),
    "hbfsim_context_destroy": (None, [_P]),
    "hbfsim_vllm_abi_version": (_U32, []),
    "hbfsim_vllm_session_create": (_INT, [ctypes.POINTER(VllmOptions), ctypes.POINTER(_P)]),
    "hbfsim_vllm_register_storage": (_INT, [_P, _SZ, _SZ]),
    "hbfsim_vllm_session_close": (_INT, [ctypes.POINTER(_P)]),
    "hbfsim_vllm_status_string": (ctypes.c_char_p, [_INT]),
    "hbfsim_vllm_session_context": (_P, [_P]),
    "hbfsim_amd_default_engine_options": (_INT, [_P, ctypes.POINTER(EngineOptions)]),
    "hbfsim_amd_set_engine_options": (_INT, [_P, ctypes.POINTER(EngineOptions)]),
    "hbfsim_amd_get_engine_options": (_INT, [_P, ctypes.POINTER(EngineOptions)]),
    "hbfsim_amd_run_device": (_INT, [_P, _P, _SZ, _P, _P, _U64, _P, ctypes.POINTER(Report)]),
    "hbfsim_amd_run_device_packed": (_INT, [_P, _P, _SZ, _P, _P, _U64, _P,
                                            ctypes.POINTER(Report)]),
    "hbfsim_amd_run_device_packed_noalloc": (_INT, [_P, _P, _SZ, _P, _P, _U64, _P,
                                                    ctypes.POINTER(Report)]),
    "hbfsim_amd_run": (_INT, [_P, _P, _SZ, _P, _P, _U64, ctypes.POINTER(Report)]),
    "hbfsim_amd_get_report": (_INT, [_P, ctypes.POINTER(Report)]),
    "hbfsim_amd_get_geometry": (_INT, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32)]),
    "hbfsim_amd_get_busy_totals": (_INT, [_P, _P, _SZ, _P, _SZ]),
    "hbfsim_amd_get_state": (_INT, [_P, _P, _P, _P, _P, _P]),
    "hbfsim_amd_set_state": (_INT, [_P, _P, _P, _P, _U64, _U64]),
    "hbfsim_amd_reset": (_INT, [_P]),
    "hbfsim_amd_last_kernel_ms": (_INT, [_P, ctypes.POINTER(ctypes.c_float), _INT]),
    "hbfsim_amd_last_apply_waves": (_INT, [_P]),
    "hbfsim_amd_lookup_range": (_INT, [_P, _U64, _U32, ctypes.POINTER(_U32),
                                        ctypes.POINTER(Range), ctypes.POINTER(_U32)]),
    "hbfsim_amd_gen_segment_lines": (_INT, [_P, _SZ, _P, _SZ, _U64, _U32, _U64, _U32, _U64,
                                            _P]),
    "hbfsim_amd_media_servers": (_INT, [_P, _SZ, _U32, _U64, _P, _P]),
    "hbfsim_amd_gen_spans": (_INT, [_P, _SZ, _P, _P, _P, _SZ, _U64, _U32, _U64, _U32, _P]),
    "hbfsim_amd_sampler_create": (_INT, [_U32, ctypes.c_double, _U64, ctypes.POINTER(_P)]),
    "hbfsim_amd_sampler_destroy": (None, [_P]),
    "hbfsim_amd_sampler_reference": (_INT, [_P, _P, _P, _U64, _SZ, _P,
                                            ctypes.POINTER(_U64), _P]),
    "hbfsim_amd_calibrate": (_INT, [_P, _P, _SZ, _P, _SZ, ctypes.POINTER(_SZ), _P]),
    "hbfsim_amd_thermal_create": (_INT, [ctypes.POINTER(ThermalGrid), ctypes.POINTER(_P)]),
    "hbfsim_amd_thermal_step": (_INT, [_P, _P, _P, _U64, _P]),
    "hbfsim_amd_thermal_last_ms": (_INT, [_P, ctypes.POINTER(ctypes.c_float)]),
    "hbfsim_amd_thermal_last_launches": (_INT, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "hbfsim_amd_thermal_destroy": (None, [_P]),
    "hbfsim_amd_run_coupled": (_INT, [_P, _P, ctypes.POINTER(ReliabilityOptions), _P, _SZ, _P,
                                      _P, _P, _P, ctypes.POINTER(CoupledReport),
                                      ctypes.POINTER(Report)]),
    "hbfsim_amd_coupled_last_ms": (_INT, [_P, ctypes.POINTER(ctypes.c_float), _INT]),
    "hbfsim_amd_coupled_trace": (_INT, [_P, _P, _SZ, _P, _SZ, _P, _SZ, ctypes.POINTER(_U64),
                                        ctypes.POINTER(_U32)]),
    "hbfsim_amd_mqsim_admission": (_INT, [_P, _P, _SZ, _U32, _U64, _U64, _P, _P, _P]),
    "hbfsim_amd_link_run": (_INT, [ctypes.POINTER(LinkProfile), _P, _U32, _P, _P, _SZ, _P, _P,
                                   _P]),
    "hbfsim_amd_link_run_traced": (_INT, [ctypes.POINTER(LinkProfile), _P, _U32, _P, _P, _SZ, _P,
                                          _P, _P, _U32, _P]),
    "hbfsim_amd_validate_profile": (_INT, [ctypes.c_char_p, ctypes.c_char_p, _SZ]),
    "hbfsim_amd_probe_bandwidth": (_INT, [_P, _SZ, ctypes.c_uint, _P,
                                          ctypes.POINTER(ctypes.c_float),
                                          ctypes.POINTER(ctypes.c_float)]),
}

_lib = None


class NativeLibraryMissing(RuntimeError):
    """The HIP engine library is not built; there is no other implementation."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m hbfsim_amd.build` "
            "(or __graft_entry__.build()); the timing engine has no fallback")
    try:
        # PyTorch bundles a HIP runtime with the same soname; loading it first
        # keeps one runtime in the process, so tensor memory and engine
        # kernels share a device context.
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def status_name(code: int) -> str:
    value = load().hbfsim_vllm_status_string(code)
    return value.decode() if value else "unknown"


class HbfSimError(RuntimeError):
    def __init__(self, what: str, code: int):
        super().__init__(f"{what}: {status_name(code)} ({code})")
        self.code = code


def check(code: int, what: str) -> None:
    if code != HBFSIM_OK:
        raise HbfSimError(what, code)
