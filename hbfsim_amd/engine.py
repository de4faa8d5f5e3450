"""Python front end of the HIP timing engine.

`Engine` owns one hbfsim_context (include/hbfsim_amd.h) and drives it through
ctypes.  Records live in device memory owned by PyTorch (or in host numpy
arrays for `run_host`); the library only sees plain addresses.

Record layout (32 bytes): addr, bytes, issue_ps, flags (bits 0-7 operation:
0 read, 1 write).  As a tensor: int64 [n, 4] on the GPU, bit patterns
interpreted as unsigned.
"""
from __future__ import annotations

import ctypes
import os
import tempfile
from typing import Any

import numpy as np

from . import _native as nat

_MODES = {"reference": nat.HBFSIM_MODEL_REFERENCE, "fast": nat.HBFSIM_MODEL_FAST,
          "hybrid": nat.HBFSIM_MODEL_HYBRID}
OPTION_FIELDS = ("model", "page_buffers", "plane_contention", "transfer_page",
                 "program_every_write", "flat_geometry", "ways", "xfer_quantum_ps",
                 "channel_bandwidth_bytes_per_s", "tile_records", "warp_grouping")

# The reference's single-tail fast model (hbf_device.cu:883-958): one
# channel at the aggregate bandwidth moving whole pages in whole nanoseconds,
# latency not serialised, every write programs.
FAST_REFERENCE_OPTIONS = dict(page_buffers=0, plane_contention=0, transfer_page=1,
                              program_every_write=1, flat_geometry=1, xfer_quantum_ps=1000)


def _ptr(x: Any) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)!r}")


class Engine:
    """One timing context: profile, registered ranges, engine state."""

    def __init__(self, profile_path: str, report_dir: str | None = None, mode: str = "fast",
                 ring_capacity: int = 64, request_timeout_ns: int = 1_000_000_000,
                 **options: Any):
        self._lib = nat.load()
        if report_dir is None:
            report_dir = tempfile.mkdtemp(prefix="hbfsim-amd-")
        self.profile_path = str(profile_path)
        self.report_dir = str(report_dir)
        opts = nat.Options(self.profile_path.encode(), self.report_dir.encode(), _MODES[mode],
                           ring_capacity, request_timeout_ns)
        handle = ctypes.c_void_p()
        nat.check(self._lib.hbfsim_context_create(ctypes.byref(opts), ctypes.byref(handle)),
                  f"context create ({profile_path})")
        self._ctx = handle
        if options:
            self.set_options(**options)

    # -- lifecycle --------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_ctx", None) is not None and self._ctx.value:
            self._lib.hbfsim_context_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __enter__(self) -> "Engine":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._ctx

    # -- registration -----------------------------------------------------
    def register(self, base: int, length: int, permissions: int = nat.HBFSIM_RANGE_READ_WRITE,
                 stream_id: int = 0) -> None:
        o = nat.RangeOptions(nat.HBFSIM_RANGE_MODE_TIMING, permissions, 0, stream_id)
        nat.check(self._lib.hbfsim_register_device(self._ctx, ctypes.c_void_p(base), length,
                                                   ctypes.byref(o)),
                  f"register 0x{base:x}+{length}")

    def lookup(self, address: int, nbytes: int = 1) -> tuple[str, dict | None]:
        """RangeTable::lookup: ('outside'|'matched'|'crosses', range fields)."""
        kind = ctypes.c_uint32()
        r = nat.Range()
        nat.check(self._lib.hbfsim_amd_lookup_range(self._ctx, address, nbytes,
                                                    ctypes.byref(kind), ctypes.byref(r), None),
                  "lookup")
        names = ("outside", "matched", "crosses")
        if kind.value == 0:
            return names[0], None
        return names[kind.value], {k: int(getattr(r, k)) for k, _ in nat.Range._fields_}

    def unregister(self, base: int) -> None:
        nat.check(self._lib.hbfsim_unregister(self._ctx, ctypes.c_void_p(base)),
                  f"unregister 0x{base:x}")

    # -- configuration ----------------------------------------------------
    def options(self) -> dict:
        o = nat.EngineOptions()
        nat.check(self._lib.hbfsim_amd_get_engine_options(self._ctx, ctypes.byref(o)),
                  "get options")
        return {k: int(getattr(o, k)) for k in OPTION_FIELDS}

    def set_options(self, **kw: Any) -> None:
        current = self.options()
        unknown = set(kw) - set(OPTION_FIELDS)
        if unknown:
            raise ValueError(f"unknown engine options {sorted(unknown)}")
        current.update({k: int(v) for k, v in kw.items()})
        o = nat.EngineOptions(struct_size=ctypes.sizeof(nat.EngineOptions), **current)
        nat.check(self._lib.hbfsim_amd_set_engine_options(self._ctx, ctypes.byref(o)),
                  "set options")

    def geometry(self) -> tuple[int, int]:
        c, p = ctypes.c_uint32(), ctypes.c_uint32()
        nat.check(self._lib.hbfsim_amd_get_geometry(self._ctx, ctypes.byref(c), ctypes.byref(p)),
                  "geometry")
        return int(c.value), int(p.value)

    # -- running ----------------------------------------------------------
    def run(self, records: Any, completion: Any, status: Any = None, base_ps: int = 0,
            stream: Any = None) -> dict:
        """Times device-resident records (torch int64 [n, 4] on the GPU)."""
        n = int(records.shape[0]) if hasattr(records, "shape") else int(len(records))
        if stream is None:
            import torch
            stream = torch.cuda.current_stream().cuda_stream
        elif hasattr(stream, "cuda_stream"):
            stream = stream.cuda_stream
        rep = nat.Report()
        nat.check(self._lib.hbfsim_amd_run_device(
            self._ctx, _ptr(records), n, _ptr(completion), _ptr(status), base_ps,
            ctypes.c_void_p(stream), ctypes.byref(rep)), "run")
        return rep.as_dict()

    def run_packed(self, records: Any, completion: Any, status: Any = None, base_ps: int = 0,
                   stream: Any = None) -> dict:
        """Times device-resident packed records (torch int64 [n, 2] on the GPU,
        hbf_record16, see pack_records)."""
        n = int(records.shape[0])
        if stream is None:
            import torch
            stream = torch.cuda.current_stream().cuda_stream
        elif hasattr(stream, "cuda_stream"):
            stream = stream.cuda_stream
        rep = nat.Report()
        nat.check(self._lib.hbfsim_amd_run_device_packed(
            self._ctx, _ptr(records), n, _ptr(completion), _ptr(status), base_ps,
            ctypes.c_void_p(stream), ctypes.byref(rep)), "run (packed)")
        return rep.as_dict()

    def run_packed_noalloc(self, records: Any, completion: Any, status: Any = None,
                           base_ps: int = 0, stream: Any = None) -> dict:
        """run_packed through hbfsim_amd_run_device_packed_noalloc, which
        allocates nothing: its scratch is the library's static per-device
        array.  ValueError when the run does not fit that array, when the
        engine has not run yet or when ranges changed since its last run."""
        n = int(records.shape[0])
        if stream is None:
            import torch
            stream = torch.cuda.current_stream().cuda_stream
        elif hasattr(stream, "cuda_stream"):
            stream = stream.cuda_stream
        rep = nat.Report()
        rc = self._lib.hbfsim_amd_run_device_packed_noalloc(
            self._ctx, _ptr(records), n, _ptr(completion), _ptr(status), base_ps,
            ctypes.c_void_p(stream), ctypes.byref(rep))
        if rc == nat.HBFSIM_UNSUPPORTED:
            raise ValueError(f"{n} records do not fit the static scratch (64 MiB per device), or "
                             "the engine has not run yet, or ranges changed since its last run")
        nat.check(rc, "run (packed, no allocation)")
        return rep.as_dict()

    def run_host(self, records: np.ndarray, base_ps: int = 0,
                 want_status: bool = True) -> tuple[np.ndarray, np.ndarray | None, dict]:
        """Copies host records in, runs on the GPU, copies completions out."""
        rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
        n = rec.shape[0]
        comp = np.zeros(n, dtype=np.uint64)
        st = np.zeros(n, dtype=np.uint8) if want_status else None
        rep = nat.Report()
        nat.check(self._lib.hbfsim_amd_run(self._ctx, _ptr(rec), n, _ptr(comp), _ptr(st),
                                           base_ps, ctypes.byref(rep)), "run (host)")
        return comp, st, rep.as_dict()

    # -- results and state ------------------------------------------------
    def report(self) -> dict:
        rep = nat.Report()
        nat.check(self._lib.hbfsim_amd_get_report(self._ctx, ctypes.byref(rep)), "report")
        return rep.as_dict()

    def stats(self) -> dict:
        s = nat.Stats()
        nat.check(self._lib.hbfsim_get_stats(self._ctx, ctypes.byref(s)), "stats")
        return {k: int(getattr(s, k)) for k, _ in nat.Stats._fields_}

    def busy_totals(self) -> tuple[np.ndarray, np.ndarray]:
        channels, planes = self.geometry()
        p = np.zeros(planes, dtype=np.uint64)
        c = np.zeros(channels, dtype=np.uint64)
        nat.check(self._lib.hbfsim_amd_get_busy_totals(self._ctx, _ptr(p), planes, _ptr(c),
                                                       channels), "busy totals")
        return p, c

    def state(self) -> dict:
        channels, planes = self.geometry()
        busy = np.zeros(planes, dtype=np.uint64)
        tags = np.zeros(planes * 2, dtype=np.uint64)
        cur = np.zeros(channels, dtype=np.uint64)
        seq = ctypes.c_uint64()
        burst = ctypes.c_uint64()
        nat.check(self._lib.hbfsim_amd_get_state(self._ctx, _ptr(busy), _ptr(tags), _ptr(cur),
                                                 ctypes.addressof(seq), ctypes.addressof(burst)),
                  "get state")
        return {"plane_busy": busy, "plane_tags": tags, "channel_cursor": cur,
                "sequence": int(seq.value), "burst_state": int(burst.value)}

    def set_state(self, state: dict) -> None:
        busy = np.ascontiguousarray(state["plane_busy"], dtype=np.uint64)
        tags = np.ascontiguousarray(state["plane_tags"], dtype=np.uint64)
        cur = np.ascontiguousarray(state["channel_cursor"], dtype=np.uint64)
        nat.check(self._lib.hbfsim_amd_set_state(self._ctx, _ptr(busy), _ptr(tags), _ptr(cur),
                                                 int(state["sequence"]),
                                                 int(state["burst_state"])), "set state")

    def reset(self) -> None:
        nat.check(self._lib.hbfsim_amd_reset(self._ctx), "reset")

    def flush(self) -> None:
        nat.check(self._lib.hbfsim_flush(self._ctx), "flush")

    def kernel_ms(self) -> list[float]:
        ms = (ctypes.c_float * 8)()
        k = self._lib.hbfsim_amd_last_kernel_ms(self._ctx, ms, 8)
        return [float(ms[i]) for i in range(k)]

    def apply_waves(self) -> int:
        """Waves per SIMD the last run's apply kernel was built for (4: the
        form for large streams of general steps; results do not depend on it)."""
        return int(self._lib.hbfsim_amd_last_apply_waves(self._ctx))

    def run_coupled(self, thermal: "Thermal", options: dict, records: Any, completion: Any,
                    temperature: Any, age_ps: np.ndarray, stream: Any = None) -> tuple[dict, dict]:
        """Thermal-coupled run (hbfsim_amd_run_coupled): returns the coupled
        report and the engine report of the merged stream; `temperature`
        (device) and `age_ps` (host uint64, one per die) are updated."""
        n = int(records.shape[0])
        stream = _stream_handle(stream)
        opts = reliability_options(**options)
        rep, erep = nat.CoupledReport(), nat.Report()
        if age_ps.dtype != np.uint64 or not age_ps.flags.c_contiguous:
            raise ValueError("age_ps must be a contiguous uint64 array")
        nat.check(self._lib.hbfsim_amd_run_coupled(
            self._ctx, thermal.handle, ctypes.byref(opts), _ptr(records), n, _ptr(completion),
            _ptr(temperature), _ptr(age_ps), ctypes.c_void_p(stream), ctypes.byref(rep),
            ctypes.byref(erep)), "coupled run")
        return rep.as_dict(), erep.as_dict()


def _stream_handle(stream: Any) -> int:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if hasattr(stream, "cuda_stream"):
        return stream.cuda_stream
    return stream


def reliability_options(**kw: Any) -> nat.ReliabilityOptions:
    """hbfsim_amd_reliability_options from keyword arguments (field names of
    include/hbfsim_amd.h); unnamed fields are zero."""
    o = nat.ReliabilityOptions()
    o.struct_size = ctypes.sizeof(o)
    names = {f for f, _ in nat.RELIABILITY_FIELDS}
    for k, v in kw.items():
        if k not in names or k == "struct_size":
            raise KeyError(f"unknown reliability option {k!r}")
        setattr(o, k, v)
    return o


class Thermal:
    """The EQ3 grid (hbfsim_amd_thermal_*): backward-Euler steps on device
    temperature arrays (float64, nx*ny*nz, x fastest)."""

    def __init__(self, nx: int, ny: int, nz: int, capacity_j_per_k: float, gx_w_per_k: float,
                 gy_w_per_k: float, gz_w_per_k: float, top_g_w_per_k: float, ambient_k: float,
                 dt_s: float, sweeps: int = 4):
        self._lib = nat.load()
        g = nat.ThermalGrid()
        g.struct_size = ctypes.sizeof(g)
        g.nx, g.ny, g.nz, g.sweeps = nx, ny, nz, sweeps
        g.capacity_j_per_k, g.gx_w_per_k, g.gy_w_per_k = capacity_j_per_k, gx_w_per_k, gy_w_per_k
        g.gz_w_per_k, g.top_g_w_per_k, g.ambient_k, g.dt_s = (gz_w_per_k, top_g_w_per_k,
                                                               ambient_k, dt_s)
        self.grid = g
        h = ctypes.c_void_p()
        nat.check(self._lib.hbfsim_amd_thermal_create(ctypes.byref(g), ctypes.byref(h)),
                  "thermal create")
        self._h = h

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("thermal grid is closed")
        return self._h

    @property
    def cells(self) -> int:
        return self.grid.nx * self.grid.ny * self.grid.nz

    def step(self, power: Any, temperature: Any, steps: int = 1, stream: Any = None) -> None:
        nat.check(self._lib.hbfsim_amd_thermal_step(self.handle, _ptr(power), _ptr(temperature),
                                                    steps, ctypes.c_void_p(_stream_handle(stream))),
                  "thermal step")

    def last_ms(self) -> float:
        ms = ctypes.c_float()
        nat.check(self._lib.hbfsim_amd_thermal_last_ms(self.handle, ctypes.byref(ms)),
                  "thermal time")
        return float(ms.value)

    def last_launches(self) -> int:
        """Kernel passes of the last step() call (a fused pass makes two steps)."""
        n = ctypes.c_uint64()
        nat.check(self._lib.hbfsim_amd_thermal_last_launches(self.handle, ctypes.byref(n)),
                  "thermal launches")
        return int(n.value)

    def coupled_ms(self) -> dict:
        """Device time of the last coupled run's phases."""
        ms = (ctypes.c_float * 5)()
        k = self._lib.hbfsim_amd_coupled_last_ms(self.handle, ms, 5)
        names = ("counts", "thermal_chain", "admission", "engine", "gather")
        return {names[i]: float(ms[i]) for i in range(k)}

    def trace(self) -> dict:
        """Per-window trace of the last coupled run."""
        w, d = ctypes.c_uint64(), ctypes.c_uint32()
        nat.check(self._lib.hbfsim_amd_coupled_trace(self.handle, None, 0, None, 0, None, 0,
                                                     ctypes.byref(w), ctypes.byref(d)), "trace")
        windows, dies = int(w.value), int(d.value)
        hot = np.zeros((windows + 1) * dies, dtype=np.float64)
        level = np.zeros(windows, dtype=np.uint8)
        refresh = np.zeros(windows * dies, dtype=np.uint8)
        nat.check(self._lib.hbfsim_amd_coupled_trace(
            self.handle, _ptr(hot), hot.size, _ptr(level), level.size, _ptr(refresh),
            refresh.size, ctypes.byref(w), ctypes.byref(d)), "trace")
        return {"windows": windows, "dies": dies, "hot": hot.reshape(windows + 1, dies),
                "level": level, "refresh": refresh.reshape(windows, dies)}

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            self._lib.hbfsim_amd_thermal_destroy(self._h)
            self._h = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def pack_records(records: Any) -> Any:
    """32-byte records (torch int64 [n, 4] on the GPU: addr, bytes, issue_ps,
    flags) packed into 16-byte ones (int64 [n, 2]: addr | bytes << 48,
    issue_ps | flags << 56).  ValueError when a record does not fit: address
    from 2^48, byte count from 2^16, issue time from 2^56 ps, flags from 256."""
    addr, nbytes, issue, flags = (records[:, k] for k in range(4))
    if bool(((addr >> 48) != 0).any() | ((nbytes >> 16) != 0).any() |
            ((issue >> 56) != 0).any() | ((flags >> 8) != 0).any()):
        raise ValueError("records do not fit the packed 16-byte form")
    import torch
    return torch.stack([addr | (nbytes << 48), issue | (flags << 56)], dim=1).contiguous()


def mqsim_admission(arrival_ns: Any, nbytes: Any, queue_depth: int, latency_ns: int,
                    bandwidth_bytes_per_s: int, stream: Any = None) -> tuple[Any, Any]:
    """hbfsim_amd_mqsim_admission: the MQSim adapter's queue-depth admission
    and bandwidth cursor over a media port of one latency (int64 tensors on
    the GPU, arrivals non-decreasing).  Returns (admission_ns,
    completion_ns); ValueError for what the library refuses."""
    import torch
    n = int(arrival_ns.shape[0])
    adm = torch.empty(max(n, 1), dtype=torch.int64, device=arrival_ns.device)
    done = torch.empty(max(n, 1), dtype=torch.int64, device=arrival_ns.device)
    rc = nat.load().hbfsim_amd_mqsim_admission(
        _ptr(arrival_ns), _ptr(nbytes), n, queue_depth, latency_ns, bandwidth_bytes_per_s,
        _ptr(adm), _ptr(done), ctypes.c_void_p(_stream_handle(stream)))
    if rc == nat.HBFSIM_INVALID_ARGUMENT:
        raise ValueError("arrivals out of order, bandwidth 0 or times from 2^63 ns")
    nat.check(rc, "mqsim admission")
    return adm[:n], done[:n]


def media_servers(now_ns: Any, servers: int, latency_ns: int, stream: Any = None) -> Any:
    """MediaServers::issue (prefetch_model.cpp:22-50) over a batch of reads
    issued at non-decreasing times `now_ns` (torch int64 on the GPU): returns
    their completion times.  Raises ValueError for issue times that decrease
    or reach 2^63 ns."""
    import torch

    n = int(now_ns.shape[0])
    out = torch.empty(max(n, 1), dtype=torch.int64, device=now_ns.device)
    lib = nat.load()
    rc = lib.hbfsim_amd_media_servers(_ptr(now_ns), n, servers, latency_ns, _ptr(out),
                                      ctypes.c_void_p(_stream_handle(stream)))
    if rc == nat.HBFSIM_INVALID_ARGUMENT:
        raise ValueError("issue times must not decrease and must stay below 2^63 ns")
    nat.check(rc, "media servers")
    return out[:n]


def validate_profile(path: str) -> str | None:
    """None when the profile is valid, else the reference's error message."""
    buf = ctypes.create_string_buffer(512)
    code = nat.load().hbfsim_amd_validate_profile(os.fsencode(path), buf, len(buf))
    return None if code == nat.HBFSIM_OK else buf.value.decode()


def probe_bandwidth(gib: int = 4, reps: int = 5, stream: Any = None) -> dict:
    """HBM ceilings of the per-record passes' access patterns on this GPU
    (hbfsim_amd_probe_bandwidth): `gib` GiB streamed with 16-byte
    non-temporal loads, then written with 16-byte non-temporal stores of
    whole 1 KiB rows; GB/s of each, averaged over `reps` passes."""
    import torch
    nbytes = gib << 30
    buf = torch.empty(nbytes // 8, dtype=torch.int64, device="cuda")
    rms, wms = ctypes.c_float(), ctypes.c_float()
    nat.check(nat.load().hbfsim_amd_probe_bandwidth(
        _ptr(buf), nbytes, reps, ctypes.c_void_p(_stream_handle(stream)), ctypes.byref(rms),
        ctypes.byref(wms)), "bandwidth probe")
    del buf
    return {"read_gbps": nbytes / (rms.value / 1e3) / 1e9,
            "write_gbps": nbytes / (wms.value / 1e3) / 1e9,
            "read_ms": rms.value, "write_ms": wms.value, "bytes": nbytes, "reps": reps,
            "how": "hbfsim_amd_probe_bandwidth: 16-B non-temporal loads (one wave per 256 KiB, "
                   "16 in flight per lane), then 16-B non-temporal stores of 1 KiB rows (one "
                   "wave per 128 KiB), HIP events"}
