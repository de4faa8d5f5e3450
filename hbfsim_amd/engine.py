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
                 "channel_bandwidth_bytes_per_s", "tile_records")

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


def validate_profile(path: str) -> str | None:
    """None when the profile is valid, else the reference's error message."""
    buf = ctypes.create_string_buffer(512)
    code = nat.load().hbfsim_amd_validate_profile(os.fsencode(path), buf, len(buf))
    return None if code == nat.HBFSIM_OK else buf.value.decode()
