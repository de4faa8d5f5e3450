"""The hybrid model's request sampler and calibrator on the GPU
(src/hybrid/calibrator.cpp:67-138, include/hbfsim/hybrid_model.hpp:13-60).

HybridSampler and Calibrator keep the reference's names, arguments and
errors: the sampler's constructor raises ValueError where the reference
throws std::invalid_argument ("sample_rate must be in [0, 1]"), observe()
raises ValueError for a zero latency, estimate() returns None for a class
never observed.  Requests travel as access-class tensors on the GPU (n x 4
int32 holding the unsigned fields operation, bytes, queue_bucket,
locality_bucket); the single-request forms wrap a batch of one.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, NamedTuple, Sequence

import numpy as np

from . import _native as nat
from .engine import _ptr, _stream_handle

READ, WRITE = 0, 1


class AccessClass(NamedTuple):
    """hybrid_model.hpp:13-20; tuples order like its operator<=>."""
    operation: int = READ
    bytes: int = 0
    queue_bucket: int = 0
    locality_bucket: int = 0


@dataclass(frozen=True)
class CalibrationEstimate:
    """hybrid_model.hpp:28-36."""
    count: int
    mean_ns: int
    p50_ns: int
    p95_ns: int
    p99_ns: int
    log_mean: float
    log_sigma: float


def access_tensor(access: Any, device: Any = "cuda") -> Any:
    """An (n, 4) int32 GPU tensor of access classes from AccessClass values,
    an (n, 4) array of unsigned 32-bit fields, or such a tensor already."""
    import torch

    if isinstance(access, torch.Tensor):
        if access.dtype != torch.int32 or access.dim() != 2 or access.shape[1] != 4:
            raise ValueError("access tensor must be (n, 4) int32")
        return access.contiguous()
    arr = np.asarray(access, dtype=np.uint64).reshape(-1, 4)
    if arr.size and int(arr.max()) > 0xFFFFFFFF:
        raise ValueError("access class fields are 32-bit")
    return torch.from_numpy(arr.astype(np.uint32).view(np.int32).copy()).to(device)


class HybridSampler:
    """HybridSampler (calibrator.cpp:67-96) with its seen set on the GPU."""

    def __init__(self, warmup_requests: int, sample_rate: float, seed: int):
        self._lib = nat.load()
        self._h = ctypes.c_void_p()
        rc = self._lib.hbfsim_amd_sampler_create(warmup_requests, float(sample_rate), seed,
                                                 ctypes.byref(self._h))
        if rc == nat.HBFSIM_INVALID_ARGUMENT:
            raise ValueError("sample_rate must be in [0, 1]")
        nat.check(rc, "sampler create")

    def close(self) -> None:
        if self._h:
            self._lib.hbfsim_amd_sampler_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reference_batch(self, access: Any, sequence: Any = None, first_sequence: int = 0,
                        stream: Any = None) -> tuple[Any, int]:
        """reference(sequence_i, access_i) for every request in order: a uint8
        GPU tensor of decisions and the number of reference requests.
        sequence_i is sequence[i] (int64 GPU tensor) or first_sequence + i."""
        import torch

        acc = access_tensor(access)
        n = int(acc.shape[0])
        flags = torch.empty(max(n, 1), dtype=torch.uint8, device=acc.device)
        seq = None
        if sequence is not None:
            seq = sequence.contiguous()
            if seq.dtype != torch.int64 or seq.shape[0] != n:
                raise ValueError("sequence must be an int64 tensor of n entries")
        count = ctypes.c_uint64()
        nat.check(self._lib.hbfsim_amd_sampler_reference(
            self._h, _ptr(acc), _ptr(seq) if seq is not None else None, first_sequence, n,
            _ptr(flags), ctypes.byref(count), ctypes.c_void_p(_stream_handle(stream))),
            "sampler reference")
        return flags[:n], int(count.value)

    def reference(self, sequence: int, access: Sequence[int]) -> bool:
        flags, _ = self.reference_batch([tuple(access)], first_sequence=sequence)
        return bool(flags[0].item())


class Calibrator:
    """Calibrator (calibrator.cpp:98-136): latencies per access class, kept
    on the GPU; estimate() computes every class's row in one pass and keeps
    them until the next observe()."""

    def __init__(self):
        self._lib = nat.load()
        self._access: list[Any] = []
        self._latency: list[Any] = []
        self._rows: dict[AccessClass, CalibrationEstimate] | None = None

    def observe_batch(self, access: Any, latency_ns: Any) -> None:
        import torch

        acc = access_tensor(access)
        lat = latency_ns if isinstance(latency_ns, torch.Tensor) else torch.from_numpy(
            np.asarray(latency_ns, dtype=np.uint64).view(np.int64).copy()).to(acc.device)
        if lat.dtype != torch.int64 or lat.shape[0] != acc.shape[0]:
            raise ValueError("latency_ns must be an int64 tensor of n entries")
        if bool((lat == 0).any().item()):
            raise ValueError("latency_ns must be positive")
        self._access.append(acc)
        self._latency.append(lat.contiguous())
        self._rows = None

    def observe(self, access: Sequence[int], latency_ns: int) -> None:
        self.observe_batch([tuple(access)], [latency_ns])

    def estimates(self, stream: Any = None) -> dict[AccessClass, CalibrationEstimate]:
        """Every observed class's estimate, in class order."""
        import torch

        if self._rows is not None:
            return self._rows
        if not self._access:
            self._rows = {}
            return self._rows
        acc = torch.cat(self._access)
        lat = torch.cat(self._latency)
        n = int(acc.shape[0])
        # one 72-byte row per class: start small, and size exactly once the
        # library has said how many classes there are
        cap = min(n, 1 << 16)
        while True:
            rows = torch.empty((cap, 9), dtype=torch.int64, device=acc.device)
            count = ctypes.c_size_t()
            rc = self._lib.hbfsim_amd_calibrate(_ptr(acc), _ptr(lat), n, _ptr(rows), cap,
                                                ctypes.byref(count),
                                                ctypes.c_void_p(_stream_handle(stream)))
            if rc == nat.HBFSIM_INVALID_ARGUMENT and count.value > cap:
                cap = count.value
                continue
            break
        if rc == nat.HBFSIM_INVALID_ARGUMENT:
            raise ValueError("latency_ns must be positive")
        nat.check(rc, "calibrate")
        raw = rows[:count.value].cpu().numpy()
        cls = raw[:, :2].copy().view(np.uint32).reshape(-1, 4)
        u64 = raw[:, 2:7].view(np.uint64)
        f64 = raw[:, 7:9].view(np.float64)
        self._rows = {
            AccessClass(*(int(v) for v in c)): CalibrationEstimate(
                int(u[0]), int(u[1]), int(u[2]), int(u[3]), int(u[4]), float(f[0]), float(f[1]))
            for c, u, f in zip(cls, u64, f64)
        }
        return self._rows

    def estimate(self, access: Sequence[int]) -> CalibrationEstimate | None:
        return self.estimates().get(AccessClass(*access))
