"""The vLLM extension path end to end: a session made by
hbfsim_vllm_session_create (hbfsim_extension.cpp:18-49), storage registered
by hbfsim_vllm_register_storage (a TIMING range with READ permission,
hbfsim_extension.cpp:51-67) at real device addresses, then records timed
through hbfsim_vllm_session_context -> hbfsim_amd_run_device, bit-exact
against the oracle holding the same read-only ranges, over two runs whose
engine state carries."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import _native as nat
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

C0 = workloads.PROFILES / "c0.json"


def session_stream(seed: int, n: int, ranges, t0: int = 0) -> np.ndarray:
    """Reads inside the registered storage (most), writes (refused: the
    storage is read-only), bypass addresses and zero-byte records."""
    rng = np.random.default_rng(seed)
    rec = np.zeros((n, 4), np.uint64)
    which = rng.integers(0, len(ranges), n)
    kind = rng.integers(0, 100, n)
    size = rng.choice([64, 128, 256, 512], n)
    for i in range(n):
        base, length, _ = ranges[which[i]]
        b = int(size[i])
        a = base + int(rng.integers(0, length // b)) * b
        op = 0
        if kind[i] >= 97:
            op = 1
        elif kind[i] >= 94:
            a = 0x1000 + int(rng.integers(0, 1 << 16)) * 64
        elif kind[i] >= 92:
            b = 0
        rec[i] = (a, b, 0, op)
    gaps = rng.integers(0, 5000, n).astype(np.uint64)
    rec[:, 2] = t0 + np.cumsum(gaps, dtype=np.uint64)
    return rec


def test_session_context_times_records(tmp_path):
    import torch
    lib = nat.load()
    w1 = torch.empty(16 << 20, dtype=torch.uint8, device="cuda")
    w2 = torch.empty(6 << 20, dtype=torch.uint8, device="cuda")
    h = ctypes.c_void_p()
    o = nat.VllmOptions(str(C0).encode(), str(tmp_path).encode(), 64, 2, 10**9)
    assert lib.hbfsim_vllm_session_create(ctypes.byref(o), ctypes.byref(h)) == 0
    try:
        ranges = [(w1.data_ptr(), w1.numel(), nat.HBFSIM_RANGE_READ),
                  (w2.data_ptr(), w2.numel(), nat.HBFSIM_RANGE_READ)]
        for base, length, _ in ranges:
            assert lib.hbfsim_vllm_register_storage(h, base, length) == 0
        ctx = lib.hbfsim_vllm_session_context(h)
        assert ctx
        prof = oracle_py.load_profile(C0)
        params = oracle_py.engine_params(prof)
        table, count = oracle_py.range_table(ranges, prof["page_bytes"], prof["capacity_bytes"])
        state = oracle_py.OracleState(params)
        stream = torch.cuda.current_stream().cuda_stream
        t0 = 0
        for k, n in enumerate((60_000, 25_000)):
            rec = session_stream(40 + k, n, ranges, t0)
            t0 = int(rec[-1, 2]) + 1
            d_rec = parity.to_device(rec)
            d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
            d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
            rep = nat.Report()
            assert lib.hbfsim_amd_run_device(ctx, d_rec.data_ptr(), n, d_comp.data_ptr(),
                                             d_st.data_ptr(), 0, ctypes.c_void_p(stream),
                                             ctypes.byref(rep)) == 0
            torch.cuda.synchronize()
            gpu = (d_comp.cpu().numpy().view(np.uint64), d_st.cpu().numpy(), rep.as_dict())
            ocomp, ost, orep, _ = oracle_py.run(params, table, count, rec, 0, state)
            parity.assert_same(gpu, (ocomp, ost, orep), f"session run {k}")
            assert (ost == 0).sum() > n // 2 and (ost != 0).any()
    finally:
        assert lib.hbfsim_vllm_session_close(ctypes.byref(h)) == 0
    assert not h.value
