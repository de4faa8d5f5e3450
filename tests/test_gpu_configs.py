"""Configs 1 and 3 on the GPU.  Config 1 (TinyLlama-1.1B weight streaming,
17.2M records a step) runs two whole decode steps bit-exact against the CPU
oracle.  Config 3 (paged KV cache) runs every step of a reduced shape
bit-exact, and one full-size step (1.17e9 records, 150 GB of KV) whose prefix
matches the oracle and whose totals match the configuration's arithmetic.
One full config-2 step (2.7e8 records) is checked the same way, and against
itself run as two runs with carried state.
The GPU record compiler is checked against its host mirror on the way."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import workloads as w

pytestmark = pytest.mark.gpu

C0 = w.PROFILES / "c0.json"
C3 = w.PROFILES / "c3.json"


def gpu_records(spans, shape):
    return w.gpu_span_records(*spans, shape.line, shape.gap_ps, shape.issuers)


def host_records(spans, shape, start=0, count=None):
    return w.span_records(*spans, shape.line, shape.gap_ps, shape.issuers, start, count)


def test_span_compiler_matches_host():
    rng = np.random.default_rng(4)
    lines = rng.choice([0, 1, 5, 255, 256, 257, 4000], 300).astype(np.uint64)
    base = (np.uint64(1 << 44) + rng.integers(0, 1 << 30, 300).astype(np.uint64) *
            np.uint64(128))
    first = np.zeros(301, np.uint64)
    np.cumsum(lines, out=first[1:])
    op = rng.integers(0, 2, 300).astype(np.uint32)
    d = w.gpu_span_records(base, first, op, 128, 7000, 96)
    np.testing.assert_array_equal(d.cpu().numpy().view(np.uint64),
                                  w.span_records(base, first, op, 128, 7000, 96))


def run_pair(pair, d_rec, n, base_ps, threads=8):
    """GPU run on device records and the oracle on the same records."""
    import torch
    d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
    d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
    grep = pair.engine.run(d_rec, d_comp, d_st, base_ps=base_ps)
    torch.cuda.synchronize()
    rec = d_rec.cpu().numpy().view(np.uint64)
    ocomp, ost, orep, _ = oracle_py.run(pair.params, pair.ranges, pair.count, rec, base_ps,
                                        pair.ostate, threads=threads)
    gpu = (d_comp.cpu().numpy().view(np.uint64), d_st.cpu().numpy(), grep)
    return gpu, (ocomp, ost, orep)


def test_tinyllama_two_decode_steps_bit_exact():
    shape = w.TINYLLAMA
    spans = w.dense_spans(shape)
    d_rec = gpu_records(spans, shape)
    n = int(d_rec.shape[0])
    assert n == 17_188_256
    np.testing.assert_array_equal(d_rec[:1 << 20].cpu().numpy().view(np.uint64),
                                  host_records(spans, shape, 0, 1 << 20))
    pair = parity.Pair(C0, w.dense_ranges(shape))
    try:
        base = 0
        for step in range(2):
            gpu, cpu = run_pair(pair, d_rec, n, base)
            parity.assert_same(gpu, cpu, f"TinyLlama step {step}")
            assert gpu[2]["modeled"] == n and gpu[2]["page_hits"] > 0
            base = gpu[2]["makespan_ps"]
        pair.check_state()
    finally:
        pair.close()


def test_kv_reduced_all_steps_bit_exact():
    shape = w.PagedKvShape(layers=3, seqs=9, min_len=40, max_len=700, steps=5)
    tables = shape.tables()
    pair = parity.Pair(C3, w.kv_ranges(shape))
    try:
        base, programs = 0, 0
        for step in range(shape.steps):
            spans = w.kv_spans(shape, step, tables)
            d_rec = gpu_records(spans, shape)
            n = int(d_rec.shape[0])
            gpu, cpu = run_pair(pair, d_rec, n, base, threads=1)
            parity.assert_same(gpu, cpu, f"paged KV step {step}")
            assert gpu[2]["writes"] == 2 * shape.layers * shape.seqs * 16
            programs += gpu[2]["programs"]
            base = gpu[2]["makespan_ps"]
        assert programs > 0  # appends that fill a page program it
        pair.check_state()
    finally:
        pair.close()


def test_kv_full_size_step():
    import torch
    shape = w.PAGED_KV
    spans = w.kv_spans(shape, 0)
    n = int(spans[1][-1])
    d_rec = gpu_records(spans, shape)
    prefix = 6_000_000
    np.testing.assert_array_equal(d_rec[:prefix].cpu().numpy().view(np.uint64),
                                  host_records(spans, shape, 0, prefix))
    pair = parity.Pair(C3, w.kv_ranges(shape))
    try:
        d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        rep = pair.engine.run(d_rec, d_comp, d_st)
        torch.cuda.synchronize()
        lens = shape.lengths()
        writes = 2 * shape.layers * shape.seqs * (shape.token_bytes // shape.line)
        per_page = shape.page // shape.token_bytes
        fills = int(((lens % per_page) == per_page - 1).sum()) * 2 * shape.layers
        assert rep["records"] == rep["modeled"] == n
        assert rep["writes"] == writes and rep["reads"] == n - writes
        assert rep["programs"] == fills
        assert rep["bypass"] == 0 and rep["unsupported"] == 0
        # completions never precede their issue, and the makespan is the last one
        issue = d_rec[:, 2]
        assert bool((d_comp >= issue).all())
        assert int(d_comp.max()) == rep["makespan_ps"]
        # the prefix is what the oracle computes for it
        rec = d_rec[:prefix].cpu().numpy().view(np.uint64)
        ocomp, ost, _, _ = oracle_py.run(pair.params, pair.ranges, pair.count, rec, 0,
                                         oracle_py.OracleState(pair.params), threads=8)
        np.testing.assert_array_equal(d_comp[:prefix].cpu().numpy().view(np.uint64), ocomp)
        np.testing.assert_array_equal(d_st[:prefix].cpu().numpy(), ost)
    finally:
        pair.close()


def test_config2_full_size_step():
    """One whole config-2 decode step (the bench's step 0: 2.7e8 records of
    48 x 128 Qwen3-30B-A3B experts on the 512-plane profile).  Its record
    prefix equals the host mirror of the compiler; its first 6M completions
    and statuses equal the oracle's (a completion depends only on earlier
    records); every record is a modeled read, no completion precedes its
    issue and the makespan is the last completion; and the same step run as
    two runs with carried state gives the same completions bit for bit."""
    import torch
    shape = w.QWEN3_30B_A3B
    seg = w.moe_segments(shape, w.moe_selection(shape, 1)[0])
    d_rec = w.gpu_segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                  shape.issuers)
    n = int(d_rec.shape[0])
    assert n > 2.5e8
    prefix = 6_000_000
    rec = d_rec[:prefix].cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(
        rec, w.segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                               shape.issuers, 0, prefix))
    c2 = w.PROFILES / "c2.json"
    whole = parity.Pair(c2, w.moe_ranges(shape))
    split = parity.Pair(c2, w.moe_ranges(shape))
    try:
        d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        rep = whole.engine.run(d_rec, d_comp, d_st)
        torch.cuda.synchronize()
        assert rep["records"] == rep["modeled"] == rep["reads"] == n
        assert rep["writes"] == 0 and rep["bypass"] == 0 and rep["unsupported"] == 0
        assert n - n // 64 <= rep["page_hits"] < n
        assert bool((d_comp >= d_rec[:, 2]).all())
        assert int(d_comp.max()) == rep["makespan_ps"]
        ocomp, ost, _, _ = oracle_py.run(whole.params, whole.ranges, whole.count, rec, 0,
                                         oracle_py.OracleState(whole.params), threads=8)
        np.testing.assert_array_equal(d_comp[:prefix].cpu().numpy().view(np.uint64), ocomp)
        np.testing.assert_array_equal(d_st[:prefix].cpu().numpy(), ost)
        cut = (n // 3) | 37  # inside a step and a tile
        s_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        s_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        r1 = split.engine.run(d_rec[:cut], s_comp[:cut], s_st[:cut])
        r2 = split.engine.run(d_rec[cut:], s_comp[cut:], s_st[cut:])
        torch.cuda.synchronize()
        assert torch.equal(s_comp, d_comp) and torch.equal(s_st, d_st)
        assert r1["page_hits"] + r2["page_hits"] == rep["page_hits"]
        assert max(r1["makespan_ps"], r2["makespan_ps"]) == rep["makespan_ps"]
    finally:
        whole.close()
        split.close()
