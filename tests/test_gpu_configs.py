"""Configs 1, 2 and 3 on the GPU, every completion against the CPU oracle.
Config 1 (TinyLlama-1.1B weight streaming, 17.2M records a step): two whole
decode steps.  Config 2 (the benchmarked Qwen3-30B-A3B MoE decode, 2.7e8
records a step): the bench's first two steps, chained with the makespan
carried as the next base as bench.py does, in both record forms; the same
two steps in hybrid mode (the bench's hybrid line), one hybrid step whose
sampler sequence crosses 2^32, and one step with two page registers per
plane.  Config 3 (paged KV cache): every step of a reduced shape, and one
whole full-size step (1.17e9 records over 150 GB of KV).  The oracle runs
over each whole step in chunks with its state carried (the steps are in issue
order, so chunks are the same as one run).  The GPU record compiler is
checked against its host mirror on the way."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import workloads as w
from hbfsim_amd.engine import pack_records

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


def packed_equals(packed, d_rec, n, base_ps, gpu, what):
    """The same step through packed records on a second engine with the same
    history (where steps crossing a page fold as split steps): completions,
    status bytes and report equal to the 32-byte run's."""
    import torch
    d_pk = pack_records(d_rec)
    comp = torch.zeros(n, dtype=torch.int64, device="cuda")
    st = torch.zeros(n, dtype=torch.uint8, device="cuda")
    rep = packed.engine.run_packed(d_pk, comp, st, base_ps=base_ps)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(comp.cpu().numpy().view(np.uint64), gpu[0], err_msg=what)
    np.testing.assert_array_equal(st.cpu().numpy(), gpu[1], err_msg=what)
    assert rep == gpu[2], what


def test_tinyllama_two_decode_steps_bit_exact():
    """Both record forms: the packed one folds the steps that cross a page
    as split steps."""
    shape = w.TINYLLAMA
    spans = w.dense_spans(shape)
    d_rec = gpu_records(spans, shape)
    n = int(d_rec.shape[0])
    assert n == 17_188_256
    np.testing.assert_array_equal(d_rec[:1 << 20].cpu().numpy().view(np.uint64),
                                  host_records(spans, shape, 0, 1 << 20))
    pair = parity.Pair(C0, w.dense_ranges(shape))
    packed = parity.Pair(C0, w.dense_ranges(shape))
    try:
        base = 0
        for step in range(2):
            gpu, cpu = run_pair(pair, d_rec, n, base)
            parity.assert_same(gpu, cpu, f"TinyLlama step {step}")
            assert gpu[2]["modeled"] == n and gpu[2]["page_hits"] > 0
            packed_equals(packed, d_rec, n, base, gpu, f"TinyLlama step {step} packed")
            base = gpu[2]["makespan_ps"]
        pair.check_state()
        for k in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(packed.engine.state()[k], pair.engine.state()[k], k)
    finally:
        pair.close()
        packed.close()


def test_kv_reduced_all_steps_bit_exact():
    shape = w.PagedKvShape(layers=3, seqs=9, min_len=40, max_len=700, steps=5)
    tables = shape.tables()
    pair = parity.Pair(C3, w.kv_ranges(shape))
    packed = parity.Pair(C3, w.kv_ranges(shape))
    try:
        base, programs = 0, 0
        for step in range(shape.steps):
            spans = w.kv_spans(shape, step, tables)
            d_rec = gpu_records(spans, shape)
            n = int(d_rec.shape[0])
            gpu, cpu = run_pair(pair, d_rec, n, base, threads=1)
            parity.assert_same(gpu, cpu, f"paged KV step {step}")
            assert gpu[2]["writes"] == 2 * shape.layers * shape.seqs * 16
            # token blocks joined inside a step fold as split steps when packed
            packed_equals(packed, d_rec, n, base, gpu, f"paged KV step {step} packed")
            programs += gpu[2]["programs"]
            base = gpu[2]["makespan_ps"]
        assert programs > 0  # appends that fill a page program it
        pair.check_state()
    finally:
        pair.close()
        packed.close()


def test_kv_full_size_step():
    """One whole full-size paged-KV step: 1.17e9 records (reads of every page
    of 64 sequences x 32 layers, one appended token per sequence and layer),
    every completion and status equal to the oracle's, in both record forms;
    the totals also match the configuration's arithmetic."""
    import torch
    shape = w.PAGED_KV
    spans = w.kv_spans(shape, 0)
    n = int(spans[1][-1])
    d_rec = gpu_records(spans, shape)
    prefix = 1 << 20
    np.testing.assert_array_equal(d_rec[:prefix].cpu().numpy().view(np.uint64),
                                  host_records(spans, shape, 0, prefix))
    pair = parity.Pair(C3, w.kv_ranges(shape))
    packed = parity.Pair(C3, w.kv_ranges(shape))
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
        # the packed form of the same step gives the same results
        d_pk = pack_records(d_rec)
        p_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        p_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        prep = packed.engine.run_packed(d_pk, p_comp, p_st)
        torch.cuda.synchronize()
        del d_pk
        assert prep == rep
        assert torch.equal(p_comp, d_comp) and torch.equal(p_st, d_st)
        del p_comp, p_st
        orep = parity.compare_whole(pair, d_rec, d_comp, d_st, 0, "paged KV full step")
        assert orep == rep
        pair.check_state()
    finally:
        pair.close()
        packed.close()


def test_config2_bench_steps_whole():
    """The benchmark's first two config-2 steps (2.7e8 records each, 48 x 128
    Qwen3-30B-A3B experts on the 512-plane profile), timed from packed
    records with the first step's makespan carried as the second's base, as
    bench.py chains them: every completion and status byte, both reports,
    the per-resource busy totals and the engine state equal the oracle's.
    The second step's issue times lie beyond 2^32 ps.  The same steps from
    32-byte records give the same results, and step 0 cut into two runs at an
    arbitrary record gives them too."""
    import torch
    shape = w.QWEN3_30B_A3B
    sel = w.moe_selection(shape, 2)
    c2 = w.PROFILES / "c2.json"
    pair = parity.Pair(c2, w.moe_ranges(shape))
    wide = parity.Pair(c2, w.moe_ranges(shape))
    split = parity.Pair(c2, w.moe_ranges(shape))
    try:
        base = 0
        for k in range(2):
            seg = w.moe_segments(shape, sel[k])
            d_rec = w.gpu_segment_records(seg, shape.lines_per_expert, shape.line,
                                          shape.gap_ps, shape.issuers)
            n = int(d_rec.shape[0])
            assert n > 2.5e8
            if k == 0:
                np.testing.assert_array_equal(
                    d_rec[:1 << 20].cpu().numpy().view(np.uint64),
                    w.segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                      shape.issuers, 0, 1 << 20))
            d_pk = pack_records(d_rec)
            d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
            d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
            rep = pair.engine.run_packed(d_pk, d_comp, d_st, base_ps=base)
            torch.cuda.synchronize()
            del d_pk
            assert rep["records"] == rep["modeled"] == rep["reads"] == n
            assert n - n // 64 <= rep["page_hits"] < n
            w_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
            w_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
            wrep = wide.engine.run(d_rec, w_comp, w_st, base_ps=base)
            torch.cuda.synchronize()
            assert wrep == rep
            assert torch.equal(w_comp, d_comp) and torch.equal(w_st, d_st)
            del w_comp, w_st
            if k == 0:
                cut = (n // 3) | 37  # inside a step and a tile
                s_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
                s_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
                r1 = split.engine.run(d_rec[:cut], s_comp[:cut], s_st[:cut])
                r2 = split.engine.run(d_rec[cut:], s_comp[cut:], s_st[cut:])
                torch.cuda.synchronize()
                assert torch.equal(s_comp, d_comp) and torch.equal(s_st, d_st)
                assert r1["page_hits"] + r2["page_hits"] == rep["page_hits"]
                del s_comp, s_st
            else:
                assert base + int(d_rec[0, 2]) > 1 << 32
            orep = parity.compare_whole(pair, d_rec, d_comp, d_st, base, f"config-2 step {k}")
            assert orep == rep
            base = rep["makespan_ps"]
            del d_rec, d_comp, d_st
        pair.check_state()
        # the 32-byte context charged the same busy time to every resource
        for got, want in zip(wide.engine.busy_totals(), pair.engine.busy_totals()):
            np.testing.assert_array_equal(got, want)
    finally:
        pair.close()
        wide.close()
        split.close()


def hybrid_c2_profile(tmp_path):
    """Config 2's profile with the bench's hybrid sampling: rate 1%, 1,000
    warm-up requests."""
    import json
    prof = json.loads((w.PROFILES / "c2.json").read_text())
    prof.update(reference_sample_rate=0.01, reference_warmup_requests=1000)
    path = tmp_path / "c2-hybrid.json"
    path.write_text(json.dumps(prof))
    return path


def c2_step(shape, sel, k):
    return w.gpu_segment_records(w.moe_segments(shape, sel[k]), shape.lines_per_expert,
                                 shape.line, shape.gap_ps, shape.issuers)


def test_config2_hybrid_two_steps_whole(tmp_path):
    """The bench's hybrid line: two chained whole config-2 steps in hybrid
    mode (context mode 2) from packed records, every completion and status
    byte (sampled flag included), both reports, busy totals and the engine
    state (sequence included) equal to the oracle's."""
    import torch
    shape = w.QWEN3_30B_A3B
    sel = w.moe_selection(shape, 2)
    pair = parity.Pair(hybrid_c2_profile(tmp_path), w.moe_ranges(shape), mode="hybrid")
    try:
        base = 0
        for k in range(2):
            d_rec = c2_step(shape, sel, k)
            n = int(d_rec.shape[0])
            d_pk = pack_records(d_rec)
            d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
            d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
            rep = pair.engine.run_packed(d_pk, d_comp, d_st, base_ps=base)
            torch.cuda.synchronize()
            del d_pk
            assert rep["modeled"] == n and rep["hybrid_sampled"] > n // 200
            orep = parity.compare_whole(pair, d_rec, d_comp, d_st, base,
                                        f"config-2 hybrid step {k}")
            assert orep == rep
            base = rep["makespan_ps"]
            del d_rec, d_comp, d_st
        pair.check_state()
    finally:
        pair.close()


def test_config2_hybrid_sequence_past_2_32(tmp_path):
    """One whole config-2 step in hybrid mode with the engine's and the
    oracle's modeled-request sequence set just below 2^32: the sampler's
    hash takes sequence ^ key in 64 bits all through the step, which
    carries the sequence past 2^32."""
    import torch
    shape = w.QWEN3_30B_A3B
    sel = w.moe_selection(shape, 1)
    pair = parity.Pair(hybrid_c2_profile(tmp_path), w.moe_ranges(shape), mode="hybrid")
    try:
        seq0 = (1 << 32) - 3_000_000
        st = pair.engine.state()
        st["sequence"] = seq0
        pair.engine.set_state(st)
        pair.ostate.s.modeled_sequence = seq0
        d_rec = c2_step(shape, sel, 0)
        n = int(d_rec.shape[0])
        d_pk = pack_records(d_rec)
        d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        rep = pair.engine.run_packed(d_pk, d_comp, d_st)
        torch.cuda.synchronize()
        del d_pk
        orep = parity.compare_whole(pair, d_rec, d_comp, d_st, 0, "config-2 hybrid near 2^32")
        assert orep == rep and rep["hybrid_sampled"] > 0
        assert pair.engine.state()["sequence"] == seq0 + n > 1 << 32
        pair.check_state()
    finally:
        pair.close()


def test_config2_two_page_registers_whole_step():
    """One whole config-2 step with two page registers per plane
    (device_coalescer.cpp:134-168), from 32-byte records: every completion
    and status byte, the report, busy totals and both tags of every plane
    equal to the oracle's."""
    import torch
    shape = w.QWEN3_30B_A3B
    sel = w.moe_selection(shape, 1)
    pair = parity.Pair(w.PROFILES / "c2.json", w.moe_ranges(shape), page_buffers=2)
    try:
        d_rec = c2_step(shape, sel, 0)
        n = int(d_rec.shape[0])
        d_comp = torch.zeros(n, dtype=torch.int64, device="cuda")
        d_st = torch.zeros(n, dtype=torch.uint8, device="cuda")
        rep = pair.engine.run(d_rec, d_comp, d_st)
        torch.cuda.synchronize()
        assert rep["modeled"] == n and rep["page_hits"] > n // 2
        orep = parity.compare_whole(pair, d_rec, d_comp, d_st, 0, "config-2 K=2 step")
        assert orep == rep
        pair.check_state()
    finally:
        pair.close()
