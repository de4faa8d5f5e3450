"""Packed 16-byte records (hbf_record16) through hbfsim_amd_run_device_packed.
The packed form is an input format of this engine: every result must be the
oracle's on the 32-byte records it packs, bit for bit, across the linear
batch and group paths, the general per-record path, split runs, tile sizes
and both profiles; a whole config-2 step must equal the 32-byte run of the
same step; modes the packed path does not take are refused."""
from __future__ import annotations

import json

import numpy as np
import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for, striding_stream
from test_gpu_parity import C0, C2
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu


def check_packed(pair, rec, what, base_ps=0):
    g, c = pair.run_packed(rec, base_ps)
    parity.assert_same(g, c, what)
    return g, c


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("options", [dict(), dict(plane_contention=0), dict(transfer_page=1),
                                     dict(tile_records=64 * 24), dict(tile_records=64 * 300)])
def test_packed_linear_and_general_paths(profile, options):
    ranges = ranges_for()
    rec = chain_clocks(linear_stream(3, 800, ranges), contiguous_stream(4, 200, ranges))
    p = parity.Pair(profile, ranges, **options)
    try:
        (_, _, grep), _ = check_packed(p, rec, f"packed {profile.name} {options}")
        assert grep["page_hits"] > 0 and grep["bypass"] > 0 and grep["unsupported"] > 0
        p.check_state()
    finally:
        p.close()


def test_packed_config0_stream_and_split_runs():
    s = workloads.config0(n=200_000 + 17, seed=9, write_fraction_per_mille=100)
    whole = parity.Pair(C0, s.ranges)
    split = parity.Pair(C0, s.ranges)
    try:
        (gw, _, _), _ = check_packed(whole, s.records, "config0 packed")
        parts = []
        for lo, hi in [(0, 64 * 100 + 3), (64 * 100 + 3, 150_000), (150_000, len(s.records))]:
            (g, _, _), _ = check_packed(split, s.records[lo:hi], f"config0 part {lo}:{hi}")
            parts.append(g)
        np.testing.assert_array_equal(np.concatenate(parts), gw)
        whole.check_state()
        split.check_state()
    finally:
        whole.close()
        split.close()


def test_packed_rising_pages_and_edge_fields():
    """Batches across one striping period, and records at the packed form's
    edges: byte counts up to 65535, addresses near 2^48, issue times near
    2^56 ps (bypass records outside every range still pass through)."""
    ranges = [(0x6400_0000_0000, 1200 * 16384, 1)]
    rec = striding_stream([k * 9 for k in range(64)], 256, 5)
    edge = np.zeros((64 * 3, 4), np.uint64)
    edge[:, 0] = np.uint64((1 << 48) - 4096) + np.arange(64 * 3, dtype=np.uint64) * np.uint64(8)
    edge[:, 1] = 8
    edge[:64, 1] = 65535
    edge[:, 2] = np.uint64((1 << 56) - 10_000_000)
    p = parity.Pair(C2, ranges)
    try:
        check_packed(p, np.concatenate([rec, edge]), "rising pages and edges")
        p.check_state()
    finally:
        p.close()


def test_packed_full_config2_step_equals_32_byte_run():
    import torch
    from hbfsim_amd.engine import pack_records
    shape = workloads.QWEN3_30B_A3B
    seg = workloads.moe_segments(shape, workloads.moe_selection(shape, 1)[0])
    d_rec = workloads.gpu_segment_records(seg, shape.lines_per_expert, shape.line, shape.gap_ps,
                                          shape.issuers)
    n = int(d_rec.shape[0])
    d_pack = pack_records(d_rec)
    c2 = workloads.PROFILES / "c2.json"
    a = parity.Pair(c2, workloads.moe_ranges(shape))
    b = parity.Pair(c2, workloads.moe_ranges(shape))
    try:
        ca = torch.zeros(n, dtype=torch.int64, device="cuda")
        cb = torch.zeros(n, dtype=torch.int64, device="cuda")
        sa = torch.zeros(n, dtype=torch.uint8, device="cuda")
        sb = torch.zeros(n, dtype=torch.uint8, device="cuda")
        ra = a.engine.run(d_rec, ca, sa)
        rb = b.engine.run_packed(d_pack, cb, sb)
        torch.cuda.synchronize()
        assert torch.equal(ca, cb) and torch.equal(sa, sb)
        assert ra == rb
        np.testing.assert_array_equal(a.engine.busy_totals()[0], b.engine.busy_totals()[0])
        np.testing.assert_array_equal(a.engine.busy_totals()[1], b.engine.busy_totals()[1])
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("options", [dict(), dict(tile_records=64 * 24)])
def test_packed_hybrid(tmp_path, profile, options):
    """Hybrid sampling on packed records: linear steps folded in the apply
    pass with each record sampled, general steps record by record; equal to
    the oracle on the 32-byte records they pack, over two runs."""
    prof = json.loads(profile.read_text())
    prof.update(reference_sample_rate=0.05, reference_warmup_requests=300)
    path = tmp_path / "hybrid.json"
    path.write_text(json.dumps(prof))
    ranges = ranges_for()
    rec = chain_clocks(linear_stream(5, 600, ranges), contiguous_stream(6, 150, ranges))
    p = parity.Pair(path, ranges, mode="hybrid", **options)
    try:
        (_, _, g1), _ = check_packed(p, rec, f"packed hybrid {profile.name} {options}")
        rec2 = rec.copy()
        rec2[:, 2] += np.uint64(int(rec[-1, 2]) + 1)
        (_, _, g2), _ = check_packed(p, rec2, f"packed hybrid second run {options}")
        assert g1["hybrid_sampled"] > 300 and g2["hybrid_sampled"] > 0
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
def test_packed_without_page_register(profile):
    """page_buffers 0: no step is batched (the linear-step path needs the
    page register), every record takes the general path, none hits."""
    ranges = ranges_for()
    rec = chain_clocks(linear_stream(7, 600, ranges), contiguous_stream(8, 100, ranges))
    p = parity.Pair(profile, ranges, page_buffers=0)
    try:
        (_, _, grep), _ = check_packed(p, rec, f"packed {profile.name}, no page register")
        assert grep["page_hits"] == 0 and grep["modeled"] > 0
        check_packed(p, rec, f"packed {profile.name}, no page register, second run",
                     base_ps=int(grep["makespan_ps"]))
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("options", [dict(page_buffers=2)])
def test_packed_refuses_other_pipelines(options):
    import torch
    from hbfsim_amd import _native as nat
    from hbfsim_amd.engine import pack_records
    ranges = ranges_for()
    rec = linear_stream(1, 10, ranges)
    mode = options.pop("mode", "fast")
    p = parity.Pair(C2, ranges, mode=mode, **options)
    try:
        d = pack_records(parity.to_device(rec))
        comp = torch.zeros(len(rec), dtype=torch.int64, device="cuda")
        with pytest.raises(nat.HbfSimError) as err:
            p.engine.run_packed(d, comp)
        assert err.value.code == nat.HBFSIM_UNSUPPORTED
    finally:
        p.close()
