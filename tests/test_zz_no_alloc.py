"""hbfsim_amd_run_device_packed_noalloc, the entry point that allocates
nothing (its scratch is the library's static per-device array), against
hbfsim_amd_run_device_packed through the C ABI: two calls in a row on one
context, the second smaller, give the same completions, status bytes,
reports and engine state as the allocating entry point; runs that do not
fit, an engine that does not exist yet and a changed range table are
refused without touching the context."""
from __future__ import annotations

import numpy as np
import pytest

from hbfsim_amd import engine as eng
from hbfsim_amd import workloads as w
from hbfsim_amd.engine import pack_records

pytestmark = pytest.mark.gpu


def engine_with(profile, ranges):
    e = eng.Engine(str(profile))
    for base, length, perms in ranges:
        e.register(base, length, perms)
    return e


def mixed_c0(n, seed):
    s = w.config0(n=n, seed=seed, write_fraction_per_mille=60)
    rec = s.records
    rec[::101, 0] -= np.uint64(1 << 21)          # below the range: bypass
    rec[7::131, 0] += np.uint64(16384 - 64)      # some cross their page: unsupported
    return s, rec


def run_both(ref, noalloc, d_rec32, base):
    import torch
    n = int(d_rec32.shape[0])
    d_pk = pack_records(d_rec32)
    out = []
    for e, run in ((ref, ref.run_packed), (noalloc, noalloc.run_packed_noalloc)):
        comp = torch.full((n,), -1, dtype=torch.int64, device="cuda")
        st = torch.full((n,), 255, dtype=torch.uint8, device="cuda")
        rep = run(d_pk, comp, st, base)
        torch.cuda.synchronize()
        out.append((comp.cpu().numpy(), st.cpu().numpy(), rep))
    (c1, s1, r1), (c2, s2, r2) = out
    np.testing.assert_array_equal(c2, c1)
    np.testing.assert_array_equal(s2, s1)
    assert r2 == r1
    return r1


def same_state(a, b):
    sa, sb = a.state(), b.state()
    for k in ("plane_busy", "plane_tags", "channel_cursor"):
        np.testing.assert_array_equal(sa[k], sb[k], k)
    assert sa["sequence"] == sb["sequence"]
    for x, y in zip(a.busy_totals(), b.busy_totals()):
        np.testing.assert_array_equal(x, y)


def test_noalloc_equals_packed_config0_two_calls():
    import torch
    s, rec = mixed_c0(300_000, 5)
    ref = engine_with(s.profile, s.ranges)
    na = engine_with(s.profile, s.ranges)
    try:
        empty = torch.zeros((0, 2), dtype=torch.int64, device="cuda")
        none = torch.zeros(1, dtype=torch.int64, device="cuda")
        na.run_packed(empty, none)  # creates the engine and uploads the ranges
        d = torch.from_numpy(rec.view(np.int64)).cuda()
        r = run_both(ref, na, d, 0)
        assert r["bypass"] > 0 and r["unsupported"] > 0 and r["writes"] > 0
        d2 = d[:70_001]  # a smaller second call, chained
        run_both(ref, na, d2, r["makespan_ps"])
        same_state(ref, na)
    finally:
        ref.close()
        na.close()


def test_noalloc_equals_packed_config2_slices():
    """512 planes: a 6M-record slice needs the doubled tile to fit the
    static scratch; then a 1M-record slice."""
    import torch
    shape = w.QWEN3_30B_A3B
    seg = w.moe_segments(shape, w.moe_selection(shape, 1)[0])
    d_all = w.gpu_segment_records(seg[:120], shape.lines_per_expert, shape.line, shape.gap_ps,
                                  shape.issuers)
    prof = w.PROFILES / "c2.json"
    ref = engine_with(prof, w.moe_ranges(shape))
    na = engine_with(prof, w.moe_ranges(shape))
    try:
        empty = torch.zeros((0, 2), dtype=torch.int64, device="cuda")
        na.run_packed(empty, torch.zeros(1, dtype=torch.int64, device="cuda"))
        r = run_both(ref, na, d_all[:6_000_000], 0)
        run_both(ref, na, d_all[6_000_000:7_000_000], r["makespan_ps"] + 123)
        same_state(ref, na)
    finally:
        ref.close()
        na.close()


def test_noalloc_refusals_leave_the_context_alone():
    import torch
    s, rec = mixed_c0(50_000, 9)
    e = engine_with(s.profile, s.ranges)
    try:
        d = pack_records(torch.from_numpy(rec.view(np.int64)).cuda())
        comp = torch.zeros(len(rec), dtype=torch.int64, device="cuda")
        with pytest.raises(ValueError):  # no engine yet
            e.run_packed_noalloc(d, comp)
        e.run_packed(d[:1000], comp[:1000])
        before = (e.state(), e.busy_totals(), e.report())
        # beyond the static scratch: at 64 planes and 8 channels about 125M
        # records fit (8.8 KB per tile of 16,384); 130M do not.  The buffers
        # are real and every record is a zero (bypass) record, so the call
        # would stay in bounds even if it ran.
        big = 130_000_000
        d_big = torch.zeros((big, 2), dtype=torch.int64, device="cuda")
        c_big = torch.zeros(big, dtype=torch.int64, device="cuda")
        with pytest.raises(ValueError):
            e.run_packed_noalloc(d_big, c_big)
        del d_big, c_big
        after = (e.state(), e.busy_totals(), e.report())
        for k in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(before[0][k], after[0][k])
        assert before[2] == after[2]
        # a range registered since the last run: refused until an ordinary run
        e.register(0x7000_0000_0000, 1 << 20, 1)
        with pytest.raises(ValueError):
            e.run_packed_noalloc(d, comp)
        e.run_packed(d[:10], comp[:10])
        e.run_packed_noalloc(d, comp)
    finally:
        e.close()


def test_noalloc_refuses_hybrid_mode():
    """Hybrid sampling reads the records again in the apply pass, which the
    run without allocation does not do: refused, while the ordinary packed
    run samples."""
    import torch
    s, rec = mixed_c0(20_000, 4)
    e = eng.Engine(str(s.profile), mode="hybrid")
    try:
        for base, length, perms in s.ranges:
            e.register(base, length, perms)
        d = pack_records(torch.from_numpy(rec.view(np.int64)).cuda())
        comp = torch.zeros(len(rec), dtype=torch.int64, device="cuda")
        e.run_packed(d, comp)
        with pytest.raises(ValueError):
            e.run_packed_noalloc(d, comp)
    finally:
        e.close()
