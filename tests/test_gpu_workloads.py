"""The benchmark workload (config 2, Qwen3-30B-A3B MoE decode) on the GPU:
the record compiler matches its host mirror, a prefix of a decode step
matches the CPU oracle bit for bit, and a full 2.68e8-record step satisfies
size-independent properties of the model exactly."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
import parity
from hbfsim_amd import engine as eng
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu

SHAPE = workloads.QWEN3_30B_A3B
C2 = workloads.PROFILES / "c2.json"


@pytest.fixture(scope="module")
def step0():
    import torch
    sel = workloads.moe_selection(SHAPE, 1)[0]
    seg = workloads.moe_segments(SHAPE, sel)
    rec = workloads.gpu_segment_records(seg, SHAPE.lines_per_expert, SHAPE.line, SHAPE.gap_ps,
                                        SHAPE.issuers)
    torch.cuda.synchronize()
    yield seg, rec
    del rec
    torch.cuda.empty_cache()


def test_record_compiler_matches_host_mirror(step0):
    seg, rec = step0
    n = rec.shape[0]
    assert n == len(seg) * SHAPE.lines_per_expert
    head = rec[:200_000].cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(head, workloads.segment_records(
        seg, SHAPE.lines_per_expert, SHAPE.line, SHAPE.gap_ps, SHAPE.issuers, 0, 200_000))
    idx = np.unique(np.linspace(0, n - 1, 5000).astype(np.int64))
    import torch
    got = rec[torch.from_numpy(idx).cuda()].cpu().numpy().view(np.uint64)
    for k, j in enumerate(idx):
        want = workloads.segment_records(seg, SHAPE.lines_per_expert, SHAPE.line, SHAPE.gap_ps,
                                         SHAPE.issuers, int(j), 1)[0]
        assert np.array_equal(got[k], want), j
    issue = rec[:, 2]
    assert bool((issue[1:] >= issue[:-1]).all())


def test_step_prefix_bit_exact(step0):
    _, rec = step0
    prefix = rec[: 1 << 22].cpu().numpy().view(np.uint64)
    p = parity.Pair(C2, workloads.moe_ranges(SHAPE))
    try:
        g, c = p.run(prefix)
        parity.assert_same(g, c, "config2 prefix")
        p.check_state()
    finally:
        p.close()


def test_full_step_properties(step0):
    """One full decode step: every line modeled; within a page the 127 lines
    after the first hit the page register (one sense per 16 KiB page); every
    channel moved exactly 4 ns per line; split runs equal one run."""
    import torch
    seg, rec = step0
    n = rec.shape[0]
    e = eng.Engine(str(C2))
    for base, length, perms in workloads.moe_ranges(SHAPE):
        e.register(base, length, perms)
    comp = torch.empty(n, dtype=torch.int64, device="cuda")
    rep = e.run(rec, comp)
    assert rep["records"] == rep["modeled"] == rep["reads"] == n
    pages = n * SHAPE.line // 16384
    assert rep["page_hits"] == n - pages
    planes, chans = e.busy_totals()
    assert int(chans.sum()) == 4000 * n
    assert int(planes.sum()) == pages * 5_000_000
    issue = rec[:, 2]
    assert bool((comp >= issue).all())
    assert int(comp.max()) == rep["makespan_ps"]
    e.close()
    # the same step in three runs, carrying state: identical completions
    e2 = eng.Engine(str(C2))
    for base, length, perms in workloads.moe_ranges(SHAPE):
        e2.register(base, length, perms)
    comp2 = torch.empty(n, dtype=torch.int64, device="cuda")
    cuts = [0, 12_345_677, 99_999_999, n]
    for a, b in zip(cuts[:-1], cuts[1:]):
        e2.run(rec[a:b], comp2[a:b])
    torch.cuda.synchronize()
    assert torch.equal(comp, comp2)
    e2.close()


def test_two_steps_carry_state(step0):
    """Step 2 starts at step 1's makespan, as the benchmark chains steps; a
    prefix of both steps together matches the oracle."""
    _, rec = step0
    prefix = rec[: 1 << 20].cpu().numpy().view(np.uint64)
    p = parity.Pair(C2, workloads.moe_ranges(SHAPE))
    try:
        g, c = p.run(prefix)
        parity.assert_same(g, c, "step 1")
        g2, c2 = p.run(prefix, base_ps=g[2]["makespan_ps"])
        parity.assert_same(g2, c2, "step 2")
        p.check_state()
    finally:
        p.close()
