"""Linear steps (64 reads addr_0 + k * bytes_0 with one issue time, inside one
page) take a batched path on the GPU: they wait in a batch of up to 64 steps
that is folded with one lane per step.  These streams mix such steps with
steps that end a batch early (writes, page crossings, bypass and unreadable
ranges, short steps, steps with two issue times), revisit planes and pages inside one
batch and jump between ranges (the uniform range cache refills), under every
plane/transfer option; results must match the CPU oracle bit for bit.  The
streams are in issue order (streams that leave it are tested in
test_gpu_order.py)."""
from __future__ import annotations

import json

import numpy as np
import pytest

import parity
from test_gpu_parity import C0, C2, check

pytestmark = pytest.mark.gpu

PAGE = 16384
BASE = 0x6400_0000_0000


def ranges_for(count=6, pages=96):
    """Readable ranges, plus a write-only one (range index `count`)."""
    out = [(BASE + r * (pages + 8) * PAGE, pages * PAGE, 3 if r % 2 else 1) for r in range(count)]
    out.append((BASE + count * (pages + 8) * PAGE, pages * PAGE, 2))
    return out


def chain_clocks(*parts):
    """Concatenates record streams, each shifted in time to start no earlier
    than the previous one ends, so that the whole stream is in issue order."""
    out, t = [], 0
    for part in parts:
        part = part.copy()
        if len(part):
            first = int(part[:, 2].min())
            part[:, 2] += np.uint64(max(0, t - first))
            t = int(part[:, 2].max())
        out.append(part)
    return np.concatenate(out)


def linear_stream(seed, steps, ranges, kinds=None):
    """One step at a time: mostly linear steps on a few hot pages (so later
    steps of a batch hit pages earlier ones opened, on the same and other
    planes), with breaking steps in between."""
    rng = np.random.default_rng(seed)
    kinds = kinds or {"lin": 0.80, "write": 0.03, "cross": 0.03, "bypass": 0.03,
                      "wo": 0.02, "ragged": 0.03, "mixed_issue": 0.03}
    names = list(kinds)
    probs = np.array([kinds[k] for k in names], float)
    probs /= probs.sum()
    readable = [r for r in ranges if r[2] & 1]
    wo = [r for r in ranges if not r[2] & 1]
    hot = [(int(rng.integers(0, len(readable))), int(rng.integers(0, 96))) for _ in range(12)]
    out = []
    t = 10_000_000
    lanes = np.arange(64, dtype=np.uint64)
    for _ in range(steps):
        kind = names[int(rng.choice(len(names), p=probs))]
        b = int(rng.choice([64, 128, 256]))
        ri, pg = hot[int(rng.integers(0, len(hot)))] if rng.random() < 0.7 else \
            (int(rng.integers(0, len(readable))), int(rng.integers(0, 96)))
        base, length, _ = readable[ri]
        slot = int(rng.integers(0, PAGE // (64 * b)))
        a0 = base + pg * PAGE + slot * 64 * b
        t += int(rng.choice([0, 0, 500, 4000, 70_000]))
        issue = t
        step = np.zeros((64, 4), np.uint64)
        step[:, 0] = np.uint64(a0) + lanes * np.uint64(b)
        step[:, 1] = b
        step[:, 2] = issue
        if kind == "write":
            step[int(rng.integers(0, 64)), 3] = 1
        elif kind == "cross":  # the step runs over the page end
            step[:, 0] = np.uint64(base + pg * PAGE + PAGE - 32 * b) + lanes * np.uint64(b)
            if pg == length // PAGE - 1:
                step[:, 0] -= np.uint64(PAGE)
        elif kind == "bypass":
            step[:, 0] = np.uint64(0x1000) + lanes * np.uint64(b)
        elif kind == "wo":
            wb = wo[0][0]
            step[:, 0] = np.uint64(wb + pg * PAGE) + lanes * np.uint64(b)
        elif kind == "ragged":  # one lane's byte count differs
            step[int(rng.integers(0, 64)), 1] = b // 2
        elif kind == "late":  # issue time falls back far (the stream leaves issue order)
            step[:, 2] = max(0, issue - 9_000_000)
        elif kind == "mixed_issue":
            step[int(rng.integers(1, 64)):, 2] = issue + 1
            t += 1
        out.append(step)
    return np.concatenate(out)


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("options", [
    dict(), dict(plane_contention=0), dict(transfer_page=1), dict(tile_records=64 * 64),
    dict(tile_records=64 * 70),
])
def test_linear_batches_bit_exact(profile, options):
    ranges = ranges_for()
    rec = linear_stream(11, 1500, ranges)
    p = parity.Pair(profile, ranges, **options)
    try:
        (_, _, grep), _ = check(p, rec, f"linear batches {profile.name} {options}")
        assert grep["page_hits"] > 0 and grep["bypass"] > 0 and grep["unsupported"] > 0
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("rate,warmup", [(0.02, 100), (0.0, 70_000), (1.0, 0), (0.3, 5)])
@pytest.mark.parametrize("options", [dict(), dict(tile_records=64 * 70),
                                     dict(plane_contention=0)])
def test_linear_batches_hybrid(tmp_path, rate, warmup, options):
    """Hybrid mode on streams of linear steps across several ranges: the apply
    pass folds linear steps and samples each of their records (sequence
    number, media page, range id), as the general path does record by record;
    a warm-up reaching past the stream, a rate of 0 and of 1."""
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=rate, reference_warmup_requests=warmup)
    path = tmp_path / "c0-hybrid-linear.json"
    path.write_text(json.dumps(prof))
    ranges = ranges_for()
    rec = linear_stream(13, 1200, ranges)
    p = parity.Pair(path, ranges, mode="hybrid", **options)
    try:
        for k in range(2):  # the second run's sequence numbers continue
            (_, _, grep), _ = check(p, rec, f"hybrid linear {rate} {warmup} {options} run {k}")
            assert grep["hybrid_sampled"] > 0 or (rate == 0.0 and k == 1 and warmup < 2 * len(rec))
            rec = rec.copy()
            rec[:, 2] += np.uint64(int(rec[-1, 2]) + 1)
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("n_linear", [1, 2, 63, 64, 65, 127, 128, 129, 4095, 4097])
def test_linear_batch_lengths(n_linear):
    """Runs of exactly n linear steps, then a breaking step, a tail of fewer
    than 64 records, and runs that end exactly at the tile end."""
    ranges = ranges_for()
    rec = linear_stream(n_linear, n_linear, ranges, kinds={"lin": 1.0})
    brk = linear_stream(n_linear + 1, 3, ranges, kinds={"write": 1.0})
    tail = linear_stream(n_linear + 2, 1, ranges, kinds={"lin": 1.0})[:37]
    stream = np.concatenate([rec, brk, rec, tail])
    for tile in (None, 64 * 64, 64 * n_linear):
        p = parity.Pair(C2, ranges, tile_records=tile)
        try:
            check(p, stream, f"{n_linear} linear steps, tile {tile}")
            p.check_state()
        finally:
            p.close()


@pytest.mark.parametrize("wide", ["issue", "sense", "transfer"])
def test_linear_wide_times_take_64_bit_scans(tmp_path, wide):
    """Values past the 32-bit relative scans inside one batch: issue gaps
    beyond 2^30 ps between steps, a sense time of 4e7 ps (> 2^24), or a
    transfer quantum that makes a step's channel time 2^26 ps."""
    ranges = ranges_for()
    rec = linear_stream(5, 600, ranges, kinds={"lin": 1.0})
    profile, opts = C2, {}
    if wide == "issue":
        steps = rec.reshape(-1, 64, 4)
        steps[:, :, 2] = (np.arange(steps.shape[0], dtype=np.uint64) *
                          np.uint64(1_500_000_000))[:, None]
    elif wide == "sense":
        prof = json.loads(C2.read_text())
        prof["read_latency_ns"] = 40_000
        profile = tmp_path / "c2-slow-sense.json"
        profile.write_text(json.dumps(prof))
    else:
        opts = dict(xfer_quantum_ps=1 << 20)
    p = parity.Pair(profile, ranges, **opts)
    try:
        check(p, rec, f"wide linear steps ({wide})")
        p.check_state()
    finally:
        p.close()


def test_linear_split_runs_resume():
    """A stream cut inside batches: the carried state after each run must let
    the next run continue exactly."""
    ranges = ranges_for()
    rec = linear_stream(17, 900, ranges)
    whole = parity.Pair(C2, ranges)
    split = parity.Pair(C2, ranges)
    try:
        (gw, _, _), _ = check(whole, rec, "whole")
        parts = []
        for lo, hi in [(0, 64 * 10), (64 * 10, 64 * 10 + 5), (64 * 10 + 5, 64 * 500),
                       (64 * 500, len(rec))]:
            (g, _, _), _ = check(split, rec[lo:hi], f"part {lo}:{hi}")
            parts.append(g)
            split.check_state()
        np.testing.assert_array_equal(np.concatenate(parts), gw)
    finally:
        whole.close()
        split.close()


def contiguous_stream(seed, runs, ranges):
    """Runs of steps that continue one another in address (groups of four
    such steps take the group path), started at arbitrary step offsets so
    groups straddle pages, range ends and batch boundaries; issue times per
    step or per run; occasional breaking records inside a run."""
    rng = np.random.default_rng(seed)
    readable = [r for r in ranges if r[2] & 1]
    lanes = np.arange(64, dtype=np.uint64)
    out = []
    t = 5_000_000
    for _ in range(runs):
        base, length, _ = readable[int(rng.integers(0, len(readable)))]
        b = int(rng.choice([64, 128, 256]))
        steps = int(rng.integers(1, 41))
        start = int(rng.integers(0, length // (64 * b))) * 64 * b
        per_step_issue = rng.random() < 0.5
        for k in range(steps):
            a0 = base + start + k * 64 * b
            if a0 + 64 * b > base + length:
                a0 = base + length - 32 * b  # runs over the range end
            if not per_step_issue and k % 4 == 0 or per_step_issue:
                t += int(rng.choice([0, 300, 2000, 90_000]))
            step = np.zeros((64, 4), np.uint64)
            step[:, 0] = np.uint64(a0) + lanes * np.uint64(b)
            step[:, 1] = b
            step[:, 2] = t
            r = rng.random()
            if r < 0.02:
                step[int(rng.integers(0, 64)), 3] = 1        # a write
            elif r < 0.04:
                step[int(rng.integers(1, 64)):, 2] += 1      # the step's later records later
                t += 1
            elif r < 0.05:
                step[int(rng.integers(0, 64)), 0] += 1       # one address off the line
            out.append(step)
    return np.concatenate(out)


@pytest.mark.parametrize("options", [dict(), dict(plane_contention=0), dict(transfer_page=1),
                                     dict(tile_records=64 * 24)])
def test_linear_groups_bit_exact(options):
    ranges = ranges_for()
    rec = contiguous_stream(23, 400, ranges)
    for profile in (C0, C2):
        p = parity.Pair(profile, ranges, **options)
        try:
            (_, _, grep), _ = check(p, rec, f"linear groups {profile.name} {options}")
            assert grep["page_hits"] > 0
            p.check_state()
        finally:
            p.close()


def striding_stream(pages, b, seed, reps=2):
    """Linear steps, one per listed page (offset 0 of the page), one batch
    of 64 steps per list; each step with its own issue time."""
    rng = np.random.default_rng(seed)
    lanes = np.arange(64, dtype=np.uint64)
    out, t = [], 1_000_000
    base = BASE
    for _ in range(reps):
        for pg in pages:
            t += int(rng.choice([0, 700, 30_000]))
            step = np.zeros((64, 4), np.uint64)
            step[:, 0] = np.uint64(base + pg * PAGE) + lanes * np.uint64(b)
            step[:, 1] = b
            step[:, 2] = t
            out.append(step)
    return np.concatenate(out)


@pytest.mark.parametrize("profile,planes", [(C0, 64), (C2, 512)], ids=["c0", "c2"])
@pytest.mark.parametrize("shape", ["stride1", "span_below", "span_equal", "stride_over",
                                   "pairs"])
def test_linear_batches_rising_pages_across_one_stripe_period(profile, planes, shape):
    """Batches whose pages rise from step to step: within one striping period
    (span below the plane count) the runs of equal page are the plane groups;
    from a span of one period on, two pages of a batch may share a plane and
    grouping goes by key.  Both must agree with the oracle."""
    if shape == "stride1":
        pages = list(range(64))
    elif shape == "span_below":
        pages = sorted(set(np.linspace(0, planes - 1, 64).astype(int).tolist()))
    elif shape == "span_equal":  # the first and last page share a plane
        pages = sorted(set(np.linspace(0, planes, 64).astype(int).tolist()))
    elif shape == "stride_over":
        pages = [k * (planes // 32 + 1) for k in range(64)]
    else:  # two steps per page, as weight streaming has them
        pages = [k // 2 for k in range(64)]
    pages = [p % 1100 for p in pages]
    assert pages == sorted(pages)
    ranges = [(BASE, 1200 * PAGE, 1)]
    rec = striding_stream(pages, 128 if shape == "pairs" else 256, len(pages) + planes)
    p = parity.Pair(profile, ranges)
    try:
        (_, _, grep), _ = check(p, rec, f"rising pages {shape} on {planes} planes")
        assert grep["modeled"] == len(rec)
        p.check_state()
    finally:
        p.close()
