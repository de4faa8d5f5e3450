"""Split steps of packed records.  A step of 64 reads with one issue time and
byte count whose addresses form two linear runs -- one run cut by a page
boundary (records 0 .. k-1 end a page, k .. 63 start the next) or two spans
joined at lane k (in one page, two pages or two ranges) -- stays on the
batched linear path as two runs: the summary pass folds both, writes the
step's descriptor with its second run beside it, and the apply pass replays
windows holding such steps from their descriptors (one batch, or two when
the window has more than 64 runs) or folds them while streaming records.
Every case must match the CPU oracle bit for bit; steps that only look
split (a record straddling the page boundary, a second span that breaks off,
leaves its range or reaches a write-only one) take the general path and must
match too."""
from __future__ import annotations

import json

import numpy as np
import pytest

import parity
from test_gpu_linear import BASE, PAGE, chain_clocks, linear_stream, ranges_for
from test_gpu_parity import C0, C2

pytestmark = pytest.mark.gpu

PAGES = 96  # pages per range of ranges_for()


def split_stream(seed, steps, ranges, kinds=None):
    rng = np.random.default_rng(seed)
    kinds = kinds or {"whole": 0.35, "cross": 0.25, "join": 0.15, "join_range": 0.08,
                      "join_same": 0.05, "straddle": 0.03, "join_broken": 0.03,
                      "cross_end": 0.02, "join_wo": 0.02, "write": 0.02}
    names = list(kinds)
    probs = np.array([kinds[k] for k in names], float)
    probs /= probs.sum()
    readable = [r for r in ranges if r[2] & 1]
    wo = [r for r in ranges if not r[2] & 1][0]
    hot = [(int(rng.integers(0, len(readable))), int(rng.integers(0, PAGES - 1)))
           for _ in range(10)]
    lanes = np.arange(64, dtype=np.uint64)
    out = []
    t = 3_000_000

    def place(b, count):
        """A page and an offset in it where `count` records of b bytes fit."""
        ri, pg = hot[int(rng.integers(0, len(hot)))] if rng.random() < 0.6 else \
            (int(rng.integers(0, len(readable))), int(rng.integers(0, PAGES - 1)))
        slots = (PAGE - count * b) // b
        return readable[ri][0] + pg * PAGE + int(rng.integers(0, slots + 1)) * b

    for _ in range(steps):
        kind = names[int(rng.choice(len(names), p=probs))]
        b = int(rng.choice([64, 128, 256]))
        k = int(rng.integers(1, 64))
        t += int(rng.choice([0, 0, 500, 4000, 70_000]))
        addr = np.zeros(64, np.uint64)
        if kind in ("whole", "write"):
            addr[:] = np.uint64(place(b, 64)) + lanes * np.uint64(b)
        elif kind in ("cross", "straddle", "cross_end"):
            base = readable[int(rng.integers(0, len(readable)))][0]
            pg = PAGES - 1 if kind == "cross_end" else int(rng.integers(0, PAGES - 1))
            end = base + (pg + 1) * PAGE
            a0 = end - k * b - (b // 2 if kind == "straddle" else 0)
            addr[:] = np.uint64(a0) + lanes * np.uint64(b)
        else:
            a0 = place(b, k)
            if kind == "join":
                a1 = place(b, 64 - k)
            elif kind == "join_range":  # the second span in another range
                other = readable[(readable.index(next(r for r in readable
                                                      if r[0] <= a0 < r[0] + r[1])) + 1)
                                 % len(readable)]
                a1 = other[0] + int(rng.integers(0, PAGES)) * PAGE
            elif kind == "join_same":  # both spans in one page
                a1 = a0 - a0 % PAGE + int(rng.integers(0, (PAGE - (64 - k) * b) // b + 1)) * b
            elif kind == "join_wo":
                a1 = wo[0] + int(rng.integers(0, PAGES)) * PAGE
            else:  # join_broken: one record after lane k leaves the line
                a1 = place(b, 64 - k)
            addr[:k] = np.uint64(a0) + lanes[:k] * np.uint64(b)
            addr[k:] = np.uint64(a1) + lanes[: 64 - k] * np.uint64(b)
            if kind == "join_broken":
                addr[int(rng.integers(k, 64))] += np.uint64(PAGE // 2)
        step = np.zeros((64, 4), np.uint64)
        step[:, 0] = addr
        step[:, 1] = b
        step[:, 2] = t
        if kind == "write":
            step[int(rng.integers(0, 64)), 3] = 1
        out.append(step)
    return np.concatenate(out)


def check_packed(pair, rec, what, base_ps=0):
    g, c = pair.run_packed(rec, base_ps)
    parity.assert_same(g, c, what)
    return g, c


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("options", [
    dict(), dict(plane_contention=0), dict(transfer_page=1), dict(tile_records=64 * 64),
    dict(tile_records=64 * 70), dict(tile_records=64 * 8)])
def test_split_steps_bit_exact(profile, options):
    ranges = ranges_for()
    rec = split_stream(31, 2500, ranges)
    p = parity.Pair(profile, ranges, **options)
    try:
        (_, _, grep), _ = check_packed(p, rec, f"split steps {profile.name} {options}")
        assert grep["page_hits"] > 0 and grep["bypass"] > 0 and grep["unsupported"] > 0
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("kinds", [{"cross": 1.0}, {"cross": 0.5, "whole": 0.5},
                                   {"join": 0.6, "join_same": 0.4},
                                   {"cross": 0.3, "join_range": 0.3, "whole": 0.4}],
                         ids=["all_split", "half_split", "joins", "mixed"])
@pytest.mark.parametrize("tile", [None, 64 * 64, 64 * 100])
def test_split_only_windows(kinds, tile):
    """Windows whose 64 steps are all split (128 runs: the apply pass replays
    them in two batches of 32 steps), half split (about 96 runs), and
    windows of joins only; batches of at most 63 runs in the summary pass."""
    ranges = ranges_for()
    rec = split_stream(37 + len(kinds), 64 * 40 + 17, ranges, kinds=kinds)
    for profile in (C0, C2):
        p = parity.Pair(profile, ranges, tile_records=tile)
        try:
            (_, _, grep), _ = check_packed(p, rec, f"{kinds} tile {tile} {profile.name}")
            assert grep["modeled"] == len(rec)
            p.check_state()
        finally:
            p.close()


@pytest.mark.parametrize("k", [1, 2, 31, 32, 33, 62, 63])
def test_split_lanes(k):
    """Every step crosses a page at lane k, each step on the next page (so
    the second run of one step and the first run of the next share a page
    and hit), then steps that join spans at lane k."""
    ranges = ranges_for()
    lanes = np.arange(64, dtype=np.uint64)
    out, t = [], 1_000_000
    b = 128
    for s in range(300):
        base = ranges[s % 3 * 2 + 1][0]
        pg = s % (PAGES - 1)
        t += [0, 800, 25_000][s % 3]
        step = np.zeros((64, 4), np.uint64)
        step[:, 0] = np.uint64(base + (pg + 1) * PAGE - k * b) + lanes * np.uint64(b)
        step[:, 1] = b
        step[:, 2] = t
        out.append(step)
    cross = np.concatenate(out)
    joins = split_stream(k, 300, ranges, kinds={"join": 1.0})
    rec = chain_clocks(cross, joins)
    p = parity.Pair(C2, ranges)
    try:
        (_, _, grep), _ = check_packed(p, rec, f"split at lane {k}")
        assert grep["modeled"] == len(rec)
        p.check_state()
    finally:
        p.close()


@pytest.mark.parametrize("rate,warmup", [(0.02, 100), (0.3, 5), (1.0, 0)])
def test_split_steps_hybrid(tmp_path, rate, warmup):
    """Hybrid sampling keys each record on its own run's page and range: a
    joined step's second span may lie in another range."""
    prof = json.loads(C0.read_text())
    prof.update(reference_sample_rate=rate, reference_warmup_requests=warmup)
    path = tmp_path / "c0-hybrid-split.json"
    path.write_text(json.dumps(prof))
    ranges = ranges_for()
    rec = split_stream(41, 1500, ranges)
    p = parity.Pair(path, ranges, mode="hybrid")
    try:
        for run in range(2):
            (_, _, grep), _ = check_packed(p, rec, f"hybrid split {rate} {warmup} run {run}")
            assert grep["hybrid_sampled"] > 0
            rec = rec.copy()
            rec[:, 2] += np.uint64(int(rec[-1, 2]) + 1)
        p.check_state()
    finally:
        p.close()


def test_split_steps_equal_32_byte_run():
    """The same stream through both record forms (32-byte records take no
    split steps): equal completions, status bytes, report and state."""
    ranges = ranges_for()
    rec = chain_clocks(split_stream(43, 3000, ranges), linear_stream(44, 800, ranges))
    a = parity.Pair(C2, ranges)
    b = parity.Pair(C2, ranges)
    try:
        ga, _ = a.run(rec)
        gb, _ = check_packed(b, rec, "packed")
        np.testing.assert_array_equal(ga[0], gb[0])
        np.testing.assert_array_equal(ga[1], gb[1])
        assert ga[2] == gb[2]
        sa, sb = a.engine.state(), b.engine.state()
        for key in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(sa[key], sb[key], key)
    finally:
        a.close()
        b.close()


def test_split_steps_noalloc_equal_ordinary():
    """The entry point that allocates nothing has no side array for second
    runs: its split steps are replayed from their records.  Results equal the
    ordinary packed run's, twice in a row (the second run smaller)."""
    import torch
    from hbfsim_amd import engine as eng
    from hbfsim_amd.engine import pack_records
    ranges = ranges_for()
    rec = split_stream(47, 2000, ranges)
    e1, e2 = eng.Engine(str(C2)), eng.Engine(str(C2))
    try:
        for e in (e1, e2):
            for base, length, perms in ranges:
                e.register(base, length, perms)
        d = pack_records(torch.from_numpy(rec.view(np.int64)).cuda())
        warm = pack_records(torch.from_numpy(linear_stream(1, 20, ranges).view(np.int64)).cuda())
        for e in (e1, e2):  # the engines exist
            c = torch.zeros(warm.shape[0], dtype=torch.int64, device="cuda")
            e.run_packed(warm, c)
        base = int(e1.report()["makespan_ps"])
        for n in (len(rec), len(rec) // 3 + 5):
            c1 = torch.zeros(n, dtype=torch.int64, device="cuda")
            c2 = torch.zeros(n, dtype=torch.int64, device="cuda")
            s1 = torch.zeros(n, dtype=torch.uint8, device="cuda")
            s2 = torch.zeros(n, dtype=torch.uint8, device="cuda")
            r1 = e1.run_packed(d[:n], c1, s1, base_ps=base)
            r2 = e2.run_packed_noalloc(d[:n], c2, s2, base_ps=base)
            torch.cuda.synchronize()
            assert r1 == r2
            assert torch.equal(c1, c2) and torch.equal(s1, s2)
            base = int(r1["makespan_ps"])
        for key in ("plane_busy", "plane_tags", "channel_cursor"):
            np.testing.assert_array_equal(e1.state()[key], e2.state()[key], key)
    finally:
        e1.close()
        e2.close()


def test_split_range_base_not_page_aligned():
    """Ranges whose base is not a multiple of the page size: pages are
    counted from the range base, so a step splits where the range's page
    ends, not where the address is page-aligned."""
    ranges = [(BASE + 4096, 40 * PAGE, 1), (BASE + 64 * PAGE + 512, 40 * PAGE, 3),
              (BASE + 200 * PAGE, 8 * PAGE, 2)]
    rng = np.random.default_rng(5)
    lanes = np.arange(64, dtype=np.uint64)
    out, t = [], 0
    for s in range(600):
        base = ranges[s % 2][0]
        k = int(rng.integers(1, 64))
        b = int(rng.choice([64, 256]))
        pg = int(rng.integers(0, 39))
        t += int(rng.choice([0, 900]))
        step = np.zeros((64, 4), np.uint64)
        step[:, 0] = np.uint64(base + (pg + 1) * PAGE - k * b) + lanes * np.uint64(b)
        step[:, 1] = b
        step[:, 2] = t
        out.append(step)
    rec = np.concatenate(out)
    p = parity.Pair(C0, ranges)
    try:
        (_, _, grep), _ = check_packed(p, rec, "unaligned range bases")
        assert grep["modeled"] == len(rec)
        p.check_state()
    finally:
        p.close()
