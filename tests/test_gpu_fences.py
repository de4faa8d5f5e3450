"""The range lookup's two levels at their boundaries.  The engine stages
every stride-th range base in LDS (at most 256 of them) and searches the
stride below in memory, so the stride steps from 1 to 2 at 257 ranges and to
3 at 513, and is 128 at the 32,768-range capacity.  Records aim at every range's first and last line, at the gaps
before and after it (bypass), and at random lines across the whole table,
in random order; both record forms must equal the oracle bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from test_gpu_linear import BASE, PAGE, ranges_for
from test_gpu_parity import C0, C2

pytestmark = pytest.mark.gpu

LINE = 64


def lookup_stream(ranges, seed, n_random=20_000):
    rng = np.random.default_rng(seed)
    addr = []
    for base, length, _ in ranges:
        addr += [base, base + length - LINE, base + length, base - LINE]
    lo, hi = BASE - PAGE, ranges[-1][0] + ranges[-1][1] + PAGE
    addr += list(lo + rng.integers(0, (hi - lo) // LINE, n_random) * LINE)
    addr = np.array(addr, dtype=np.uint64)
    rng.shuffle(addr)
    rec = np.zeros((len(addr), 4), np.uint64)
    rec[:, 0] = addr
    rec[:, 1] = LINE
    rec[:, 2] = np.arange(len(addr), dtype=np.uint64) * np.uint64(3000)
    return rec


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("count", [255, 256, 257, 511, 512, 513, 1000, 16384, 32767, 32768])
def test_range_lookup_stride_boundaries(profile, count):
    ranges = ranges_for(count=count - 1, pages=2)  # count - 1 readable + 1 write-only
    assert len(ranges) == count
    rec = lookup_stream(ranges, seed=count)
    a = parity.Pair(profile, ranges)
    b = parity.Pair(profile, ranges)
    try:
        (ga, sa, ra), ca = a.run(rec)
        parity.assert_same((ga, sa, ra), ca, f"{count} ranges, 32-byte")
        assert ra["bypass"] > 0 and ra["unsupported"] > 0
        gb, cb = b.run_packed(rec)
        parity.assert_same(gb, cb, f"{count} ranges, packed")
        a.check_state()
        b.check_state()
    finally:
        a.close()
        b.close()
