"""Deterministic synthetic access streams for the benchmark configurations.

Every random draw is a counter-based SplitMix64 output, so a stream is a pure
function of (seed, stream id, index) and the same on every machine and on the
GPU.  Exponential inter-arrival gaps use a fixed inverse-CDF table in
picoseconds with integer interpolation; the table is built once on the host
from `math.log` and its checksum is pinned in the tests.

Record layout: uint64 [n, 4] = addr, bytes, issue_ps, flags (0 read, 1 write).
"""
from __future__ import annotations

import dataclasses
import math
import pathlib

import numpy as np

PROFILES = pathlib.Path(__file__).resolve().parent / "profiles"
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
EXP_TABLE_BITS = 12
EXP_TABLE_CAP = 20.0  # the last bucket ends at 20 x mean instead of infinity


def splitmix(v: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser with its increment (uint64 arrays, wrapping)."""
    with np.errstate(over="ignore"):
        z = (v + GOLDEN).astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> np.uint64:
    x = np.array([(seed * 0x100000001B3 + stream * 0xD1B54A32D192ED03) & (2**64 - 1)],
                 dtype=np.uint64)
    return splitmix(x)[0]


def draws(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """Outputs start..start+count-1 of the SplitMix64 sequence keyed by (seed, stream)."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return splitmix(stream_key(seed, stream) + idx * GOLDEN)


def exp_table(mean_ps: int) -> np.ndarray:
    """T[k] = round(mean * -ln(1 - k / 2^bits)), k = 0..2^bits, last capped."""
    size = 1 << EXP_TABLE_BITS
    t = np.zeros(size + 1, dtype=np.uint64)
    for k in range(size):
        t[k] = int(round(mean_ps * -math.log1p(-k / size)))
    t[size] = int(round(mean_ps * EXP_TABLE_CAP))
    return t


def exp_gaps(u: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Integer inverse-CDF sample: top bits pick the bucket, the next 20 bits
    interpolate linearly inside it."""
    hi = (u >> np.uint64(64 - EXP_TABLE_BITS)).astype(np.int64)
    lo = ((u >> np.uint64(64 - EXP_TABLE_BITS - 20)) & np.uint64(0xFFFFF))
    a = table[hi]
    b = table[hi + 1]
    return a + (((b - a) * lo) >> np.uint64(20))


@dataclasses.dataclass
class Stream:
    """A workload: ranges to register and the records to time."""
    profile: pathlib.Path
    ranges: list[tuple[int, int, int]]  # (base, length, permissions)
    records: np.ndarray                  # uint64 [n, 4]
    name: str = ""


RANGE_BASE = 0x7F00_0000_0000  # where synthetic ranges start (any address works)


def config0(n: int = 1 << 20, seed: int = 0, mean_gap_ps: int = 2000,
            range_bytes: int = 1 << 30, line: int = 128,
            write_fraction_per_mille: int = 0) -> Stream:
    """Config 0: uniform random 128-B lines in one 1 GiB range, Poisson issue
    with mean gap 2 ns, all reads (writes optional for wider tests)."""
    lines = range_bytes // line
    u_addr = draws(seed, 1, 0, n)
    idx = (u_addr % np.uint64(lines)).astype(np.uint64)
    gaps = exp_gaps(draws(seed, 2, 0, n), exp_table(mean_gap_ps))
    issue = np.cumsum(gaps, dtype=np.uint64)
    rec = np.zeros((n, 4), dtype=np.uint64)
    rec[:, 0] = np.uint64(RANGE_BASE) + idx * np.uint64(line)
    rec[:, 1] = line
    rec[:, 2] = issue
    if write_fraction_per_mille:
        w = (draws(seed, 3, 0, n) % np.uint64(1000)) < np.uint64(write_fraction_per_mille)
        rec[:, 3] = w.astype(np.uint64)
    return Stream(PROFILES / "c0.json", [(RANGE_BASE, range_bytes, 3)], rec, "config0")
