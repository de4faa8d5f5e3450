"""HybridSampler and Calibrator (src/hybrid/calibrator.cpp:67-138) in the
oracle, pinned by the reference's own known answers
(tests/cpu/calibrator_test.cpp:18-26, 92-105), by vectors from the compiled
calibrator.cpp (tests/golden/ref_vectors.json "hybrid"), live against that
build when it is present, and by closed forms: a set-based replay of the
sampler, percentile ranks counted by hand, the mean of logs and the
population deviation from the math library."""
from __future__ import annotations

import json
import math
import pathlib

import numpy as np
import pytest

import oracle_py

READ, WRITE = 0, 1
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "ref_vectors.json"


def hybrid_golden():
    return json.loads(GOLDEN.read_text())["hybrid"]


def test_sampler_known_answers():
    """calibrator_test.cpp:18-26: warm-up sequences 0..3 are references, a
    class never seen before is one, and the decision is a pure function of
    (sequence, class) once the class has been seen."""
    read_class = [READ, 16384, 0, 0]
    write_class = [WRITE, 16384, 0, 0]
    acc = [read_class] * 4 + [write_class, read_class, read_class]
    seq = [0, 1, 2, 3, 4, 12345, 12345]
    flags = oracle_py.sampler_run(4, 0.25, 7, acc, seq)
    assert flags[:5].tolist() == [1, 1, 1, 1, 1]
    assert flags[5] == flags[6]


def test_sampler_rejects_bad_rates():
    for rate in (-0.1, 1.5, math.nan, math.inf):
        with pytest.raises(ValueError):
            oracle_py.sampler_run(0, rate, 0, [[0, 1, 0, 0]], [0])


def mix(v):
    m = (1 << 64) - 1
    v = (v + 0x9E3779B97F4A7C15) & m
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & m
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & m
    return v ^ (v >> 31)


def replay_sampler(warmup, rate, seed, access, sequence):
    """The sampler as a Python set and a loop, one request at a time."""
    thr = (1 << 64) - 1 if rate >= 1.0 else oracle_py.lib().orc_sample_threshold(rate)
    seen, out = set(), []
    for (op, b, q, l), s in zip(access, sequence):
        key = (op, b, q, l)
        unseen = key not in seen
        seen.add(key)
        v = (s ^ seed ^ (b << 17) ^ ((q << 33) & ((1 << 64) - 1)) ^
             ((l << 49) & ((1 << 64) - 1)) ^ ((op << 61) & ((1 << 64) - 1)))
        out.append(1 if (s < warmup or unseen or mix(v) <= thr) else 0)
    return out


def test_sampler_equals_set_replay():
    rng = np.random.default_rng(4)
    for trial in range(30):
        n = int(rng.integers(0, 200))
        classes = rng.integers(0, 2**32, (int(rng.integers(1, 9)), 4), dtype=np.uint64)
        classes[:, 0] %= 2
        acc = classes[rng.integers(0, len(classes), n)].astype(np.uint32)
        seq = np.arange(n, dtype=np.uint64) + np.uint64(rng.integers(0, 2**40))
        warm, rate, seed = int(rng.integers(0, 20)), float(rng.random()), int(rng.integers(0, 2**63))
        got = oracle_py.sampler_run(warm, rate, seed, acc, seq).tolist()
        want = replay_sampler(warm, rate, seed, acc.astype(int).tolist(), seq.astype(int).tolist())
        assert got == want, trial


def test_sampler_matches_reference_vectors():
    for c in hybrid_golden()["sampler"]:
        assert c["ok"] == 1
        n = len(c["access"])
        acc = np.array(c["access"], np.uint32).reshape(n, 4)
        seq = np.arange(c["first"], c["first"] + n, dtype=np.uint64)
        got = oracle_py.sampler_run(c["warmup"], c["rate"], c["seed"], acc, seq)
        assert got.tolist() == c["flags"]


def test_calibrator_known_answers():
    """calibrator_test.cpp:92-105."""
    rows = oracle_py.calibrate([[READ, 16384, 0, 0]] * 3, [10_000, 12_000, 14_000])
    assert len(rows) == 1
    r = rows[0]
    assert (r["count"], r["mean_ns"], r["p50_ns"], r["p95_ns"]) == (3, 12_000, 12_000, 14_000)
    assert math.isfinite(r["log_mean"]) and math.isfinite(r["log_sigma"])
    assert not any(row["operation"] == WRITE for row in rows)
    with pytest.raises(ValueError):
        oracle_py.calibrate([[READ, 1, 0, 0]], [0])


def closed_form(samples):
    s = sorted(samples)
    n = len(s)

    def pct(num):
        rank = (n * num + 99) // 100
        return s[min(max(rank - 1, 0), n - 1)]

    logs = [math.log(x) for x in s]
    lm = math.fsum(logs) / n
    sigma = math.sqrt(math.fsum((x - lm) ** 2 for x in logs) / n)
    return n, sum(s) // n, pct(50), pct(95), pct(99), lm, sigma


def test_calibrator_closed_forms():
    rng = np.random.default_rng(9)
    for trial in range(20):
        n = int(rng.integers(1, 300))
        acc = np.zeros((n, 4), np.uint32)
        acc[:, 0] = rng.integers(0, 2, n)
        acc[:, 1] = rng.choice([512, 4096, 16384], n)
        lat = rng.integers(1, 2**40, n, dtype=np.uint64)
        rows = oracle_py.calibrate(acc, lat)
        keys = sorted({tuple(int(v) for v in a) for a in acc})
        assert [tuple(int(r[f]) for f in ("operation", "bytes", "queue_bucket",
                                          "locality_bucket")) for r in rows] == keys
        for r, key in zip(rows, keys):
            samples = [int(x) for a, x in zip(acc, lat) if tuple(int(v) for v in a) == key]
            cnt, mean, p50, p95, p99, lm, sg = closed_form(samples)
            assert (r["count"], r["mean_ns"], r["p50_ns"], r["p95_ns"], r["p99_ns"]) == \
                (cnt, mean, p50, p95, p99), trial
            assert r["log_mean"] == pytest.approx(lm, rel=1e-14)
            assert r["log_sigma"] == pytest.approx(sg, rel=1e-9, abs=1e-12)


def test_calibrator_matches_reference_vectors():
    for c in hybrid_golden()["calibrate"]:
        n = len(c["access"])
        acc = np.array(c["access"], np.uint32).reshape(n, 4)
        lat = np.array(c["latency"], np.uint64)
        rows = oracle_py.calibrate(acc, lat)
        assert len(rows) == len(c["rows"])
        for r, want in zip(rows, c["rows"]):
            assert want["ok"] == 1
            assert [int(r[f]) for f in ("operation", "bytes", "queue_bucket",
                                        "locality_bucket")] == want["class"]
            assert [int(r[f]) for f in ("count", "mean_ns", "p50_ns", "p95_ns",
                                        "p99_ns")] == want["u64"]
            assert [float(r["log_mean"]), float(r["log_sigma"])] == want["f64"]


def test_live_against_compiled_reference():
    ref = oracle_py.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref/libhbfref.so not built here")
    import ctypes
    P, U32, U64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
    ref.ref_sampler_run.argtypes = [U32, ctypes.c_double, U64, P, P, ctypes.c_size_t, P]
    ref.ref_calibrate.argtypes = [P, P, ctypes.c_size_t, P, P, P]
    rng = np.random.default_rng(31)
    for _ in range(10):
        n = 5000
        classes = rng.integers(0, 2**32, (int(rng.integers(1, 40)), 4), dtype=np.uint64)
        classes[:, 0] %= 2
        acc = np.ascontiguousarray(classes[rng.integers(0, len(classes), n)].astype(np.uint32))
        seq = np.arange(n, dtype=np.uint64)
        rate = float(rng.random())
        want = np.zeros(n, np.uint8)
        assert ref.ref_sampler_run(100, rate, 3, acc.ctypes.data, seq.ctypes.data, n,
                                   want.ctypes.data) == 1
        np.testing.assert_array_equal(oracle_py.sampler_run(100, rate, 3, acc, seq), want)
        lat = rng.integers(1, 2**50, n, dtype=np.uint64)
        rows = oracle_py.calibrate(acc, lat)
        for r in rows:
            q = np.array([r["operation"], r["bytes"], r["queue_bucket"], r["locality_bucket"]],
                         np.uint32)
            u = np.zeros(5, np.uint64)
            f = np.zeros(2, np.float64)
            assert ref.ref_calibrate(acc.ctypes.data, lat.ctypes.data, n, q.ctypes.data,
                                     u.ctypes.data, f.ctypes.data) == 1
            assert [int(r[k]) for k in ("count", "mean_ns", "p50_ns", "p95_ns", "p99_ns")] == \
                u.tolist()
            assert [float(r["log_mean"]), float(r["log_sigma"])] == f.tolist()
