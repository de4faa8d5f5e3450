"""HybridSampler and Calibrator (calibrator.cpp:67-138) on the GPU, through
the C ABI, against the oracle and the compiled reference's vectors
(tests/golden/ref_vectors.json "hybrid").  Sampler flags and the
calibrator's count, mean and percentiles are bit-exact; log_mean and
log_sigma come from double arithmetic on the GPU where the reference sums in
long double, and must agree to 1e-12 relative (1e-12 absolute for a
deviation near zero)."""
from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest

import oracle_py

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "ref_vectors.json"
LOG_REL = 1e-12
LOG_ABS = 1e-12


@pytest.fixture(scope="module")
def hy():
    import torch
    assert torch.cuda.is_available()
    from hbfsim_amd import hybrid
    return hybrid


def golden():
    return json.loads(GOLDEN.read_text())["hybrid"]


def random_classes(rng, n, classes):
    pool = rng.integers(0, 2**32, (classes, 4), dtype=np.uint64)
    pool[:, 0] %= 2
    pool[: classes // 2, 2:] = 0  # some classes differ only in the low key
    return np.ascontiguousarray(pool[rng.integers(0, classes, n)].astype(np.uint32))


def test_sampler_known_answers(hy):
    """calibrator_test.cpp:18-26."""
    s = hy.HybridSampler(4, 0.25, 7)
    read_class, write_class = (0, 16384, 0, 0), (1, 16384, 0, 0)
    assert all(s.reference(q, read_class) for q in range(4))
    assert s.reference(4, write_class)
    assert s.reference(12345, read_class) == s.reference(12345, read_class)
    s.close()
    for rate in (-0.5, 1.01, float("nan")):
        with pytest.raises(ValueError):
            hy.HybridSampler(0, rate, 0)


def test_sampler_reference_vectors(hy):
    for c in golden()["sampler"]:
        n = len(c["access"])
        s = hy.HybridSampler(c["warmup"], c["rate"], c["seed"])
        if n == 0:
            flags, count = s.reference_batch(np.zeros((0, 4), np.uint32),
                                             first_sequence=c["first"])
            assert count == 0 and flags.numel() == 0
            continue
        flags, count = s.reference_batch(np.array(c["access"], np.uint32),
                                         first_sequence=c["first"])
        got = flags.cpu().numpy().tolist()
        assert got == c["flags"], c["seed"]
        assert count == sum(c["flags"])
        s.close()


@pytest.mark.parametrize("n,classes,cuts", [
    (1000, 3, [0, 1, 10, 500, 1000]),
    (200_000, 64, [0, 100_000, 100_001, 200_000]),
    (1_000_000, 5000, [0, 1_000_000]),
])
def test_sampler_batches_equal_oracle(hy, n, classes, cuts):
    """A stream cut into batches: the seen set carries across calls, so the
    flags of the batches together equal the oracle's over the whole stream;
    explicit sequence tensors and consecutive ones agree."""
    import torch
    rng = np.random.default_rng(n + classes)
    acc = random_classes(rng, n, classes)
    first = int(rng.integers(0, 2**40))
    seq = np.arange(first, first + n, dtype=np.uint64)
    want = oracle_py.sampler_run(300, 0.05, 99, acc, seq)
    s = hy.HybridSampler(300, 0.05, 99)
    s2 = hy.HybridSampler(300, 0.05, 99)
    parts, total = [], 0
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        flags, count = s.reference_batch(acc[lo:hi], first_sequence=first + lo)
        seq_t = torch.from_numpy(seq[lo:hi].view(np.int64).copy()).cuda()
        flags2, _ = s2.reference_batch(acc[lo:hi], sequence=seq_t)
        assert torch.equal(flags, flags2)
        parts.append(flags.cpu().numpy())
        total += count
    got = np.concatenate(parts)
    np.testing.assert_array_equal(got, want)
    assert total == int(want.sum())
    s.close()
    s2.close()


def test_sampler_rate_edges(hy):
    rng = np.random.default_rng(5)
    acc = random_classes(rng, 5000, 10)
    seq = np.arange(5000, dtype=np.uint64)
    for warm, rate in ((0, 0.0), (0, 1.0), (2**32 - 1, 0.3), (17, 0.999999)):
        s = hy.HybridSampler(warm, rate, 123)
        flags, count = s.reference_batch(acc)
        want = oracle_py.sampler_run(warm, rate, 123, acc, seq)
        np.testing.assert_array_equal(flags.cpu().numpy(), want)
        assert count == int(want.sum())
        s.close()


def check_rows(got, want_rows):
    """got: {AccessClass: estimate}; want_rows: oracle rows."""
    assert list(got) == [tuple(int(r[f]) for f in ("operation", "bytes", "queue_bucket",
                                                   "locality_bucket")) for r in want_rows]
    for (cls, e), r in zip(got.items(), want_rows):
        assert (e.count, e.mean_ns, e.p50_ns, e.p95_ns, e.p99_ns) == \
            tuple(int(r[f]) for f in ("count", "mean_ns", "p50_ns", "p95_ns", "p99_ns")), cls
        assert e.log_mean == pytest.approx(float(r["log_mean"]), rel=LOG_REL, abs=LOG_ABS)
        assert e.log_sigma == pytest.approx(float(r["log_sigma"]), rel=LOG_REL, abs=LOG_ABS)


def test_calibrator_known_answers(hy):
    """calibrator_test.cpp:92-105."""
    c = hy.Calibrator()
    read_class, write_class = (0, 16384, 0, 0), (1, 16384, 0, 0)
    for v in (10_000, 12_000, 14_000):
        c.observe(read_class, v)
    e = c.estimate(read_class)
    assert e is not None
    assert (e.count, e.mean_ns, e.p50_ns, e.p95_ns) == (3, 12_000, 12_000, 14_000)
    assert np.isfinite(e.log_mean) and np.isfinite(e.log_sigma)
    assert c.estimate(write_class) is None
    with pytest.raises(ValueError):
        c.observe(read_class, 0)
    assert hy.Calibrator().estimates() == {}


def test_calibrator_reference_vectors(hy):
    for case in golden()["calibrate"]:
        c = hy.Calibrator()
        c.observe_batch(np.array(case["access"], np.uint32), np.array(case["latency"], np.uint64))
        got = c.estimates()
        assert [list(k) for k in got] == [r["class"] for r in case["rows"]]
        for e, r in zip(got.values(), case["rows"]):
            assert [e.count, e.mean_ns, e.p50_ns, e.p95_ns, e.p99_ns] == r["u64"]
            assert e.log_mean == pytest.approx(r["f64"][0], rel=LOG_REL, abs=LOG_ABS)
            assert e.log_sigma == pytest.approx(r["f64"][1], rel=LOG_REL, abs=LOG_ABS)


@pytest.mark.parametrize("n,classes", [(1, 1), (300_000, 1), (500_000, 40), (200_000, 20_000)])
def test_calibrator_equals_oracle(hy, n, classes):
    """One class of many samples (one block loops over it), many classes of
    few, latencies with repeats and 64-bit extremes (128-bit sums)."""
    rng = np.random.default_rng(n ^ classes)
    acc = random_classes(rng, n, classes)
    lat = rng.integers(1, 5_000_000, n, dtype=np.uint64)
    big = rng.random(n) < 0.01
    lat[big] = np.uint64(2**64 - 1) - rng.integers(0, 1000, int(big.sum()), dtype=np.uint64)
    c = hy.Calibrator()
    half = n // 2
    c.observe_batch(acc[:half], lat[:half])
    c.observe_batch(acc[half:], lat[half:])
    check_rows(c.estimates(), oracle_py.calibrate(acc, lat))


def test_calibrate_reports_row_count_and_zero_latency(hy):
    import ctypes
    import torch
    from hbfsim_amd import _native as nat
    from hbfsim_amd.engine import _ptr
    lib = nat.load()
    acc = hy.access_tensor(np.array([[0, 1, 0, 0], [1, 1, 0, 0], [0, 1, 0, 0]], np.uint32))
    lat = torch.tensor([5, 6, 7], dtype=torch.int64, device="cuda")
    rows = torch.empty((3, 9), dtype=torch.int64, device="cuda")
    count = ctypes.c_size_t()
    rc = lib.hbfsim_amd_calibrate(_ptr(acc), _ptr(lat), 3, _ptr(rows), 1, ctypes.byref(count),
                                  None)
    assert rc == nat.HBFSIM_INVALID_ARGUMENT and count.value == 2
    lat[1] = 0
    rc = lib.hbfsim_amd_calibrate(_ptr(acc), _ptr(lat), 3, _ptr(rows), 3, ctypes.byref(count),
                                  None)
    assert rc == nat.HBFSIM_INVALID_ARGUMENT
