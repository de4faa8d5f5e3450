"""hbf_media_bench (hbfsim_amd/hbf_media_bench), the counterpart of the
reference's hbf_mqsim_bench (benchmarks/mqsim/hbf_mqsim_bench.cpp): its
argument contract and exit codes (:40-145, 357-367) here; its report, with
the engine's timing checked against the oracle over the same workload
(same slots, arrivals and operations, regenerated here), on the GPU."""
from __future__ import annotations

import json
import pathlib
import subprocess

import numpy as np
import pytest

import oracle_py

ROOT = pathlib.Path(__file__).resolve().parent.parent
BENCH = ROOT / "hbfsim_amd" / "hbf_media_bench"
NOMINAL = ROOT / "tests" / "golden" / "profiles" / "nominal.json"
RANGE_BASE = 0x4000_0000_0000


@pytest.fixture(scope="module")
def bench():
    if not BENCH.exists():
        from hbfsim_amd import build
        build.build_cli()
    return BENCH


def run(bench, *args):
    return subprocess.run([str(bench), *map(str, args)], capture_output=True, text=True)


def test_arguments_and_exit_codes(bench, tmp_path):
    assert run(bench).returncode == 64
    for bad in (["--requests", "0"], ["--bytes", "1000"], ["--bytes", "0"],
                ["--operation", "erase"], ["--pattern", "zigzag"], ["--bogus", "1"],
                ["--requests"], ["--capacity-bytes", "512", "--bytes", "1024"],
                ["--requests", "x"], ["--bytes", str(1 << 33)],
                ["--requests", "3", "--arrival-gap-ns", str(2**63)]):
        p = run(bench, "--profile", NOMINAL, *bad)
        assert p.returncode == 64, (bad, p.stderr)
        assert p.stderr.startswith("hbf_media_bench: ")
    assert run(bench, "--profile", tmp_path / "missing.json").returncode == 70
    # writes need more than 10 blocks per plane (MQSim's garbage collector)
    prof = json.loads(NOMINAL.read_text())
    small = prof["page_bytes"] * prof["pages_per_block"] * prof["planes_per_die"] * \
        prof["dies_per_channel"] * prof["channels"] * 4
    p = run(bench, "--profile", NOMINAL, "--operation", "write", "--capacity-bytes", small)
    assert p.returncode == 64 and "blocks per plane" in p.stderr


def splitmix64(state: int):
    state = (state + 0x9E3779B97F4A7C15) & (2**64 - 1)
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
    return state, z ^ (z >> 31)


def workload(prof, requests, nbytes, operation, gap, pattern, seed, capacity):
    """Records of the bench's workload and each request's last record."""
    page = prof["page_bytes"]
    slots = capacity // nbytes
    state = seed
    rec, last = [], []
    for i in range(requests):
        if pattern == "random":
            state, v = splitmix64(state)
            slot = v % slots
        else:
            slot = i % slots
        write = operation == "write" or (operation == "mixed" and i % 2 == 1)
        addr, left = slot * nbytes, nbytes
        while left:
            piece = min(left, page - addr % page)
            rec.append((RANGE_BASE + addr, piece, i * gap * 1000, int(write)))
            addr += piece
            left -= piece
        last.append(len(rec) - 1)
    return np.array(rec, np.uint64), last


def oracle_report(raw, prof, args, capacity, depth):
    """The report's timing from the oracle's event loop (orc_engine_admission:
    the adapter's queue-depth admission and bandwidth cursor with the engine
    as the media port) over the regenerated workload."""
    rec, last = workload(raw, args["requests"], args["nbytes"], args["operation"], args["gap"],
                         args["pattern"], args["seed"], capacity)
    first = np.concatenate([[0], np.array(last, np.uint64) + 1]).astype(np.uint64)
    params = oracle_py.engine_params(prof)
    table, count = oracle_py.range_table([(RANGE_BASE, capacity, 3)], prof["page_bytes"],
                                         prof["capacity_bytes"])
    n = args["requests"]
    arrival = np.arange(n, dtype=np.uint64) * np.uint64(args["gap"])
    adm, dev, bounded = oracle_py.engine_admission(
        params, table, count, rec, first, arrival, np.full(n, args["nbytes"], np.uint64), depth,
        prof["aggregate_bandwidth_bytes_per_s"])
    lat = sorted(int(b) - int(a) for a, b in zip(arrival, bounded))
    pct = lambda q: lat[max(1, (q * len(lat) + 99) // 100) - 1]  # noqa: E731
    return adm, dev, bounded, lat, pct, int(bounded.max())


@pytest.mark.gpu
@pytest.mark.parametrize("args", [
    dict(requests=1024, nbytes=16384, operation="read", gap=0, pattern="sequential", seed=0),
    dict(requests=3000, nbytes=4096, operation="mixed", gap=50, pattern="random", seed=7),
    dict(requests=500, nbytes=65536, operation="read", gap=200, pattern="random", seed=3),
    dict(requests=2000, nbytes=1536, operation="write", gap=10, pattern="sequential", seed=0),
    dict(requests=700, nbytes=16384, operation="read", gap=0, pattern="random", seed=5, depth=4),
    dict(requests=300, nbytes=8192, operation="mixed", gap=700, pattern="random", seed=9,
         depth=1),
    dict(requests=1200, nbytes=32768, operation="read", gap=40, pattern="sequential", seed=0,
         depth=16)])
def test_report_matches_oracle(bench, args, tmp_path):
    """Every latency statistic, the modeled time and bandwidth equal the
    oracle's event loop; the nominal profile's queue depth (128) and smaller
    ones (16, 4 and 1) that make requests wait for earlier completions."""
    raw = json.loads(NOMINAL.read_text())
    path = NOMINAL
    if "depth" in args:
        raw["queue_depth"] = args["depth"]
        path = tmp_path / "nominal-qd.json"
        path.write_text(json.dumps(raw))
    prof = oracle_py.load_profile(path)
    depth = raw["queue_depth"]
    blocks16 = raw["page_bytes"] * raw["pages_per_block"] * raw["planes_per_die"] * \
        raw["dies_per_channel"] * raw["channels"] * 16
    capacity = min(raw["capacity_bytes"], blocks16)
    p = run(bench, "--profile", path, "--requests", args["requests"], "--bytes",
            args["nbytes"], "--operation", args["operation"], "--arrival-gap-ns", args["gap"],
            "--pattern", args["pattern"], "--seed", args["seed"])
    assert p.returncode == 0, p.stderr
    out = json.loads(p.stdout)
    assert list(out) == sorted(out)
    assert set(out) == {"effective_profile", "engine", "latency_ns",
                        "modeled_bandwidth_bytes_per_s", "profile", "queue_depth",
                        "queue_depth_applied", "requests", "schema_version",
                        "simulator_requests_per_s", "timing_ns", "workload"}
    assert out["engine"] == "hbf-amd-media-only" and out["queue_depth_applied"] is True
    assert out["queue_depth"] == depth
    assert out["effective_profile"]["capacity_bytes"] == capacity
    assert out["requests"] == {"submitted": args["requests"], "completed": args["requests"]}
    assert out["workload"] == {"operation": args["operation"], "pattern": args["pattern"],
                               "seed": args["seed"], "requests": args["requests"],
                               "bytes_per_request": args["nbytes"],
                               "arrival_gap_ns": args["gap"]}
    adm, dev, bounded, lat, pct, end = oracle_report(raw, prof, args, capacity, depth)
    if depth < args["requests"] and args["gap"] == 0:
        assert adm.max() > 0  # requests waited for slots
    assert out["timing_ns"]["modeled"] == end
    assert out["latency_ns"] == {"average": sum(lat) // len(lat), "p50": pct(50), "p99": pct(99)}
    expect = args["requests"] * args["nbytes"] * 1e9 / end
    assert out["modeled_bandwidth_bytes_per_s"] == pytest.approx(expect, rel=1e-12)
