"""The hbf_trace_timing drop-in (hbfsim_amd/hbf_trace_timing) against the
CPU restatement of the reference's fast loop (hbf_trace_timing.cpp:181-233)
and the reference's argument and exit-code contract (:40-66, 92-121,
264-269).  Events are written the way the reference's caller writes them
(adapters/vllm_capacity/trace_replay.py:218-238)."""
from __future__ import annotations

import ctypes
import json
import math
import pathlib
import subprocess

import numpy as np
import pytest

import oracle_py

ROOT = pathlib.Path(__file__).resolve().parent.parent
CLI = ROOT / "hbfsim_amd" / "hbf_trace_timing"
PROFILES = ROOT / "tests" / "golden" / "profiles"


@pytest.fixture(scope="module")
def cli():
    if not CLI.exists():
        from hbfsim_amd import build
        build.build_cli()
    return CLI


def run(cli, *args):
    return subprocess.run([str(cli), *map(str, args)], capture_output=True, text=True)


def write_events(path, events):
    lines = []
    for seq, (addr, nbytes, page, op) in enumerate(events, start=1):
        lines.append(json.dumps({"schema_version": 1, "sequence": seq, "logical_address": addr,
                                 "bytes": nbytes, "page_bytes": page, "operation": op},
                                sort_keys=True, separators=(",", ":")) + "\n")
    path.write_text("".join(lines))


def oracle_loop(events, prof):
    ev = (oracle_py.OrcTraceEvent * len(events))()
    for i, (addr, nbytes, page, op) in enumerate(events):
        ev[i].logical_address, ev[i].bytes, ev[i].page_bytes = addr, nbytes, page
        ev[i].operation = 1 if op == "write" else 0
    sub, svc, clk = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    rc = oracle_py.lib().orc_trace_timing_fast(
        ev, len(events), prof["read_latency_ns"], prof["program_latency_ns"],
        prof["aggregate_bandwidth_bytes_per_s"], prof["page_bytes"], prof["capacity_bytes"],
        ctypes.byref(sub), ctypes.byref(svc), ctypes.byref(clk))
    return rc, sub.value, svc.value, clk.value


@pytest.mark.parametrize("name", ["nominal", "aggressive", "conservative"])
def test_fast_mode_matches_restatement(cli, tmp_path, name):
    prof = json.loads((PROFILES / f"{name}.json").read_text())
    page = prof["page_bytes"]
    rng = np.random.default_rng(len(name))
    events = []
    for _ in range(300):
        pages = int(rng.integers(1, 40))
        addr = int(rng.integers(0, prof["capacity_bytes"] // page - pages)) * page
        events.append((addr, pages * page, page, "write" if rng.random() < 0.2 else "read"))
    ev_path = tmp_path / "events.jsonl"
    write_events(ev_path, events)
    p = run(cli, "--profile", PROFILES / f"{name}.json", "--events", ev_path, "--mode", "fast")
    assert p.returncode == 0, p.stderr
    out = json.loads(p.stdout)
    rc, sub, svc, clk = oracle_loop(events, prof)
    assert rc == 0
    assert out["status"] == "PASS" and out["engine"] == "hbf-fast" and out["schema_version"] == 1
    assert out["profile"] == prof["name"]
    assert out["requests"] == {"input_expert_misses": len(events), "submitted": sub,
                               "fast": sub, "reference": 0}
    assert out["modeled_device_service_ns"] == svc
    assert out["demand_exposed_stall_ns"] == clk
    assert out["reference_sample_rate"] == prof["reference_sample_rate"]
    assert out["reference_warmup_requests"] == prof["reference_warmup_requests"]
    assert out["scheduling_semantics"] == "ordered blocking demand misses with no compute gaps"
    # nlohmann::json dump(2) layout: sorted keys, two-space indent
    assert list(out) == sorted(out) and list(out["requests"]) == sorted(out["requests"])
    assert p.stdout.startswith('{\n  "demand_exposed_stall_ns": ')
    assert '\n    "fast": ' in p.stdout and p.stdout.endswith('  "status": "PASS"\n}\n')


def test_trace_replay_contract(cli, tmp_path):
    """What run_timing_engine checks: PASS, misses, and pages submitted =
    misses x ceil(expert bytes / page)."""
    prof = json.loads((PROFILES / "nominal.json").read_text())
    page = prof["page_bytes"]
    expert_bytes = 3 * 2048 * 1024 * 2 + 1000
    slot = math.ceil(expert_bytes / page) * page
    misses = [(l_, e) for l_ in range(2) for e in (3, 17, 40)]
    events = [((l_ * 64 + e) * slot, slot, page, "read") for l_, e in misses]
    ev_path = tmp_path / "ev.jsonl"
    write_events(ev_path, events)
    p = run(cli, "--profile", PROFILES / "nominal.json", "--events", ev_path, "--mode", "fast")
    assert p.returncode == 0, p.stderr
    out = json.loads(p.stdout)
    assert out["requests"]["input_expert_misses"] == len(misses)
    assert out["requests"]["submitted"] == len(misses) * math.ceil(expert_bytes / page)


def test_exit_codes(cli, tmp_path):
    nominal = PROFILES / "nominal.json"
    good = tmp_path / "good.jsonl"
    write_events(good, [(0, 16384, 16384, "read")])
    # usage errors: std::invalid_argument -> 64
    assert run(cli).returncode == 64
    assert run(cli, "--profile", nominal, "--events").returncode == 64
    assert run(cli, "--profile", nominal, "--events", good, "--mode", "slow").returncode == 64
    assert run(cli, "--profile", nominal, "--bogus", good, "--mode", "fast").returncode == 64
    # MQSim is not part of this build -> 2
    p = run(cli, "--profile", nominal, "--events", good, "--mode", "mqsim")
    assert p.returncode == 2 and "MQSim" in p.stderr
    # hybrid mode samples on the GPU: without one it fails with 2
    p = run(cli, "--profile", nominal, "--events", good, "--mode", "hybrid")
    assert p.returncode == 0 or (p.returncode == 2 and "GPU" in p.stderr)
    # profile and file errors -> 2
    assert run(cli, "--profile", tmp_path / "nope.json", "--events", good,
               "--mode", "fast").returncode == 2
    assert run(cli, "--profile", nominal, "--events", tmp_path / "nope.jsonl",
               "--mode", "fast").returncode == 2
    bad_json = tmp_path / "bad.jsonl"
    bad_json.write_text("{not json\n")
    assert run(cli, "--profile", nominal, "--events", bad_json, "--mode", "fast").returncode == 2
    # invalid events -> 64
    cases = {
        "gap": [(0, 16384, 16384, "read"), (16384, 16384, 16384, "read")],
        "misaligned": [(512, 16384, 16384, "read")],
        "page size": [(0, 8192, 8192, "read")],
        "ragged": [(0, 16384 + 512, 16384, "read")],
        "operation": [(0, 16384, 16384, "erase")],
        "capacity": [(1 << 50, 16384, 16384, "read")],
    }
    for label, events in cases.items():
        path = tmp_path / f"{label.replace(' ', '_')}.jsonl"
        write_events(path, events)
        if label == "gap":
            lines = path.read_text().splitlines()
            lines[1] = lines[1].replace('"sequence":2', '"sequence":3')
            path.write_text("\n".join(lines) + "\n")
        p = run(cli, "--profile", nominal, "--events", path, "--mode", "fast")
        assert p.returncode == 64, (label, p.returncode, p.stderr)
    # blank lines are skipped
    blank = tmp_path / "blank.jsonl"
    write_events(blank, [(0, 16384, 16384, "read"), (16384, 16384, 16384, "write")])
    blank.write_text(blank.read_text().replace("\n", "\n\n", 1))
    p = run(cli, "--profile", nominal, "--events", blank, "--mode", "fast")
    assert p.returncode == 0 and json.loads(p.stdout)["requests"]["submitted"] == 2


def test_reference_known_answers(cli, tmp_path):
    """Known answers of the reference's own CLI tests on the nominal profile:
    one 32,768-byte read event over 16,384-byte pages is two page requests,
    each max(10,000 ns first-byte latency, 32 ns transfer)
    (tests/integration/test_trace_timing.py:14-68); three one-page misses cost
    30,000 ns (tests/integration/test_trace_replay_timing.py:131-134)."""
    nominal = PROFILES / "nominal.json"
    one = tmp_path / "one.jsonl"
    one.write_text(json.dumps({"schema_version": 1, "sequence": 1, "logical_address": 0,
                               "bytes": 32_768, "page_bytes": 16_384,
                               "operation": "read"}) + "\n")
    p = run(cli, "--profile", nominal, "--events", one, "--mode", "fast")
    assert p.returncode == 0, p.stderr
    out = json.loads(p.stdout)
    assert out["status"] == "PASS" and out["engine"] == "hbf-fast"
    assert out["requests"] == {"input_expert_misses": 1, "submitted": 2, "fast": 2,
                               "reference": 0}
    assert out["modeled_device_service_ns"] == 20_000
    assert out["demand_exposed_stall_ns"] == 20_000
    assert out["emulator_dispatcher_wall_time_ns"] > 0
    three = tmp_path / "three.jsonl"
    write_events(three, [(e * 16_384, 16_384, 16_384, "read") for e in (0, 1, 0)])
    p = run(cli, "--profile", nominal, "--events", three, "--mode", "fast")
    assert p.returncode == 0, p.stderr
    out = json.loads(p.stdout)
    assert out["requests"]["submitted"] == 3
    assert out["modeled_device_service_ns"] == 30_000
