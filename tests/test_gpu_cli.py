"""hbf_trace_timing --mode hybrid: the page requests the reference's replay
sends to MQSim (hbf_trace_timing.cpp:196-213: HybridSampler(warmup, rate,
0).reference(sequence - 1, access)) are picked by the library's GPU sampler
and timed by the library's engine in MQSim's place: the request arrives at
the demand clock, and its completion becomes the clock.  The count must equal
the CPU oracle's sampler over the same request sequence, and both clocks the
replay recomputed here with the oracle's engine (state carried from one
picked request to the next) for the picked requests and the fast model's
arithmetic for the others."""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle_py
from test_cli import PROFILES, cli, run, write_events  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["nominal", "aggressive", "conservative"])
def test_hybrid_mode_counts_sampled_requests(cli, tmp_path, name):  # noqa: F811
    path = PROFILES / f"{name}.json"
    prof = json.loads(path.read_text())
    page = prof["page_bytes"]
    rng = np.random.default_rng(3 + len(name))
    events = []
    for _ in range(2000):
        pages = int(rng.integers(1, 30))
        addr = int(rng.integers(0, prof["capacity_bytes"] // page - pages)) * page
        events.append((addr, pages * page, page, "write" if rng.random() < 0.3 else "read"))
    ev_path = tmp_path / "events.jsonl"
    write_events(ev_path, events)
    fast = run(cli, "--profile", path, "--events", ev_path, "--mode", "fast")
    hyb = run(cli, "--profile", path, "--events", ev_path, "--mode", "hybrid")
    assert fast.returncode == 0 and hyb.returncode == 0, hyb.stderr
    f, h = json.loads(fast.stdout), json.loads(hyb.stdout)
    access = []
    for _, nbytes, pg, op in events:
        access += [(1 if op == "write" else 0, pg, 0, 0)] * (nbytes // pg)
    flags = oracle_py.sampler_run(prof["reference_warmup_requests"],
                                  prof["reference_sample_rate"], 0, np.array(access),
                                  np.arange(len(access), dtype=np.uint64))
    ref = int(flags.sum())
    assert 0 < ref < len(access)
    assert h["engine"] == "hbf-hybrid" and h["status"] == "PASS"
    assert h["requests"] == {"input_expert_misses": len(events), "submitted": len(access),
                             "fast": len(access) - ref, "reference": ref}
    assert h["reference_timing"].startswith("hbf-amd-engine")
    for k in ("profile", "reference_sample_rate", "reference_warmup_requests",
              "scheduling_semantics"):
        assert h[k] == f[k], k
    clock, service = replay(prof, path, events, flags)
    assert h["demand_exposed_stall_ns"] == clock
    assert h["modeled_device_service_ns"] == service
    assert list(h) == sorted(h)


def replay(prof, path, events, flags):
    """The hybrid replay (hbf_trace_timing.cpp:181-233) with the oracle's
    engine standing in for MQSim on the picked requests."""
    o = oracle_py.load_profile(path)
    params = oracle_py.engine_params(o)
    base = 0x4000_0000_0000
    table, count = oracle_py.range_table([(base, o["capacity_bytes"], 3)], o["page_bytes"],
                                         o["capacity_bytes"])
    state = oracle_py.OracleState(params)
    bw = o["aggregate_bandwidth_bytes_per_s"]
    clock = service = 0
    k = 0
    for addr, nbytes, pg, op in events:
        write = op == "write"
        lat = o["program_latency_ns"] if write else o["read_latency_ns"]
        xfer = -(-pg * 10**9 // bw)
        for p in range(nbytes // pg):
            if flags[k]:
                rec = np.array([[base + addr + p * pg, pg, clock * 1000, int(write)]], np.uint64)
                comp, st, _, _ = oracle_py.run(params, table, count, rec, 0, state)
                assert st[0] & 3 == 0
                done = -(-int(comp[0]) // 1000)
                service += done - clock
                clock = done
            else:
                service += max(lat, xfer)
                clock += max(lat, xfer)
            k += 1
    return clock, service


def test_hybrid_reference_known_answer(cli, tmp_path):  # noqa: F811
    """tests/integration/test_trace_timing.py:69-77 of the reference: in hybrid
    mode the two page requests of one event fall inside the sampler's warm-up,
    so both are reference requests and none is fast."""
    one = tmp_path / "one.jsonl"
    write_events(one, [(0, 32_768, 16_384, "read")])
    p = run(cli, "--profile", PROFILES / "nominal.json", "--events", one, "--mode", "hybrid")
    assert p.returncode == 0, p.stderr
    h = json.loads(p.stdout)
    assert h["status"] == "PASS" and h["engine"] == "hbf-hybrid"
    assert h["requests"] == {"input_expert_misses": 1, "submitted": 2, "fast": 0,
                             "reference": 2}
    assert h["modeled_device_service_ns"] > 0 and h["demand_exposed_stall_ns"] > 0
    assert h["emulator_dispatcher_wall_time_ns"] > 0
