"""Profile loading and validation through the C ABI, mirroring the
reference's tests/cpu/profile_test.cpp (same inputs, same messages)."""
from __future__ import annotations

import json
import pathlib

import pytest

from hbfsim_amd import engine as eng

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "profiles"


def write(tmp_path, doc, name="p.json"):
    p = tmp_path / name
    p.write_text(json.dumps(doc))
    return str(p)


@pytest.mark.parametrize("name", ["nominal", "aggressive", "conservative", "cd8p-vmem-p50"])
def test_reference_profiles_load(name):
    assert eng.validate_profile(str(GOLDEN / f"{name}.json")) is None


def nominal():
    return json.loads((GOLDEN / "nominal.json").read_text())


def tuned():
    return json.loads((GOLDEN / "cd8p-vmem-p50.json").read_text())


CASES = [
    (nominal, lambda d: d.update(page_bytes=12288), "page_bytes must be a power of two"),
    (nominal, lambda d: d.update(page_bytes=256),
     "page_bytes must be at least 512 for MQSim sector alignment"),
    (nominal, lambda d: d.update(capacity_bytes=0), "capacity_bytes must be greater than zero"),
    (nominal, lambda d: d.update(reference_sample_rate=-0.01),
     "reference_sample_rate must be in [0, 1]"),
    (nominal, lambda d: d.update(reference_sample_rate=1.01),
     "reference_sample_rate must be in [0, 1]"),
    (nominal, lambda d: d.update(hbm_cache_bytes=d["capacity_bytes"] + 1),
     "hbm_cache_bytes must not exceed capacity_bytes"),
    (nominal, lambda d: d.update(capacity_bytes=d["capacity_bytes"] - d["page_bytes"]),
     "capacity geometry must contain an integral number of blocks per plane"),
    (nominal, lambda d: d.update(read_latency_ns=0), "read_latency_ns must be greater than zero"),
    (nominal, lambda d: d.update(program_latency_ns=0),
     "program_latency_ns must be greater than zero"),
    (nominal, lambda d: d.update(channels=0), "channels must be greater than zero"),
    (nominal, lambda d: d.update(queue_depth=0), "queue_depth must be greater than zero"),
    (nominal, lambda d: d.update(time_scale=0), "time_scale must be greater than zero"),
    (nominal, lambda d: d.update(aggregate_bandwidth_bytes_per_s=0),
     "aggregate_bandwidth_bytes_per_s must be greater than zero"),
    (nominal, lambda d: d.update(page_read_latency_msb_ns=0),
     "per-level page read/program latencies must be greater than zero"),
    (nominal, lambda d: d.update(nand_technology="PLC"),
     "nand_technology must be one of SLC, MLC, TLC, QLC"),
    (nominal, lambda d: d.update(plane_allocation_scheme="CCDP"),
     "plane_allocation_scheme must be one of the 24 channel/way/die/plane orderings, e.g. CWDP"),
    (tuned, lambda d: d.update(page_bytes=16384), "empirical_vmem requires page_bytes == 4096"),
    (tuned, lambda d: d["empirical_vmem"].update(source_sha256="invalid"),
     "empirical_vmem source_sha256 must be lowercase hexadecimal SHA256"),
    (tuned, lambda d: d["empirical_vmem"]["read_curve"][1].update(pages=1),
     "empirical_vmem pages must be strictly increasing"),
    (tuned, lambda d: d["empirical_vmem"]["read_curve"][1].update(cumulative_ns=11133),
     "empirical_vmem P50 latency must be strictly increasing"),
    (tuned, lambda d: d["empirical_vmem"]["read_curve"][0].update(p95_ns=1),
     "empirical_vmem P95 latency must not be below P50"),
    (tuned, lambda d: d["empirical_vmem"].update(quantile="p95"),
     "empirical_vmem quantile must be p50"),
    (tuned, lambda d: d["empirical_vmem"]["read_curve"].pop(),
     "empirical_vmem read_curve must contain exactly 6 points"),
    (tuned, lambda d: d["empirical_vmem"].update(program_p95_ns=1),
     "empirical_vmem program P95 must not be below P50"),
]


@pytest.mark.parametrize("base,mutate,message", CASES)
def test_validation_messages(tmp_path, base, mutate, message):
    doc = base()
    mutate(doc)
    assert eng.validate_profile(write(tmp_path, doc)) == message


def test_missing_key_and_bad_json(tmp_path):
    doc = nominal()
    del doc["queue_depth"]
    msg = eng.validate_profile(write(tmp_path, doc))
    assert msg.startswith("invalid profile JSON:") and "queue_depth" in msg
    p = tmp_path / "broken.json"
    p.write_text('{"name": "x",')
    assert eng.validate_profile(str(p)).startswith("invalid profile JSON:")
    assert eng.validate_profile(str(tmp_path / "absent.json")).startswith(
        "could not open profile:")


def test_allocation_scheme_and_defaults(tmp_path):
    doc = nominal()
    doc["plane_allocation_scheme"] = "PDWC"
    doc["nand_technology"] = "QLC"
    assert eng.validate_profile(write(tmp_path, doc)) is None
