"""The C-ABI library: loads, exports exactly what include/hbfsim_amd.h
declares, and behaves like the reference's API on every path that needs no
GPU (argument validation, registry semantics, error codes, vLLM session)."""
from __future__ import annotations

import ctypes
import json
import pathlib
import re
import subprocess

import pytest

from hbfsim_amd import _native as nat
from hbfsim_amd import engine as eng
from hbfsim_amd import workloads

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "hbfsim_amd.h"
C0 = str(workloads.PROFILES / "c0.json")


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*"
                          r"(hbfsim_[a-z0-9_]+)\s*\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    names = declared_functions()
    assert len(names) >= 29
    for name in names:
        assert hasattr(lib, name), name
    assert names == set(nat.SIGNATURES), "binding and header disagree"
    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert names <= exported
    assert {n for n in exported if n.startswith("hbfsim")} == names


def test_versions_and_status_strings():
    lib = nat.load()
    assert lib.hbfsim_abi_version() == 1            # src/api.cpp:3-6
    assert lib.hbfsim_vllm_abi_version() == 2       # hbfsim_extension.cpp:13-16
    names = ["ok", "invalid_argument", "io_error", "cuda_error", "timeout", "unsupported",
             "daemon_lost", "unknown"]
    for code, name in enumerate(names):
        assert lib.hbfsim_vllm_status_string(code).decode() == name
    assert lib.hbfsim_vllm_status_string(-1).decode() == "unknown"


def create(profile=C0, report="/tmp/hbfsim-abi", mode=1, ring=64, timeout=10**9):
    lib = nat.load()
    h = ctypes.c_void_p(12345)
    o = nat.Options(profile.encode() if profile else None, report.encode() if report else None,
                    mode, ring, timeout)
    rc = lib.hbfsim_context_create(ctypes.byref(o), ctypes.byref(h))
    return rc, h


def test_context_create_validation(tmp_path):
    lib = nat.load()
    assert lib.hbfsim_context_create(None, None) == nat.HBFSIM_INVALID_ARGUMENT
    # out-pointer nulled before validation (context.cpp:867-870)
    rc, h = create(profile=None)
    assert rc == nat.HBFSIM_INVALID_ARGUMENT and not h.value
    for kw in (dict(report=""), dict(mode=3), dict(ring=3), dict(ring=1), dict(ring=8192),
               dict(timeout=0)):
        assert create(**kw)[0] == nat.HBFSIM_INVALID_ARGUMENT, kw
    assert create(profile=str(tmp_path / "missing.json"))[0] == nat.HBFSIM_INVALID_ARGUMENT
    bad = tmp_path / "bad.json"
    bad.write_text("{not json")
    assert create(profile=str(bad))[0] == nat.HBFSIM_INVALID_ARGUMENT
    # reference mode needs the MQSim daemon
    assert create(mode=0)[0] == nat.HBFSIM_UNSUPPORTED
    blocker = tmp_path / "file"
    blocker.write_text("x")
    assert create(report=str(blocker / "sub"))[0] == nat.HBFSIM_IO_ERROR
    rc, h = create(report=str(tmp_path / "r"), mode=2, ring=4096)
    assert rc == 0 and h.value
    lib.hbfsim_context_destroy(h)
    lib.hbfsim_context_destroy(None)


def test_registry_semantics(tmp_path):
    """range_table_test.cpp expectations through the C ABI: sorted insert,
    cumulative page-rounded media offsets, overlap and argument checks."""
    e = eng.Engine(C0, str(tmp_path))
    e.register(0x3000, 0x1000, nat.HBFSIM_RANGE_READ)
    e.register(0x1000, 0x1000, nat.HBFSIM_RANGE_READ_WRITE)
    kind, r = e.lookup(0x1000, 4)
    assert kind == "matched" and r["permissions"] == 3 and r["file_offset"] == 16384
    assert r["page_bytes"] == 16384
    kind, r2 = e.lookup(0x3000, 4)
    assert r2["file_offset"] == 0 and r2["range_id"] != r["range_id"]
    assert e.lookup(0x1FFF, 1)[0] == "matched"
    assert e.lookup(0x2000, 1)[0] == "outside"
    assert e.lookup(0x1FFF, 2)[0] == "crosses"
    assert e.lookup(2**64 - 1, 2)[0] == "outside"
    lib = nat.load()
    ro = lambda m=1, p=3, c=0: nat.RangeOptions(m, p, c, 0)  # noqa: E731
    reg = lambda b, n, o: lib.hbfsim_register_device(e.handle, ctypes.c_void_p(b), n,  # noqa
                                                     ctypes.byref(o))
    assert reg(0x1800, 0x1000, ro()) == nat.HBFSIM_INVALID_ARGUMENT   # overlap
    assert reg(2**64 - 8, 9, ro()) == nat.HBFSIM_INVALID_ARGUMENT      # wraps
    assert reg(0x9000, 0x10, ro(m=2)) == nat.HBFSIM_UNSUPPORTED        # capacity mode
    assert reg(0x9000, 0x10, ro(m=99)) == nat.HBFSIM_INVALID_ARGUMENT
    assert reg(0x9000, 0x10, ro(p=0)) == nat.HBFSIM_INVALID_ARGUMENT
    assert reg(0x9000, 0x10, ro(p=4)) == nat.HBFSIM_INVALID_ARGUMENT
    assert reg(0x9000, 0x10, ro(c=1)) == nat.HBFSIM_INVALID_ARGUMENT
    assert reg(0x9000, 0, ro()) == nat.HBFSIM_INVALID_ARGUMENT
    assert lib.hbfsim_register_device(e.handle, None, 16, ctypes.byref(ro())) == 1
    assert reg(0x10_0000, 1 << 37, ro()) == nat.HBFSIM_UNSUPPORTED   # beyond capacity
    e.unregister(0x1000)
    assert e.lookup(0x1000, 1)[0] == "outside"
    with pytest.raises(nat.HbfSimError):
        e.unregister(0x1000)
    e.close()


def test_range_capacity(tmp_path):
    """The table holds 32,768 ranges (hbf_device.cuh:21); the next
    registration is refused with HBFSIM_UNSUPPORTED and leaves the table as
    it was; removing one range makes room again."""
    e = eng.Engine(C0, str(tmp_path))
    base, page = 0x5000_0000_0000, 16384
    for r in range(32768):
        e.register(base + 2 * r * page, page, nat.HBFSIM_RANGE_READ)
    lib = nat.load()
    o = nat.RangeOptions(nat.HBFSIM_RANGE_MODE_TIMING, nat.HBFSIM_RANGE_READ, 0, 0)
    extra = base + 2 * 32768 * page
    assert lib.hbfsim_register_device(e.handle, ctypes.c_void_p(extra), page,
                                      ctypes.byref(o)) == nat.HBFSIM_UNSUPPORTED
    assert e.lookup(extra)[0] == "outside"
    assert e.lookup(base + 2 * 32767 * page)[0] == "matched"
    e.unregister(base)
    assert lib.hbfsim_register_device(e.handle, ctypes.c_void_p(extra), page,
                                      ctypes.byref(o)) == 0
    e.close()


def test_map_file_and_capacity_stats(tmp_path):
    e = eng.Engine(C0, str(tmp_path))
    lib = nat.load()
    out = ctypes.c_void_p(99)
    cap = nat.RangeOptions(2, 1, 0, 0)
    assert lib.hbfsim_map_file(e.handle, b"/x", 0, 4096, ctypes.byref(cap),
                               ctypes.byref(out)) == nat.HBFSIM_UNSUPPORTED
    assert not out.value
    timing = nat.RangeOptions(1, 1, 0, 0)
    assert lib.hbfsim_map_file(e.handle, b"/x", 0, 4096, ctypes.byref(timing),
                               ctypes.byref(out)) == nat.HBFSIM_UNSUPPORTED
    bad = nat.RangeOptions(2, 2, 0, 0)
    assert lib.hbfsim_map_file(e.handle, b"/x", 0, 4096, ctypes.byref(bad),
                               ctypes.byref(out)) == nat.HBFSIM_INVALID_ARGUMENT
    assert lib.hbfsim_map_file(e.handle, b"", 0, 4096, ctypes.byref(cap),
                               ctypes.byref(out)) == nat.HBFSIM_INVALID_ARGUMENT
    cs = nat.CapacityStats()
    assert lib.hbfsim_get_capacity_stats_v1(e.handle, ctypes.byref(cs)) == 0
    assert cs.enabled == 0 and cs.version == 1 and cs.struct_size == ctypes.sizeof(cs)
    assert e.stats() == {"requests_submitted": 0, "requests_completed": 0, "fast_requests": 0,
                         "reference_requests": 0, "fast_modeled_ns": 0}
    e.close()


def test_vllm_session_lifecycle(tmp_path):
    lib = nat.load()
    h = ctypes.c_void_p(7)
    o = nat.VllmOptions(C0.encode(), str(tmp_path).encode(), 64, 2, 10**9)
    assert lib.hbfsim_vllm_session_create(None, ctypes.byref(h)) == 1 and not h.value
    bad = nat.VllmOptions(C0.encode(), str(tmp_path).encode(), 0, 2, 10**9)
    assert lib.hbfsim_vllm_session_create(ctypes.byref(bad), ctypes.byref(h)) == 1
    bad = nat.VllmOptions(C0.encode(), str(tmp_path).encode(), 64, 3, 10**9)
    assert lib.hbfsim_vllm_session_create(ctypes.byref(bad), ctypes.byref(h)) == 1
    assert lib.hbfsim_vllm_session_create(ctypes.byref(o), ctypes.byref(h)) == 0 and h.value
    assert lib.hbfsim_vllm_register_storage(h, 0x10000, 4096) == 0
    assert lib.hbfsim_vllm_register_storage(h, 0x10800, 4096) == nat.HBFSIM_INVALID_ARGUMENT
    assert lib.hbfsim_vllm_register_storage(h, 0, 4096) == nat.HBFSIM_INVALID_ARGUMENT
    assert lib.hbfsim_vllm_register_storage(None, 0x20000, 4096) == 1
    ctx = lib.hbfsim_vllm_session_context(h)
    assert ctx
    kind, rng = ctypes.c_uint32(), nat.Range()
    assert lib.hbfsim_amd_lookup_range(ctx, 0x10000, 8, ctypes.byref(kind), ctypes.byref(rng),
                                       None) == 0
    assert kind.value == 1 and rng.permissions == nat.HBFSIM_RANGE_READ and rng.mode == 1
    assert lib.hbfsim_vllm_session_close(ctypes.byref(h)) == 0 and not h.value
    assert lib.hbfsim_vllm_session_close(ctypes.byref(h)) == 0
    assert lib.hbfsim_vllm_session_close(None) == nat.HBFSIM_INVALID_ARGUMENT


def test_engine_options_validation(tmp_path):
    e = eng.Engine(C0, str(tmp_path))
    assert e.options()["page_buffers"] == 1 and e.options()["model"] == nat.MODEL_HBF
    assert e.geometry() == (8, 64)
    e.set_options(ways=2)
    assert e.geometry() == (8, 128)
    e.set_options(flat_geometry=1)
    assert e.geometry() == (1, 1)
    for bad in (dict(page_buffers=3), dict(tile_records=100), dict(model=2),
                dict(model=nat.MODEL_EMPIRICAL)):
        with pytest.raises(nat.HbfSimError):
            e.set_options(**bad)
    lib = nat.load()
    o = nat.EngineOptions()
    assert lib.hbfsim_amd_set_engine_options(e.handle, ctypes.byref(o)) == 1  # struct_size 0
    e.close()
    emp = ROOT / "tests" / "golden" / "profiles" / "cd8p-vmem-p50.json"
    e = eng.Engine(str(emp), str(tmp_path))
    assert e.options()["model"] == nat.MODEL_EMPIRICAL
    e.close()


def test_run_arguments_without_gpu(tmp_path):
    """Argument checks happen before any device work."""
    lib = nat.load()
    e = eng.Engine(C0, str(tmp_path))
    rep = nat.Report()
    assert lib.hbfsim_amd_run_device(None, None, 0, None, None, 0, None,
                                     ctypes.byref(rep)) == 1
    assert lib.hbfsim_amd_run_device(e.handle, None, 4, None, None, 0, None,
                                     ctypes.byref(rep)) == 1
    assert lib.hbfsim_amd_run(e.handle, None, 4, None, None, 0, ctypes.byref(rep)) == 1
    e.close()


def test_report_written_on_flush(tmp_path):
    e = eng.Engine(C0, str(tmp_path / "rep"))
    assert (tmp_path / "rep").is_dir()  # created like the reference (context.cpp:892-896)
    e.close()


def test_profiles_are_reference_schema():
    """Config profiles use only the reference schema's keys."""
    keys = {"name", "capacity_bytes", "page_bytes", "read_latency_ns", "program_latency_ns",
            "channels", "dies_per_channel", "planes_per_die", "pages_per_block",
            "channel_width_bits", "channel_transfer_rate_mtps", "queue_depth",
            "aggregate_bandwidth_bytes_per_s", "hbm_cache_bytes", "reference_sample_rate",
            "reference_warmup_requests", "time_scale", "timing_tolerance_ns"}
    for p in workloads.PROFILES.glob("*.json"):
        assert set(json.loads(p.read_text())) <= keys | {"plane_allocation_scheme",
                                                        "nand_technology"}, p
        assert eng.validate_profile(str(p)) is None
