"""The CPU oracle against the reference's compiled sources: committed golden
vectors (tests/golden/ref_vectors.json, written by tests/golden/make_golden.py)
and, when oracle/_ref/libhbfref.so was built in this container, fresh random
inputs checked live."""
from __future__ import annotations

import ctypes
import json
import pathlib

import numpy as np
import pytest

import oracle_py

GOLDEN = json.loads((pathlib.Path(__file__).parent / "golden" / "ref_vectors.json").read_text())


def table(ranges):
    recs = (oracle_py.OrcRange * len(ranges))()
    for i, r in enumerate(ranges):
        recs[i].base = r["base"]
        recs[i].length = r["length"]
        recs[i].file_offset = r["file_offset"]
        recs[i].range_id = r["range_id"]
        recs[i].mode = r["mode"]
        recs[i].permissions = r["permissions"]
        recs[i].page_bytes = r["page_bytes"]
    return recs


def test_fast_hash(oracle):
    for v, expect in GOLDEN["fast_hash"]:
        assert oracle.orc_fast_hash(v) == expect


def test_hybrid_reference_sample(oracle):
    for seq, warm, thr, key, expect in GOLDEN["hybrid_reference_sample"]:
        assert oracle.orc_hybrid_reference_sample(seq, warm, thr, key) == expect


def test_transfer_and_service(oracle):
    for b, bw, base, xfer, svc in GOLDEN["transfer_service"]:
        assert oracle.orc_fast_transfer_ns(b, bw) == xfer
        assert oracle.orc_fast_service_ns(base, b, bw) == svc


def test_host_mirror_equals_device_rule(oracle):
    # calibrator.cpp:33-65 is the host mirror of the device rule
    for rd, pg, bw, op, b, expect in GOLDEN["host_fast_service"]:
        assert oracle.orc_fast_service_ns(pg if op else rd, b, bw) == expect


def test_range_functions(oracle):
    for t in GOLDEN["range_tables"]:
        recs = table(t["ranges"])
        count = len(t["ranges"])
        for a, b, op, idx, sup, ovl, touch, md, lg, by in t["queries"]:
            assert oracle.orc_find_range_index(recs, count, a) == idx
            if idx < count:
                r = ctypes.byref(recs[idx])
                assert oracle.orc_access_supported(r, a, b, op) == sup
                assert oracle.orc_range_overlaps(r, a, b) == ovl
                m = oracle.orc_media_descriptor(r, a, b, op)
                assert m.valid == md
                if md:
                    assert (m.logical_address, m.bytes) == (lg, by)
            assert oracle.orc_span_touches_any_range(recs, count, a, b) == touch


def test_empirical_curve_and_burst(oracle):
    for e in GOLDEN["empirical"]:
        pa = (ctypes.c_uint32 * 6)(*e["pages"])
        ca = (ctypes.c_uint64 * 6)(*e["cumulative_ns"])
        for run, cum, svc in e["curve"]:
            assert oracle.orc_empirical_cumulative_ns(pa, ca, 6, run) == cum
            assert oracle.orc_empirical_service_ns(pa, ca, 6, run) == svc
        emp = oracle_py.OrcEmpirical()
        emp.flags, emp.point_count = 1, 6
        emp.pages[:] = e["pages"]
        emp.cumulative_ns[:] = e["cumulative_ns"]
        emp.program_latency_ns = e["program_ns"]
        for prev, page, op, ok, svc, packed, run in e["requests"]:
            s, pk, rn = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32()
            got = oracle.orc_empirical_request_service(ctypes.byref(emp), prev, page, op,
                                                       ctypes.byref(s), ctypes.byref(pk),
                                                       ctypes.byref(rn))
            assert got == ok
            if ok:
                assert (s.value, pk.value, rn.value) == (svc, packed, run)


def test_bank_layout(oracle):
    for lpa, ch, ncdu, nb, ok, c, d, b, chip, q, mod, ok2, lp in GOLDEN["bank_layout"]:
        assert ok and ok2
        oc, od, ob, ochip = (ctypes.c_uint32() for _ in range(4))
        oracle.orc_hbf_cold_read_bank(lpa, ch, ncdu, nb, ctypes.byref(oc), ctypes.byref(od),
                                      ctypes.byref(ob), ctypes.byref(ochip))
        assert (oc.value, od.value, ob.value, ochip.value) == (c, d, b, chip)
        assert oracle.orc_hbf_media_lpa(q, mod, ch) == lp


def test_page_register_two_slot_rule(oracle):
    for case in GOLDEN["pagebuf_two_slots"]:
        assert case["ok"] == 1
        pages = np.array(case["pages"], np.uint64)
        hits = np.zeros(len(pages), np.uint8)
        oracle.orc_pagebuf_sequence(pages.ctypes.data, len(pages), 2, hits.ctypes.data)
        assert hits.tolist() == case["hits"]


def thermal_step(oracle, case):
    n = len(case["capacity"])
    cap = np.array(case["capacity"])
    t = np.array(case["initial"])
    sp = np.array(case["static_power"])
    gb = np.array(case["boundary_g"])
    tb = np.array(case["boundary_t"])
    ea = np.array([e[0] for e in case["edges"]], np.uint32)
    eb = np.array([e[1] for e in case["edges"]], np.uint32)
    eg = np.array([e[2] for e in case["edges"]], np.float64)
    en = np.array(case["energy"])
    f = lambda a: a.ctypes.data  # noqa: E731
    for _ in range(case["steps"]):
        rc = oracle.orc_thermal_dense_step(n, f(cap), f(gb), f(tb), f(sp), ea.size,
                                           f(ea) if ea.size else None,
                                           f(eb) if eb.size else None,
                                           f(eg) if eg.size else None, case["dt"], f(en), f(t))
        assert rc == 0
    return t


def test_thermal_backward_euler(oracle):
    """Temperatures within 1e-4 K relative (the engine's thermal bar); in
    practice the dense restatement agrees to ~1e-13."""
    for case in GOLDEN["thermal"]:
        got = thermal_step(oracle, case)
        expect = np.array(case["temperature"])
        np.testing.assert_allclose(got, expect, rtol=1e-10, atol=0)


@pytest.mark.skipif(not oracle_py.ref_available(), reason="reference shim not built here")
def test_live_random_against_reference(oracle):
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).parent / "golden"))
    import make_golden
    ref = make_golden.bind(oracle_py.ref_lib())
    rng = np.random.default_rng()
    for v in make_golden.interesting_u64(rng, 500):
        assert oracle.orc_fast_hash(v) == ref.ref_fast_hash(v)
    for _ in range(2000):
        b = int(rng.integers(0, 2**32))
        bw = int(rng.integers(0, 2**44))
        base = int(rng.integers(0, 10**8))
        assert oracle.orc_fast_service_ns(base, b, bw) == ref.ref_fast_service_ns(base, b, bw)
    for _ in range(20):
        count = int(rng.integers(1, 12))
        recs = make_golden.random_table(rng, count)
        lo = recs[0].base - 0x3000
        hi = recs[count - 1].base + recs[count - 1].length + 0x3000
        for _ in range(300):
            a = int(rng.integers(max(0, lo), hi))
            b = int(rng.choice([0, 1, 8, 64, 0x1000, 0x3000]))
            op = int(rng.integers(0, 3))
            idx = ref.ref_find_range_index(recs, count, a)
            assert oracle.orc_find_range_index(recs, count, a) == idx
            assert (oracle.orc_span_touches_any_range(recs, count, a, b) ==
                    ref.ref_span_touches_any_range(recs, count, a, b))
            if idx < count:
                r = ctypes.byref(recs[idx])
                assert oracle.orc_access_supported(r, a, b, op) == \
                    ref.ref_access_supported(r, a, b, op)
    for _ in range(50):
        n = int(rng.integers(1, 300))
        pages = rng.integers(0, int(rng.integers(1, 8)), n).astype(np.uint64)
        h1 = np.zeros(n, np.uint8)
        h2 = np.zeros(n, np.uint8)
        assert ref.ref_pagebuf_sequence(pages.ctypes.data, n, h1.ctypes.data) == 1
        oracle.orc_pagebuf_sequence(pages.ctypes.data, n, 2, h2.ctypes.data)
        assert h1.tolist() == h2.tolist()
