"""Writes tests/golden/ref_vectors.json from the reference's own compiled
sources (oracle/_ref/libhbfref.so, built by `make -C oracle ref` in the
container that holds the reference tree).

The vectors are inputs and the reference's outputs only; they pin the CPU
oracle where the reference's unit tests leave cases open.  Run:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import oracle_py  # noqa: E402

U64 = ctypes.c_uint64
U32 = ctypes.c_uint32
P = ctypes.c_void_p


def bind(ref):
    sig = {
        "ref_fast_hash": (U64, [U64]),
        "ref_hybrid_reference_sample": (ctypes.c_int, [U64, U32, U64, U64]),
        "ref_fast_transfer_ns": (U64, [U32, U64]),
        "ref_fast_service_ns": (U64, [U64, U32, U64]),
        "ref_host_fast_service_ns": (U64, [U64, U64, U64, U32, U32]),
        "ref_find_range_index": (U32, [P, U32, U64]),
        "ref_access_supported": (ctypes.c_int, [P, U64, U32, U32]),
        "ref_range_overlaps": (ctypes.c_int, [P, U64, U32]),
        "ref_span_touches_any_range": (ctypes.c_int, [P, U32, U64, U32]),
        "ref_media_descriptor": (ctypes.c_int, [P, U64, U32, U32, P, P]),
        "ref_empirical_cumulative_ns": (U64, [P, P, U32, U32]),
        "ref_empirical_service_ns": (U64, [P, P, U32, U32]),
        "ref_update_empirical_burst": (ctypes.c_int, [U64, U64, U32, P, P]),
        "ref_empirical_request_service": (ctypes.c_int, [P, P, U64, U64, U64, U32, P, P, P]),
        "ref_cold_read_bank": (ctypes.c_int, [U64, U32, U32, U32, P, P, P, P]),
        "ref_hbf_media_lpa": (ctypes.c_int, [U64, U32, U32, P]),
        "ref_pagebuf_sequence": (ctypes.c_int, [P, ctypes.c_size_t, P]),
        "ref_thermal_step": (ctypes.c_int, [ctypes.c_size_t, P, P, P, P, P, ctypes.c_size_t, P,
                                            P, P, P, U32, ctypes.c_double, P]),
        "ref_simulate_prefetch": (ctypes.c_int, [P, ctypes.c_size_t, U32, ctypes.c_double, U32,
                                                 U32, U32, U64, U64, U64, P]),
        "ref_sampler_run": (ctypes.c_int, [U32, ctypes.c_double, U64, P, P, ctypes.c_size_t,
                                           P]),
        "ref_calibrate": (ctypes.c_int, [P, P, ctypes.c_size_t, P, P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(ref, name)
        f.restype = res
        f.argtypes = args
    return ref


def interesting_u64(rng, n):
    edge = [0, 1, 2, 63, 64, 4095, 4096, 2**31, 2**32 - 1, 2**32, 2**53, 2**63 - 1, 2**63,
            2**64 - 2, 2**64 - 1]
    vals = list(edge) + [int(x) for x in rng.integers(0, 2**63, n, dtype=np.uint64)]
    vals += [int(x) << 1 | 1 for x in rng.integers(0, 2**62, n // 4, dtype=np.uint64)]
    return vals


def random_table(rng, count):
    recs = (oracle_py.OrcRange * count)()
    base = int(rng.integers(0x1000, 0x100000))
    for i in range(count):
        length = int(rng.choice([0x100, 0x1000, 0x2000, 0x3000, 0x10000]))
        page = int(rng.choice([0x100, 0x1000, 0x4000]))
        recs[i].base = base
        recs[i].length = length
        recs[i].file_offset = int(rng.integers(0, 1 << 20)) * page
        recs[i].range_id = i + 1
        recs[i].mode = int(rng.choice([1, 1, 1, 2, 3]))
        recs[i].permissions = int(rng.choice([1, 2, 3, 3, 0]))
        recs[i].page_bytes = page
        base += length + int(rng.choice([0, 0x10, 0x1000, 0x8000]))
    return recs


def table_json(recs, count):
    return [{"base": r.base, "length": r.length, "file_offset": r.file_offset,
             "range_id": r.range_id, "mode": r.mode, "permissions": r.permissions,
             "page_bytes": r.page_bytes} for r in recs[:count]]


def prefetch_stream(rng, n):
    kind = int(rng.integers(0, 4))
    if kind == 0:                                   # sequential
        return np.arange(n, dtype=np.uint64) + np.uint64(rng.integers(0, 1000))
    if kind == 1:                                   # few pages, repeats
        return rng.integers(0, 6, n).astype(np.uint64)
    if kind == 2:                                   # random over many pages
        return rng.integers(0, 10**6, n).astype(np.uint64)
    runs = []                                       # runs of consecutive pages
    while sum(len(r) for r in runs) < n:
        start = int(rng.integers(0, 500))
        runs.append(np.arange(start, start + int(rng.integers(1, 30)), dtype=np.uint64))
    return np.concatenate(runs)[:n]


def prefetch_cases(ref):
    """simulate_prefetch with the policies that draw no random numbers (the
    Accuracy policy's draws come from the C++ library's distribution)."""
    rng = np.random.default_rng(20261201)  # its own stream: earlier vectors stay as they are
    cases = []
    for _ in range(80):
        n = int(rng.integers(0, 400))
        pages = prefetch_stream(rng, n) if n else np.zeros(0, np.uint64)
        cfg = [int(rng.integers(0, 2)), int(rng.choice([0, 1, 3])),
               int(rng.choice([0, 1, 2, 8, 64])), int(rng.choice([0, 1, 2, 4, 32])),
               int(rng.choice([0, 1, 1000, 10_000])), int(rng.choice([0, 5, 3000]))]
        stats = np.zeros(7, np.uint64)
        ok = ref.ref_simulate_prefetch(pages.ctypes.data, n, cfg[0], 1.0, cfg[1], cfg[2], cfg[3],
                                       cfg[4], cfg[5], 1, stats.ctypes.data)
        cases.append({"pages": pages.tolist(), "config": cfg, "ok": ok,
                      "stats": stats.tolist()})
    return cases


def class_stream(rng, n, classes):
    """n access classes (n x 4 u32) drawn from `classes` distinct ones, the
    fields mixing small values, both operations and 32-bit extremes."""
    pool = np.stack([rng.integers(0, 2, classes),
                     rng.choice([0, 1, 4096, 16384, 65536, 2**31, 2**32 - 1], classes),
                     rng.choice([0, 1, 7, 2**32 - 1], classes),
                     rng.choice([0, 3, 2**16, 2**32 - 1], classes)], axis=1).astype(np.uint32)
    return np.ascontiguousarray(pool[rng.integers(0, classes, n)])


def hybrid_cases(ref):
    """HybridSampler flags and Calibrator estimates from the compiled
    calibrator.cpp: streams with few and many classes, warm-up and rate
    edges (0, 1, in between), sequences from 0 and from far out."""
    rng = np.random.default_rng(20261202)
    sampler = []
    for _ in range(40):
        n = int(rng.integers(0, 300))
        acc = class_stream(rng, n, int(rng.integers(1, 12)))
        first = int(rng.choice([0, 1, 1000, 2**40]))
        seq = np.arange(first, first + n, dtype=np.uint64)
        warm = int(rng.choice([0, 4, 64, 2**32 - 1]))
        rate = float(rng.choice([0.0, 0.01, 0.25, 0.5, 1.0]))
        seed = int(rng.choice([0, 7, 2**63 + 5]))
        flags = np.zeros(max(n, 1), np.uint8)
        ok = ref.ref_sampler_run(warm, rate, seed, acc.ctypes.data, seq.ctypes.data, n,
                                 flags.ctypes.data)
        sampler.append({"access": acc.tolist(), "first": first, "warmup": warm, "rate": rate,
                        "seed": seed, "ok": ok, "flags": flags[:n].tolist()})
    calib = []
    for _ in range(30):
        n = int(rng.integers(1, 400))
        acc = class_stream(rng, n, int(rng.integers(1, 8)))
        edge = np.array([1, 2, 999, 10_000, 123_456, 2**40, 2**63, 2**64 - 1], np.uint64)
        lat = edge[rng.integers(0, len(edge), n)] if rng.random() < 0.3 else \
            rng.integers(1, 200_000, n).astype(np.uint64)
        lat = np.ascontiguousarray(lat, np.uint64)
        rows = []
        for q in np.unique(acc, axis=0):
            q = np.ascontiguousarray(q, np.uint32)
            u = np.zeros(5, np.uint64)
            f = np.zeros(2, np.float64)
            ok = ref.ref_calibrate(acc.ctypes.data, lat.ctypes.data, n, q.ctypes.data,
                                   u.ctypes.data, f.ctypes.data)
            rows.append({"class": q.tolist(), "ok": ok, "u64": u.tolist(), "f64": f.tolist()})
        calib.append({"access": acc.tolist(), "latency": lat.tolist(), "rows": rows})
    return {"sampler": sampler, "calibrate": calib}


def main() -> None:
    ref = oracle_py.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libhbfref.so is missing: run `make -C oracle ref`")
    ref = bind(ref)
    rng = np.random.default_rng(20260801)
    out: dict = {"source": "SlugLab/HBFSim sources compiled by oracle/Makefile ref"}

    out["fast_hash"] = [[v, ref.ref_fast_hash(v)] for v in interesting_u64(rng, 64)]

    hs = []
    for _ in range(300):
        seq = int(rng.integers(0, 5000))
        warm = int(rng.choice([0, 4, 1024]))
        thr = int(rng.choice([0, 2**64 - 1, int(rng.integers(0, 2**63, dtype=np.uint64))]))
        key = int(rng.integers(0, 2**63, dtype=np.uint64))
        hs.append([seq, warm, thr, key, ref.ref_hybrid_reference_sample(seq, warm, thr, key)])
    out["hybrid_reference_sample"] = hs

    xs = []
    for _ in range(400):
        b = int(rng.choice([0, 1, 64, 128, 512, 4096, 16384, 1 << 20, 2**32 - 1,
                            int(rng.integers(1, 2**32))]))
        bw = int(rng.choice([0, 1, 103540697, 512 * 10**9, 10**12, 2**40,
                             int(rng.integers(1, 2**44))]))
        base = int(rng.choice([0, 5000, 10000, 11133, int(rng.integers(0, 10**7))]))
        xs.append([b, bw, base, ref.ref_fast_transfer_ns(b, bw),
                   ref.ref_fast_service_ns(base, b, bw)])
    out["transfer_service"] = xs

    hsv = []
    for _ in range(200):
        rd = int(rng.integers(1, 10**6))
        pg = int(rng.integers(1, 10**7))
        bw = int(rng.integers(1, 2**42))
        op = int(rng.integers(0, 2))
        b = int(rng.integers(1, 2**32))
        hsv.append([rd, pg, bw, op, b, ref.ref_host_fast_service_ns(rd, pg, bw, op, b)])
    out["host_fast_service"] = hsv

    tables = []
    for t in range(12):
        count = int(rng.integers(1, 9))
        recs = random_table(rng, count)
        lo = recs[0].base - 0x2000
        hi = recs[count - 1].base + recs[count - 1].length + 0x2000
        qs = []
        for _ in range(120):
            a = int(rng.integers(max(0, lo), hi))
            if rng.integers(0, 4) == 0:
                r = recs[int(rng.integers(0, count))]
                a = int(rng.choice([r.base - 8, r.base, r.base + r.length - 8, r.base + r.length,
                                    r.base + r.page_bytes - 4]))
            b = int(rng.choice([0, 1, 2, 8, 16, 64, 128, 0x1000, 0x2001]))
            op = int(rng.choice([0, 1, 2]))
            idx = ref.ref_find_range_index(recs, count, a)
            lg, by = U64(), U32()
            if idx < count:
                sup = ref.ref_access_supported(ctypes.byref(recs[idx]), a, b, op)
                ovl = ref.ref_range_overlaps(ctypes.byref(recs[idx]), a, b)
                md = ref.ref_media_descriptor(ctypes.byref(recs[idx]), a, b, op,
                                              ctypes.byref(lg), ctypes.byref(by))
            else:
                sup = ovl = md = 0
            touch = ref.ref_span_touches_any_range(recs, count, a, b)
            qs.append([a, b, op, idx, sup, ovl, touch, md, lg.value, by.value])
        tables.append({"ranges": table_json(recs, count), "queries": qs})
    out["range_tables"] = tables

    curves = [([1, 4, 16, 64, 256, 512], [11133, 41495, 168606, 2824351, 10767793, 20254374],
               408305)]
    for _ in range(4):
        pages = sorted(rng.choice(np.arange(1, 1024), 6, replace=False).tolist())
        cum = sorted(rng.choice(np.arange(1, 10**8), 6, replace=False).tolist())
        curves.append((pages, cum, int(rng.integers(1, 10**6))))
    emp = []
    for pages, cum, prog in curves:
        pa = (U32 * 6)(*pages)
        ca = (U64 * 6)(*cum)
        runs = list(range(0, 1100, 7)) + [1, 2, 3, 4, 5, 511, 512, 513, 1023, 2**32 - 1]
        vals = [[r, ref.ref_empirical_cumulative_ns(pa, ca, 6, r),
                 ref.ref_empirical_service_ns(pa, ca, 6, r)] for r in runs]
        seqs = []
        prev = 0
        page = int(rng.integers(0, 1000))
        for _ in range(300):
            step = int(rng.choice([1, 1, 1, 1, 2, 0, -1, 50]))
            page = max(0, page + step)
            op = int(rng.choice([0, 0, 0, 0, 1]))
            svc, packed, run = U64(), U64(), U32()
            ok = ref.ref_empirical_request_service(pa, ca, prog, prev, page, op,
                                                   ctypes.byref(svc), ctypes.byref(packed),
                                                   ctypes.byref(run))
            seqs.append([prev, page, op, ok, svc.value, packed.value, run.value])
            if ok:
                prev = packed.value
        emp.append({"pages": pages, "cumulative_ns": cum, "program_ns": prog,
                    "curve": vals, "requests": seqs})
    out["empirical"] = emp

    banks = []
    for _ in range(200):
        ch = int(rng.choice([1, 2, 4, 8, 16]))
        ncdu = int(rng.choice([1, 2, 4, 8, 16]))
        nb = int(rng.choice([1, 2, 4, 8, 16]))
        lpa = int(rng.integers(0, 2**40))
        c, d, b, chip = U32(), U32(), U32(), U32()
        ok = ref.ref_cold_read_bank(lpa, ch, ncdu, nb, ctypes.byref(c), ctypes.byref(d),
                                    ctypes.byref(b), ctypes.byref(chip))
        q = int(rng.integers(0, 2**30))
        mod = int(rng.integers(0, ch))
        lp = U64()
        ok2 = ref.ref_hbf_media_lpa(q, mod, ch, ctypes.byref(lp))
        banks.append([lpa, ch, ncdu, nb, ok, c.value, d.value, b.value, chip.value,
                      q, mod, ok2, lp.value])
    out["bank_layout"] = banks

    pb = []
    for _ in range(40):
        n = int(rng.integers(1, 200))
        alphabet = int(rng.integers(1, 6))
        pages = rng.integers(0, alphabet, n).astype(np.uint64)
        hits = np.zeros(n, np.uint8)
        ok = ref.ref_pagebuf_sequence(pages.ctypes.data, n, hits.ctypes.data)
        pb.append({"pages": pages.tolist(), "ok": ok, "hits": hits.tolist()})
    out["pagebuf_two_slots"] = pb

    th = []
    for _ in range(8):
        n = int(rng.integers(1, 24))
        cap = rng.uniform(0.5, 5.0, n)
        init = rng.uniform(290, 340, n)
        sp = rng.uniform(0, 2, n)
        gb = rng.uniform(0, 1.5, n) * (rng.integers(0, 2, n))
        tb = rng.uniform(280, 310, n)
        m = int(rng.integers(0, 3 * n))
        ea = rng.integers(0, n, m).astype(np.uint32)
        eb = ((ea + rng.integers(1, max(2, n), m)) % n).astype(np.uint32)
        keep = ea != eb
        ea, eb = ea[keep], eb[keep]
        eg = rng.uniform(0.1, 4.0, ea.size)
        energy = rng.uniform(0, 3, n) * (rng.integers(0, 2, n))
        steps = int(rng.integers(1, 5))
        dt = float(rng.choice([1e-6, 1e-3, 0.25, 1.0]))
        outv = np.zeros(n)
        f = lambda a: a.ctypes.data  # noqa: E731
        ok = ref.ref_thermal_step(n, f(cap), f(init), f(sp), f(gb), f(tb), ea.size, f(ea),
                                  f(eb), f(eg), f(energy), steps, dt, f(outv))
        th.append({"capacity": cap.tolist(), "initial": init.tolist(), "static_power": sp.tolist(),
                   "boundary_g": gb.tolist(), "boundary_t": tb.tolist(),
                   "edges": [[int(a), int(b), float(g)] for a, b, g in zip(ea, eb, eg)],
                   "energy": energy.tolist(), "steps": steps, "dt": dt, "ok": ok,
                   "temperature": outv.tolist()})
    out["thermal"] = th
    out["prefetch"] = prefetch_cases(ref)
    out["hybrid"] = hybrid_cases(ref)

    path = HERE / "ref_vectors.json"
    path.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
