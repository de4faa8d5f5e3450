"""Runs one access stream through the HIP engine (C ABI) and the CPU oracle
and compares every output bit for bit."""
from __future__ import annotations

import numpy as np

import oracle_py
from hbfsim_amd import engine as eng

OPTION_KEYS = ("page_buffers", "plane_contention", "transfer_page", "program_every_write",
               "flat_geometry", "ways", "xfer_quantum_ps", "channel_bandwidth_bytes_per_s",
               "warp_grouping")


def to_device(records: np.ndarray):
    import torch
    rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
    return torch.from_numpy(rec.view(np.int64)).cuda()


class Pair:
    """An engine context and an oracle state fed the same ranges and runs."""

    def __init__(self, profile_path, ranges, mode="fast", tile_records=None, **options):
        import torch  # noqa: F401  (device memory owner)
        self.profile = oracle_py.load_profile(profile_path)
        self.engine = eng.Engine(str(profile_path), mode=mode)
        for base, length, perms in ranges:
            self.engine.register(base, length, perms)
        opts = {k: v for k, v in options.items() if k in OPTION_KEYS}
        if tile_records is not None:
            opts["tile_records"] = tile_records
        if opts:
            self.engine.set_options(**opts)
        self.params = oracle_py.engine_params(self.profile, hybrid=(mode == "hybrid"),
                                              **{k: v for k, v in options.items()
                                                 if k in OPTION_KEYS})
        self.ranges, self.count = oracle_py.range_table(ranges, self.profile["page_bytes"],
                                                        self.profile["capacity_bytes"])
        self.ostate = oracle_py.OracleState(self.params)

    def run(self, records: np.ndarray, base_ps: int = 0):
        import torch
        rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
        n = rec.shape[0]
        d_rec = to_device(rec)
        d_comp = torch.zeros(max(n, 1), dtype=torch.int64, device="cuda")
        d_st = torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda")
        grep = self.engine.run(d_rec, d_comp, d_st, base_ps=base_ps)
        torch.cuda.synchronize()
        gcomp = d_comp.cpu().numpy().view(np.uint64)[:n]
        gst = d_st.cpu().numpy()[:n]
        ocomp, ost, orep, _ = oracle_py.run(self.params, self.ranges, self.count, rec, base_ps,
                                            self.ostate)
        return (gcomp, gst, grep), (ocomp, ost, orep)

    def run_packed(self, records: np.ndarray, base_ps: int = 0):
        """run() through the packed 16-byte records; the oracle takes the
        32-byte records they pack."""
        import torch
        from hbfsim_amd.engine import pack_records
        rec = np.ascontiguousarray(records, dtype=np.uint64).reshape(-1, 4)
        n = rec.shape[0]
        d_rec = pack_records(to_device(rec))
        d_comp = torch.zeros(max(n, 1), dtype=torch.int64, device="cuda")
        d_st = torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda")
        grep = self.engine.run_packed(d_rec, d_comp, d_st, base_ps=base_ps)
        torch.cuda.synchronize()
        gcomp = d_comp.cpu().numpy().view(np.uint64)[:n]
        gst = d_st.cpu().numpy()[:n]
        ocomp, ost, orep, _ = oracle_py.run(self.params, self.ranges, self.count, rec, base_ps,
                                            self.ostate)
        return (gcomp, gst, grep), (ocomp, ost, orep)

    def check_state(self):
        gp, gc = self.engine.busy_totals()
        np.testing.assert_array_equal(gp, self.ostate.plane_busy_total, "plane busy totals")
        np.testing.assert_array_equal(gc, self.ostate.channel_busy_total, "channel busy totals")
        st = self.engine.state()
        np.testing.assert_array_equal(st["channel_cursor"], self.ostate.channel_cursor,
                                      "channel cursors")
        if self.params.plane_contention:
            np.testing.assert_array_equal(st["plane_busy"], self.ostate.plane_busy,
                                          "plane busy-until")
        if self.params.page_buffers:
            k = self.params.page_buffers
            g = st["plane_tags"].reshape(-1, 2)[:, :k]
            o = self.ostate.plane_tag.reshape(-1, 2)[:, :k]
            np.testing.assert_array_equal(g, o, "page-register tags")
        assert st["sequence"] == self.ostate.s.modeled_sequence

    def close(self):
        self.engine.close()


def assert_same(gpu, cpu, what=""):
    gcomp, gst, grep = gpu
    ocomp, ost, orep = cpu
    if not np.array_equal(gcomp, ocomp):
        bad = np.nonzero(gcomp != ocomp)[0]
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.size} completion mismatches; first at {i}: "
                             f"gpu {int(gcomp[i])} oracle {int(ocomp[i])}")
    if not np.array_equal(gst, ost):
        bad = np.nonzero(gst != ost)[0]
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.size} status mismatches; first at {i}: "
                             f"gpu {int(gst[i])} oracle {int(ost[i])}")
    assert grep == orep, f"{what}: report differs\n gpu {grep}\n cpu {orep}"


ORACLE_THREADS = max(1, min(16, __import__("os").cpu_count() or 1))
CHUNK = 1 << 26


def merge_reports(a: dict | None, b: dict) -> dict:
    """Report of two consecutive runs (counts add, extremes take the max)."""
    if a is None:
        return dict(b)
    out = {k: a[k] + b[k] for k in a if k not in ("makespan_ps", "latency_max_ps",
                                                  "latency_sum_lo", "latency_sum_hi",
                                                  "latency_sum_ps")}
    out["makespan_ps"] = max(a["makespan_ps"], b["makespan_ps"])
    out["latency_max_ps"] = max(a["latency_max_ps"], b["latency_max_ps"])
    total = a["latency_sum_ps"] + b["latency_sum_ps"]
    out["latency_sum_ps"] = total
    out["latency_sum_lo"] = total & ((1 << 64) - 1)
    out["latency_sum_hi"] = total >> 64
    return out


def compare_whole(pair: "Pair", d_rec, d_comp, d_st, base_ps: int, what: str,
                  chunk: int = CHUNK) -> dict:
    """Every completion and status byte of a GPU run of the 32-byte records
    d_rec (int64 [n, 4] on the GPU) against the OpenMP oracle run over the
    same records, taken in chunks with the oracle's state carried (the same
    as one run; the records must be in issue order, since the oracle serves a
    stream that goes back in time from its sorted copy, per run).  Returns the
    oracle's report of the whole run."""
    n = int(d_rec.shape[0])
    rep = None
    for a in range(0, n, chunk):
        b = min(n, a + chunk)
        rec = d_rec[a:b].cpu().numpy().view(np.uint64)
        ocomp, ost, orep, _ = oracle_py.run(pair.params, pair.ranges, pair.count, rec, base_ps,
                                            pair.ostate, threads=ORACLE_THREADS)
        gcomp = d_comp[a:b].cpu().numpy().view(np.uint64)
        gst = d_st[a:b].cpu().numpy()
        if not np.array_equal(gcomp, ocomp):
            bad = np.nonzero(gcomp != ocomp)[0]
            i = int(bad[0])
            raise AssertionError(f"{what}: {bad.size} completion mismatches in records "
                                 f"[{a}, {b}); first at {a + i}: gpu {int(gcomp[i])} "
                                 f"oracle {int(ocomp[i])}")
        if not np.array_equal(gst, ost):
            bad = np.nonzero(gst != ost)[0]
            i = int(bad[0])
            raise AssertionError(f"{what}: {bad.size} status mismatches in records "
                                 f"[{a}, {b}); first at {a + i}: gpu {int(gst[i])} "
                                 f"oracle {int(ost[i])}")
        rep = merge_reports(rep, orep)
    return rep
