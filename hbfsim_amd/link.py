"""UCIe Streaming / AoU link stage on the GPU (hbfsim_amd_link_run).

The reference's StreamingLink (src/ucie/link.cpp) for batches of independent
links: messages (direction 0 = AR request, 1 = R return; ready time in ns)
grouped by link, delivered through each link's flit serializers and credit
loop; the caller admits at most `max_accepted` messages per direction at a
time and consumes each delivery `consume_delay_ns[direction]` later.
"""
from __future__ import annotations

import ctypes
from typing import Any

import numpy as np

from . import _native as nat

REQUEST = 0
RETURN = 1


def link_profile(gt_per_second: int = 16, initial_ar_granules: int = 12,
                 initial_r_granules: int = 56, max_accepted: int = 4, propagation_ns: int = 0,
                 consume_delay_ns: tuple[int, int] = (0, 0)) -> nat.LinkProfile:
    """hbfsim_amd_link_profile; the defaults are LinkProfile's
    (include/hbfsim/ucie/profile.hpp:10-25)."""
    p = nat.LinkProfile()
    p.struct_size = ctypes.sizeof(p)
    p.gt_per_second = gt_per_second
    p.initial_ar_granules = initial_ar_granules
    p.initial_r_granules = initial_r_granules
    p.max_accepted = max_accepted
    p.propagation_ns = propagation_ns
    p.consume_delay_ns[0], p.consume_delay_ns[1] = consume_delay_ns
    return p


def run(profile: nat.LinkProfile, first: Any, ready_ns: Any, direction: Any,
        stream: Any = None) -> tuple[Any, np.ndarray]:
    """Runs every link to quiescence.  first: int64 [links + 1] offsets,
    ready_ns: int64 [n], direction: uint8 [n] (torch tensors on the GPU).
    Returns (delivered_ns int64 [n] on the GPU, counters uint64 [links, 2, 9]
    on the host, fields in nat.LINK_COUNTER_FIELDS order).  ValueError for
    the inputs the library rejects."""
    return _run(profile, first, ready_ns, direction, stream, 0)[:2]


def run_traced(profile: nat.LinkProfile, first: Any, ready_ns: Any, direction: Any,
               limit: int = 4096, stream: Any = None) -> tuple[Any, np.ndarray, list, list]:
    """run() through hbfsim_amd_link_run_traced.  Also returns, per link, its
    flit records in the reference's order (StreamingLink::flits(): both
    directions in step order, the request direction first within a step),
    the first `limit` of them, as dicts of FlitRecord's fields with request
    ids = message position in the link + 1, and the number of flits not
    recorded (flit_records_dropped).  The reference's order is the link's
    step order, the request direction first within a step."""
    delivered, counters, raw = _run(profile, first, ready_ns, direction, stream, limit)
    links = counters.shape[0]
    flits, dropped = [], []
    for l in range(links):
        recs = []
        for d in (0, 1):
            k = min(limit, int(counters[l, d, 0]))
            recs += [(int(r["step"]), d, r) for r in raw[l, d, :k]]
        recs.sort(key=lambda x: (x[0], x[1]))
        flits.append([flit_dict(r) for _, _, r in recs[:limit]])
        dropped.append(int(counters[l, 0, 0] + counters[l, 1, 0]) - len(flits[-1]))
    return delivered, counters, flits, dropped


def flit_dict(r) -> dict:
    """One hbfsim_amd_link_flit record as a dict of FlitRecord's fields."""
    return {"direction": int(r["direction"]), "start_ns": int(r["start_ns"]),
            "delivered_ns": int(r["delivered_ns"]),
            "message_granules": int(r["message_granules"]),
            "grant_granules": int(r["grant_granules"]), "credit_only": bool(r["credit_only"]),
            "fragments": [dict(request_id=int(f["request_id"]),
                               flit_granule=int(f["flit_granule"]),
                               message_granule=int(f["message_granule"]),
                               granules=int(f["granules"]), msg_start=bool(f["msg_start"]),
                               msg_end=bool(f["msg_end"]))
                          for f in r["fragment"][:int(r["fragments"])]]}


def run_into(profile: nat.LinkProfile, first: Any, ready_ns: Any, direction: Any,
             delivered: Any, counters: Any, stream: Any = None) -> None:
    """hbfsim_amd_link_run into caller-owned device tensors (delivered int64
    [n], counters int64 [links, 2, 9]); nothing is copied to the host."""
    import torch
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    rc = nat.load().hbfsim_amd_link_run(ctypes.byref(profile), first.data_ptr(),
                                        int(first.shape[0]) - 1, ready_ns.data_ptr(),
                                        direction.data_ptr(), int(ready_ns.shape[0]),
                                        delivered.data_ptr(), counters.data_ptr(),
                                        ctypes.c_void_p(stream))
    if rc in (nat.HBFSIM_INVALID_ARGUMENT, nat.HBFSIM_UNSUPPORTED):
        raise ValueError(f"link run refused: {nat.status_name(rc)} ({rc})")
    nat.check(rc, "link run")


def _run(profile, first, ready_ns, direction, stream, limit):
    import torch
    links = int(first.shape[0]) - 1
    n = int(ready_ns.shape[0])
    fields = len(nat.LINK_COUNTER_FIELDS)
    delivered = torch.zeros(max(n, 1), dtype=torch.int64, device=ready_ns.device)
    counters = torch.zeros((max(links, 1), 2, fields), dtype=torch.int64, device=ready_ns.device)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    L = nat.load()
    raw = None
    if limit == 0:
        rc = L.hbfsim_amd_link_run(ctypes.byref(profile), first.data_ptr(), links,
                                   ready_ns.data_ptr(), direction.data_ptr(), n,
                                   delivered.data_ptr(), counters.data_ptr(),
                                   ctypes.c_void_p(stream))
    else:
        size = nat.LINK_FLIT_DTYPE.itemsize
        buf = torch.zeros(max(links, 1) * 2 * limit * size, dtype=torch.uint8,
                          device=ready_ns.device)
        rc = L.hbfsim_amd_link_run_traced(ctypes.byref(profile), first.data_ptr(), links,
                                          ready_ns.data_ptr(), direction.data_ptr(), n,
                                          delivered.data_ptr(), counters.data_ptr(),
                                          buf.data_ptr(), limit, ctypes.c_void_p(stream))
        if rc == nat.HBFSIM_OK:
            raw = buf.cpu().numpy().view(nat.LINK_FLIT_DTYPE).reshape(max(links, 1), 2, limit)
    if rc in (nat.HBFSIM_INVALID_ARGUMENT, nat.HBFSIM_UNSUPPORTED):
        raise ValueError(f"link run refused: {nat.status_name(rc)} ({rc})")
    nat.check(rc, "link run")
    return delivered[:n], counters[:links].cpu().numpy().view(np.uint64), raw
