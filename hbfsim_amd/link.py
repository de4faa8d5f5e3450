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
    Returns (delivered_ns int64 [n] on the GPU, counters uint64 [links, 2, 8]
    on the host, fields in nat.LINK_COUNTER_FIELDS order).  ValueError for
    the inputs the library rejects."""
    import torch
    links = int(first.shape[0]) - 1
    n = int(ready_ns.shape[0])
    delivered = torch.zeros(max(n, 1), dtype=torch.int64, device=ready_ns.device)
    counters = torch.zeros((max(links, 1), 2, 8), dtype=torch.int64, device=ready_ns.device)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    rc = nat.load().hbfsim_amd_link_run(ctypes.byref(profile), first.data_ptr(), links,
                                        ready_ns.data_ptr(), direction.data_ptr(), n,
                                        delivered.data_ptr(), counters.data_ptr(),
                                        ctypes.c_void_p(stream))
    if rc in (nat.HBFSIM_INVALID_ARGUMENT, nat.HBFSIM_UNSUPPORTED):
        raise ValueError(f"link run refused: {nat.status_name(rc)} ({rc})")
    nat.check(rc, "link run")
    return delivered[:n], counters[:links].cpu().numpy().view(np.uint64)
