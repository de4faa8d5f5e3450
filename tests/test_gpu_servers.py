"""The k-server media queue (MediaServers::issue, prefetch_model.cpp:22-50)
on the GPU against the oracle's min-heap, bit for bit: server counts from 1
to more than the reads, bursts of equal issue times, idle gaps, zero and
large latencies, batch sizes around the kernel's tile edges; decreasing or
oversized issue times are rejected."""
from __future__ import annotations

import numpy as np
import pytest

from hbfsim_amd import engine
from test_oracle_servers import oracle_servers

pytestmark = pytest.mark.gpu


def run(now, k, latency):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(now, np.uint64).view(np.int64)).cuda()
    out = engine.media_servers(t, k, latency)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint64)


def stream(n, seed):
    rng = np.random.default_rng(seed)
    gaps = rng.choice([0, 0, 0, 1, 7, 300, 20_000], n).astype(np.uint64)
    return np.cumsum(gaps, dtype=np.uint64) + np.uint64(rng.integers(0, 10**9))


@pytest.mark.parametrize("n", [1, 5, 63, 64, 65, 2047, 2048, 2049, 100_003])
@pytest.mark.parametrize("k", [0, 1, 3, 64, 100, 4096])
def test_servers_bit_exact(n, k):
    now = stream(n, n + k)
    for latency in (0, 5000, 123_456_789):
        got = run(now, k, latency)
        np.testing.assert_array_equal(got, np.array(oracle_servers(now, k, latency), np.uint64),
                                      f"n={n} k={k} L={latency}")


def test_servers_large_batch_against_chains():
    """2e6 reads on 1000 servers: the oracle's heap agrees on a prefix, and
    every completion obeys c_i = max(now_i, c_{i-k}) + L."""
    n, k, latency = 2_000_000, 1000, 25_000
    now = stream(n, 99)
    got = run(now, k, latency)
    np.testing.assert_array_equal(got[:20_000],
                                  np.array(oracle_servers(now[:20_000], k, latency), np.uint64))
    prev = np.concatenate([np.zeros(k, np.uint64), got[:-k]])
    np.testing.assert_array_equal(got, np.maximum(now, prev) + np.uint64(latency))


def test_servers_reject_bad_issue_times():
    now = stream(5000, 7)
    now[1234], now[1235] = now[1235] + np.uint64(10), now[1235]
    with pytest.raises(ValueError):
        run(now, 4, 100)
    big = stream(10, 8)
    big[-1] = np.uint64(1 << 63)
    with pytest.raises(ValueError):
        run(big, 2, 100)
    assert run(np.zeros(0, np.uint64), 3, 10).shape == (0,)
