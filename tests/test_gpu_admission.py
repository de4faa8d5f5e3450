"""hbfsim_amd_mqsim_admission (the MQSim adapter's queue-depth admission and
bandwidth cursor, mqsim_online.cpp:291-376, over a one-latency media port)
against the oracle's event-loop restatement, bit for bit: admission times
and bounded completions, across queue depths from 0 (taken as 1) to beyond
the request count, tied arrivals, bursts, byte counts and bandwidths."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py
from hbfsim_amd import engine as eng

pytestmark = pytest.mark.gpu


def gpu(arrival, nbytes, depth, latency, bw):
    import torch
    a = torch.from_numpy(np.asarray(arrival, np.uint64).view(np.int64).copy()).cuda()
    b = torch.from_numpy(np.asarray(nbytes, np.uint64).view(np.int64).copy()).cuda()
    adm, done = eng.mqsim_admission(a, b, depth, latency, bw)
    return adm.cpu().numpy().view(np.uint64), done.cpu().numpy().view(np.uint64)


@pytest.mark.parametrize("seed", range(10))
def test_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.choice([1, 7, 1000, 50_000, 300_000]))
    gaps = rng.integers(0, int(rng.choice([1, 50, 2000])), n)
    gaps[rng.random(n) < 0.2] = 0
    arrival = np.cumsum(gaps).astype(np.uint64)
    nbytes = (rng.integers(1, 128, n) * 512).astype(np.uint64)
    depth = int(rng.choice([0, 1, 3, 32, 64, 1000, n + 5]))
    latency = int(rng.integers(1, 100_000))
    bw = int(rng.integers(10**8, 10**11))
    adm, done = gpu(arrival, nbytes, depth, latency, bw)
    o_adm, o_dev, o_done = oracle_py.mqsim_admission(arrival, nbytes, latency, depth, bw)
    np.testing.assert_array_equal(adm, o_adm)
    np.testing.assert_array_equal(done, o_done)
    np.testing.assert_array_equal(o_dev, o_adm + np.uint64(latency))


def test_reference_burst_properties():
    """mqsim_queue_depth_test.cpp:73-124 with a 45 us port."""
    arrival = np.zeros(32, np.uint64)
    nbytes = np.full(32, 16384, np.uint64)
    _, shallow = gpu(arrival, nbytes, 1, 45_000, 32 * 10**9)
    _, deep = gpu(arrival, nbytes, 32, 45_000, 32 * 10**9)
    assert shallow.max() > deep.max() and shallow.max() >= 32 * 45_000


def test_refusals():
    with pytest.raises(ValueError):
        gpu([5, 3], [512, 512], 1, 10, 10**9)
    with pytest.raises(ValueError):
        gpu([0, 1], [512, 512], 1, 10, 0)
    with pytest.raises(ValueError):
        gpu([0, 2**63], [512, 512], 1, 10, 10**9)
