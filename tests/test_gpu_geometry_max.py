"""Large geometries: 1,024 planes (16 channels, and 256 channels, the channel
maximum); 2,048 planes as the reference's aggressive profile has them (64
channels x 8 dies x 4 planes: the summary pass's per-plane LDS state passes
64 KB); 4,096 planes, the engine's maximum (256 channels; 135 KB of LDS per
summary wave).  Random config-0 records and linear/contiguous streams must
equal the oracle bit for bit in both record forms; a geometry beyond 4,096
planes is refused with HBFSIM_UNSUPPORTED when the first run builds the
engine."""
from __future__ import annotations

import json

import numpy as np
import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0
from hbfsim_amd import _native as nat
from hbfsim_amd import workloads

pytestmark = pytest.mark.gpu


def geometry_profile(tmp_path, channels, dies, planes):
    prof = json.loads(C0.read_text())
    prof.update(channels=channels, dies_per_channel=dies, planes_per_die=planes,
                aggregate_bandwidth_bytes_per_s=channels * 32_000_000_000)
    path = tmp_path / f"geom-{channels}x{dies}x{planes}.json"
    path.write_text(json.dumps(prof))
    return path


@pytest.mark.parametrize("channels,dies,planes", [(16, 16, 4), (256, 1, 4), (64, 8, 4),
                                                  (256, 4, 4)],
                         ids=["1024p-16ch", "1024p-256ch", "2048p-64ch", "4096p-256ch"])
def test_maximum_geometry(tmp_path, channels, dies, planes):
    path = geometry_profile(tmp_path, channels, dies, planes)
    s = workloads.config0(n=100_000, seed=5, write_fraction_per_mille=50)
    ranges = ranges_for()
    lin = chain_clocks(linear_stream(8, 700, ranges), contiguous_stream(9, 150, ranges))
    for rng_set, rec, what in [(s.ranges, s.records, "config0"), (ranges, lin, "linear")]:
        a = parity.Pair(path, rng_set)
        b = parity.Pair(path, rng_set)
        try:
            ga, ca = a.run(rec)
            parity.assert_same(ga, ca, f"{channels}x{dies}x{planes} {what} 32-byte")
            gb, cb = b.run_packed(rec)
            parity.assert_same(gb, cb, f"{channels}x{dies}x{planes} {what} packed")
            a.check_state()
            b.check_state()
        finally:
            a.close()
            b.close()


def test_geometry_beyond_maximum_is_refused(tmp_path):
    import torch
    from hbfsim_amd.engine import Engine
    path = geometry_profile(tmp_path, 256, 4, 8)  # 8,192 planes
    rec = linear_stream(1, 4, ranges_for())
    e = Engine(str(path))
    try:
        for base, length, perms in ranges_for():
            e.register(base, length, perms)
        comp = torch.zeros(len(rec), dtype=torch.int64, device="cuda")
        with pytest.raises(nat.HbfSimError) as err:
            e.run(parity.to_device(rec), comp)
        assert err.value.code == nat.HBFSIM_UNSUPPORTED
    finally:
        e.close()
