"""Empty, single-record and ragged runs in sequence on one engine: an empty
run reports nothing and leaves the state alone, and runs of 1, 63, 65 and
an odd remainder of records (partial steps and partial groups) continue the
state of the runs before them.  Both record forms, against the oracle bit
for bit after every run."""
from __future__ import annotations

import numpy as np
import pytest

import parity
from test_gpu_linear import chain_clocks, contiguous_stream, linear_stream, ranges_for
from test_gpu_parity import C0, C2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("profile", [C0, C2], ids=["c0", "c2"])
@pytest.mark.parametrize("form", ["32", "packed"])
def test_empty_single_and_ragged_runs(profile, form):
    ranges = ranges_for()
    rec = chain_clocks(linear_stream(11, 60, ranges), contiguous_stream(12, 12, ranges))
    p = parity.Pair(profile, ranges)
    run = p.run if form == "32" else p.run_packed
    cuts = [(0, 0), (0, 1), (1, 1), (1, 64), (64, 129), (129, 129), (129, len(rec)),
            (len(rec), len(rec))]
    try:
        for lo, hi in cuts:
            g, c = run(rec[lo:hi], 7 * lo)
            parity.assert_same(g, c, f"{form} {profile.name} {lo}:{hi}")
            assert g[2]["records"] == hi - lo
        p.check_state()
    finally:
        p.close()
