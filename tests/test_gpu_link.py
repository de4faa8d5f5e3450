"""The UCIe Streaming / AoU link kernel (hbfsim_amd_link_run) against the CPU
oracle's restatement of StreamingLink, link by link: every delivery time and
every direction counter bit-exact, on the reference test's own scenarios
(tests/cpu/ucie_link_test.cpp:50-104) and on seeded random batches of links
across profiles, credits, capacities, propagation and consume delays."""
from __future__ import annotations

import numpy as np
import pytest

import oracle_py as o
from hbfsim_amd import link as lk
from hbfsim_amd import _native as nat

pytestmark = pytest.mark.gpu

FIELDS = nat.LINK_COUNTER_FIELDS


def gpu_run(profile, links):
    """links: list of (direction[], ready[]) per link."""
    import torch
    first = np.zeros(len(links) + 1, np.uint64)
    first[1:] = np.cumsum([len(r) for _, r in links])
    dirs = np.concatenate([np.asarray(d, np.uint8) for d, _ in links]) if links else \
        np.zeros(0, np.uint8)
    ready = np.concatenate([np.asarray(r, np.uint64) for _, r in links]) if links else \
        np.zeros(0, np.uint64)
    t_first = torch.from_numpy(first.view(np.int64)).cuda()
    t_ready = torch.from_numpy(ready.view(np.int64).copy()).cuda()
    t_dir = torch.from_numpy(dirs.copy()).cuda()
    delivered, counters = lk.run(profile, t_first, t_ready, t_dir)
    return delivered.cpu().numpy().view(np.uint64), counters, first


def oracle_profile(p):
    return o.link_profile(gt=p.gt_per_second, ar=p.initial_ar_granules, r=p.initial_r_granules,
                          max_accepted=p.max_accepted, propagation_ns=p.propagation_ns)


def check_against_oracle(profile, links):
    delivered, counters, first = gpu_run(profile, links)
    delay = (int(profile.consume_delay_ns[0]), int(profile.consume_delay_ns[1]))
    for k, (d, r) in enumerate(links):
        want, wc = o.link_scenario(oracle_profile(profile), d, r, delay)
        got = delivered[first[k]:first[k + 1]]
        np.testing.assert_array_equal(got, want, err_msg=f"link {k}")
        for dirn in (0, 1):
            assert dict(zip(FIELDS, counters[k, dirn].tolist())) == wc[dirn], (k, dirn)
    return delivered, counters


def test_reference_scenarios():
    p = lk.link_profile(gt_per_second=16, initial_ar_granules=128, initial_r_granules=128,
                        max_accepted=128)
    links = [([0] * 16, [0] * 16), ([0] * 17, [0] * 17), ([1] * 4, [0] * 4)]
    _, c = check_against_oracle(p, links)
    # ucie_link_test.cpp:50-87
    assert c[0, 0, 0] == 1 and c[0, 0, 5] == 240 and c[0, 0, 6] == 0
    assert c[1, 0, 0] == 2 and c[1, 0, 5] == 255 and c[1, 0, 6] == 225
    assert c[2, 1, 0] == 2 and c[2, 1, 5] == 280 and c[2, 1, 6] == 200
    # ucie_link_test.cpp:88-104: three unit grants on the return direction
    p3 = lk.link_profile(gt_per_second=16, initial_ar_granules=3, initial_r_granules=14,
                         max_accepted=128)
    _, c3 = check_against_oracle(p3, [([0], [0])])
    assert c3[0, 1, 7] == 3 and c3[0, 1, 1] == 768 and c3[0, 1, 6] == 720


@pytest.mark.parametrize("seed", range(12))
def test_random_batches(seed):
    """Seeds 0, 3, 6, 9 fit the small LDS form (at most 4 messages admitted
    per direction, at most 4 flits in flight: propagation below 2 flit
    times); seeds 2, 5, 8, 11 the large one (at most 16 admitted, at most 8
    flits: propagation up to 5 flit times); the others need the HBM form
    (more admitted messages or a longer propagation delay)."""
    rng = np.random.default_rng(100 + seed)
    gt = int(rng.choice([8, 16, 32]))
    ser = 32 // gt
    if seed % 3 == 0:
        accepted, prop = int(rng.integers(1, 5)), int(rng.integers(0, 2 * ser))
    elif seed % 3 == 2:
        accepted, prop = int(rng.integers(1, 17)), int(rng.integers(0, 5 * ser + 1))
        if accepted <= 4 and prop < 2 * ser:
            accepted = 5 + int(rng.integers(0, 12))
    else:
        accepted, prop = int(rng.integers(1, 41)), int(rng.integers(0, 60))
        if accepted <= 16 and prop <= 5 * ser:
            accepted = 17 + int(rng.integers(0, 24))
    p = lk.link_profile(gt_per_second=gt, initial_ar_granules=int(rng.integers(3, 80)),
                        initial_r_granules=int(rng.integers(14, 200)), max_accepted=accepted,
                        propagation_ns=prop,
                        consume_delay_ns=(int(rng.integers(0, 30)), int(rng.integers(0, 90))))
    links = []
    for _ in range(int(rng.integers(20, 130))):
        m = int(rng.integers(0, 300))
        d = rng.integers(0, 2, m).astype(np.uint8)
        r = np.sort(rng.integers(0, int(rng.integers(1, 40)) * max(m, 1), m)).astype(np.uint64)
        links.append((d, r))
    check_against_oracle(p, links)


@pytest.mark.parametrize("accepted,prop", [(4, 7), (5, 7), (4, 8), (4, 5), (16, 23), (17, 5),
                                           (4, 24)])
def test_bursts_and_idle_gaps(accepted, prop):
    """Bursts separated by idle periods longer than the pipeline, equal ready
    times across directions, one direction only, empty links; at the edges of
    the small LDS form (4 admitted, 4 flits in flight at 8 GT/s), of the large
    one (16 admitted, 8 flits) and just past them."""
    p = lk.link_profile(gt_per_second=8, initial_ar_granules=12, initial_r_granules=56,
                        max_accepted=accepted, propagation_ns=prop, consume_delay_ns=(3, 0))
    links = [
        ([0, 1, 0, 1, 1, 0], [0, 0, 0, 0, 1000, 1000]),
        ([1] * 30, [0] * 10 + [500] * 10 + [501] * 10),
        ([], []),
        ([0] * 100, list(range(0, 1000, 10))),
        ([0, 1] * 50, [7] * 100),
    ]
    check_against_oracle(p, links)


def test_refusals():
    import torch
    p = lk.link_profile()
    with pytest.raises(ValueError):  # ready times out of order within a direction
        gpu_run(p, [([0, 0], [10, 5])])
    with pytest.raises(ValueError):  # direction above 1
        gpu_run(p, [([2], [0])])
    bad = lk.link_profile(gt_per_second=64)
    with pytest.raises(ValueError):
        gpu_run(bad, [([0], [0])])
    with pytest.raises(ValueError):  # an event time past 2^64 - 1 ns
        gpu_run(p, [([0], [2**64 - 1])])
    # malformed offsets (decreasing) are refused before anything is read
    first = torch.tensor([0, 3, 1], dtype=torch.int64, device="cuda")
    ready = torch.zeros(3, dtype=torch.int64, device="cuda")
    dirs = torch.zeros(3, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        lk.run(p, first, ready, dirs)


def traced_against_oracle(profile, links, limit=4096):
    """hbfsim_amd_link_run_traced: deliveries and counters as the untraced
    run's, and each link's flit records (the reference's single list, first
    4,096, plus the dropped count) equal to the oracle's StreamingLink."""
    import torch
    first = np.zeros(len(links) + 1, np.uint64)
    first[1:] = np.cumsum([len(r) for _, r in links])
    dirs = np.concatenate([np.asarray(d, np.uint8) for d, _ in links])
    ready = np.concatenate([np.asarray(r, np.uint64) for _, r in links])
    t_first = torch.from_numpy(first.view(np.int64)).cuda()
    t_ready = torch.from_numpy(ready.view(np.int64).copy()).cuda()
    t_dir = torch.from_numpy(dirs.copy()).cuda()
    delivered, counters, flits, dropped = lk.run_traced(profile, t_first, t_ready, t_dir, limit)
    plain, plain_c = lk.run(profile, t_first, t_ready, t_dir)
    assert torch.equal(delivered, plain)
    np.testing.assert_array_equal(counters, plain_c)
    delivered = delivered.cpu().numpy().view(np.uint64)
    delay = (int(profile.consume_delay_ns[0]), int(profile.consume_delay_ns[1]))
    for k, (d, r) in enumerate(links):
        want, wc, wflits, wdropped = o.link_scenario_traced(oracle_profile(profile), d, r, delay)
        np.testing.assert_array_equal(delivered[first[k]:first[k + 1]], want)
        for dirn in (0, 1):
            assert dict(zip(FIELDS, counters[k, dirn].tolist())) == wc[dirn], (k, dirn)
        assert flits[k] == wflits, f"link {k}: flit records"
        assert dropped[k] == wdropped, f"link {k}: dropped"
    return flits, dropped, counters


def test_traced_reference_known_answers():
    """ucie_link_test.cpp:74-87: four R messages (14 granules each) cross
    the 48-granule flit boundary; the fourth message's first fragment ends
    flit 0 without MsgEnd and its second starts flit 1 at message granule 6
    with MsgEnd.  ucie_link_test.cpp:88-104: every grant is a legal AoU
    amount; the three-granule credit return takes three unit grants."""
    p = lk.link_profile(gt_per_second=16, initial_ar_granules=128, initial_r_granules=128,
                        max_accepted=128)
    flits, dropped, _ = traced_against_oracle(p, [([1] * 4, [0] * 4), ([0] * 17, [0] * 17)])
    f0, f1 = flits[0][0], flits[0][1]
    assert f0["fragments"][-1]["request_id"] == 4 and not f0["fragments"][-1]["msg_end"]
    assert f1["fragments"][0]["request_id"] == 4 and f1["fragments"][0]["message_granule"] == 6
    assert f1["fragments"][0]["msg_end"]
    assert [len(f["fragments"]) for f in flits[1] if f["direction"] == 0] == [16, 1]
    assert dropped == [0, 0]
    p3 = lk.link_profile(gt_per_second=16, initial_ar_granules=3, initial_r_granules=14,
                         max_accepted=128)
    flits3, _, c3 = traced_against_oracle(p3, [([0], [0])])
    legal = {0, 1, 4, 8, 16, 32, 64, 128}
    assert all(f["grant_granules"] in legal for f in flits3[0])
    assert sum(f["credit_only"] for f in flits3[0] if f["direction"] == 1) == 3
    assert c3[0, 1, 8] == 0 and c3[0, 0, 8] == 0  # accounting_saturated


@pytest.mark.parametrize("form", ["small", "large", "hbm"])
def test_traced_random_links(form):
    """Random links on each kernel form; some carry more than 4,096 flits,
    whose later flits the reference counts as dropped."""
    rng = np.random.default_rng({"small": 1, "large": 2, "hbm": 3}[form])
    accepted, prop = {"small": (4, 1), "large": (12, 9), "hbm": (30, 40)}[form]
    p = lk.link_profile(gt_per_second=8, initial_ar_granules=int(rng.integers(3, 60)),
                        initial_r_granules=int(rng.integers(14, 120)), max_accepted=accepted,
                        propagation_ns=prop, consume_delay_ns=(int(rng.integers(0, 20)),
                                                               int(rng.integers(0, 60))))
    links = []
    for k in range(40):
        m = 6000 if k < 3 else int(rng.integers(0, 400))
        d = rng.integers(0, 2, m).astype(np.uint8)
        r = np.sort(rng.integers(0, 20 * max(m, 1), m)).astype(np.uint64)
        links.append((d, r))
    flits, dropped, _ = traced_against_oracle(p, links)
    assert any(x > 0 for x in dropped[:3]) and all(len(f) <= 4096 for f in flits)


def test_traced_small_limit_and_refusal():
    """A limit below the flit count keeps each direction's first flits; the
    merged list is the oracle's prefix.  A zero limit is refused."""
    import ctypes
    import torch
    p = lk.link_profile(gt_per_second=32, max_accepted=8)
    rng = np.random.default_rng(9)
    d = rng.integers(0, 2, 500).astype(np.uint8)
    r = np.sort(rng.integers(0, 3000, 500)).astype(np.uint64)
    t_first = torch.tensor([0, 500], dtype=torch.int64, device="cuda")
    t_ready = torch.from_numpy(r.view(np.int64).copy()).cuda()
    t_dir = torch.from_numpy(d.copy()).cuda()
    _, _, flits, dropped = lk.run_traced(p, t_first, t_ready, t_dir, limit=37)
    _, _, wflits, _ = o.link_scenario_traced(oracle_profile(p), d, r, (0, 0))
    assert flits[0] == wflits[:37]
    assert dropped[0] == len(wflits) - 37
    L = nat.load()
    out = torch.zeros(2 * nat.LINK_FLIT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    dl = torch.zeros(500, dtype=torch.int64, device="cuda")
    cnt = torch.zeros(18, dtype=torch.int64, device="cuda")
    rc = L.hbfsim_amd_link_run_traced(ctypes.byref(p), t_first.data_ptr(), 1, t_ready.data_ptr(),
                                      t_dir.data_ptr(), 500, dl.data_ptr(), cnt.data_ptr(),
                                      out.data_ptr(), 0, None)
    assert rc == nat.HBFSIM_INVALID_ARGUMENT
