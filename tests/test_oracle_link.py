"""The oracle's UCIe Streaming / AoU link against the known answers of the
reference's own test (tests/cpu/ucie_link_test.cpp:41-183), replayed call
for call through the same object API, plus invariants of the flit and
credit accounting the restatement must keep."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle_py as o
from oracle_py import REQUEST, RETURN


def drain(link: o.Link) -> int:
    """ucie_link_test.cpp:28-39: step until quiescent, consuming every
    delivery at its delivery time."""
    delivered = 0
    for _ in range(1000):
        if link.next_event_ns() is None:
            break
        for d, rid, at in link.step():
            delivered += 1
            link.consume(d, rid, at)
    assert link.next_event_ns() is None, "link did not quiesce"
    return delivered


def test_grade_serialization():
    # ucie_link_test.cpp:44-49
    L = o._link_lib()
    assert L.orc_link_serialization_ns(ctypes.byref(o.link_profile(gt=16))) == 2
    for grade, ns in ((8, 4), (16, 2), (32, 1)):
        assert L.orc_link_serialization_ns(ctypes.byref(o.link_profile(gt=grade))) == ns
    # ucie_link_test.cpp:137-143: an unsupported rate is rejected
    assert not L.orc_link_profile_valid(ctypes.byref(o.link_profile(gt=64)))
    with pytest.raises(ValueError):
        o.Link(o.link_profile(gt=64))


def test_sixteen_requests_fill_one_flit():
    # ucie_link_test.cpp:50-60: 16 * 15 B = one 240 B AoU message area
    link = o.Link(o.link_profile())
    for i in range(1, 17):
        link.enqueue(REQUEST, i, 0)
    assert drain(link) == 16
    c = link.counters(REQUEST)
    assert (c["flits"], c["wire_bytes"], c["aou_message_bytes"], c["unused_message_bytes"],
            c["aou_header_bytes"], c["ucie_header_bytes"], c["crc_position_bytes"]) == \
        (1, 256, 240, 0, 10, 2, 4)
    link.close()


def test_seventeen_requests():
    # ucie_link_test.cpp:61-71: 255 message + 225 unused + 20 AoU + 12 UCIe = 512 B
    link = o.Link(o.link_profile())
    for i in range(1, 18):
        link.enqueue(REQUEST, i, 0)
    drain(link)
    c = link.counters(REQUEST)
    assert (c["flits"], c["wire_bytes"], c["aou_message_bytes"], c["unused_message_bytes"],
            c["aou_header_bytes"]) == (2, 512, 255, 225, 20)
    assert c["ucie_header_bytes"] + c["crc_position_bytes"] == 12
    link.close()


def test_returns_cross_flits_with_fragment_offsets():
    # ucie_link_test.cpp:72-87: 4 * 70 B = 280 B across two 240 B areas
    link = o.Link(o.link_profile())
    for i in range(1, 5):
        link.enqueue(RETURN, i, 0)
    drain(link)
    c = link.counters(RETURN)
    assert (c["flits"], c["wire_bytes"], c["aou_message_bytes"], c["unused_message_bytes"]) == \
        (2, 512, 280, 200)
    f = [x for x in link.flits() if x["direction"] == RETURN]
    last0, first1 = f[0]["fragments"][-1], f[1]["fragments"][0]
    assert last0["request_id"] == 4 and not last0["msg_end"]
    assert first1["request_id"] == 4 and first1["message_granule"] == 6 and first1["msg_end"]
    link.close()


def test_three_granule_credit_return_uses_unit_grants():
    # ucie_link_test.cpp:88-104
    link = o.Link(o.link_profile(ar=3, r=14))
    link.enqueue(REQUEST, 1, 0)
    drain(link)
    rev = link.counters(RETURN)
    assert (rev["credit_only_flits"], rev["wire_bytes"], rev["aou_message_bytes"],
            rev["unused_message_bytes"]) == (3, 768, 0, 720)
    assert link.credits(REQUEST) == 3
    for f in link.flits():
        assert f["grant_granules"] in (0, 1, 4, 8, 16, 32, 64, 128)
    link.close()


def test_slow_consume_and_capacity():
    # ucie_link_test.cpp:105-136
    link = o.Link(o.link_profile(ar=3, r=14, max_accepted=2))
    link.enqueue(RETURN, 1, 0)
    link.enqueue(RETURN, 2, 0)
    assert link.step() == []  # return data not delivered before serialization
    first = link.step()
    assert first == [(RETURN, 1, 2)]
    assert link.next_event_ns() is None  # unconsumed R made no phantom credit
    with pytest.raises(o.LinkError) as dup:
        link.enqueue(RETURN, 1, 2)
    assert dup.value.code == 1  # duplicate active message id
    with pytest.raises(o.LinkError) as full:
        link.enqueue(RETURN, 3, 2)
    assert full.value.code == 2  # in-flight direction capacity
    link.consume(RETURN, 1, 100)  # a deliberately slow caller
    second, granted = 0, 0
    for _ in range(20):
        if link.next_event_ns() is None:
            break
        for d, rid, at in link.step():
            if rid == 2:
                second = at
    for f in link.flits():
        if f["direction"] == REQUEST:
            granted += f["grant_granules"]
    assert granted == 14
    assert link.counters(REQUEST)["credit_only_flits"] == 4
    assert second >= 110
    link.consume(RETURN, 2, second)
    link.step()  # processes the consume: only now does capacity free
    link.enqueue(RETURN, 3, link.now())
    link.close()


def test_event_time_overflow_is_an_error():
    # ucie_link_test.cpp:174-181
    link = o.Link(o.link_profile())
    link.enqueue(REQUEST, 1, 2**64 - 1)
    with pytest.raises(o.LinkError) as e:
        link.step()
    assert e.value.code == 2
    link.close()


def test_legal_grant_encoding():
    # link.cpp:103-110: no two-granule grant; powers of two from 4 to 128
    L = o._link_lib()
    assert [L.orc_link_legal_grant(p) for p in (0, 1, 2, 3, 4, 7, 8, 15, 16, 200, 255, 256)] == \
        [0, 1, 1, 1, 4, 4, 8, 8, 16, 128, 128, 128]


def random_scenario(rng, n):
    direction = rng.integers(0, 2, n).astype(np.uint32)
    ready = np.sort(rng.integers(0, 20 * n, n)).astype(np.uint64)
    return direction, ready


@pytest.mark.parametrize("seed", range(12))
def test_scenario_invariants(seed):
    """Random two-direction streams through the scenario caller: every
    message is delivered once, in order within its direction, no earlier than
    its ready time plus one flit and the propagation; all of a direction's
    message granules cross the wire (3 per AR, 14 per R, 5 bytes each); every
    flit carries 48 granule slots; credits all come back at quiescence."""
    rng = np.random.default_rng(seed)
    prof = o.link_profile(gt=int(rng.choice([8, 16, 32])), ar=int(rng.integers(3, 40)),
                          r=int(rng.integers(14, 120)), max_accepted=int(rng.integers(1, 9)),
                          propagation_ns=int(rng.integers(0, 30)))
    n = int(rng.integers(1, 400))
    direction, ready = random_scenario(rng, n)
    delay = (int(rng.integers(0, 20)), int(rng.integers(0, 50)))
    delivered, counters = o.link_scenario(prof, direction, ready, delay)
    ser = 32 // prof.gt_per_second
    assert np.all(delivered >= ready + np.uint64(ser + prof.propagation_ns))
    for d, gran in ((REQUEST, 3), (RETURN, 14)):
        idx = np.nonzero(direction == d)[0]
        assert np.all(np.diff(delivered[idx].astype(np.int64)) >= 0)
        c = counters[d]
        assert c["aou_message_bytes"] == 5 * gran * len(idx)
        assert c["aou_message_bytes"] + c["unused_message_bytes"] == 240 * c["flits"]
        assert c["wire_bytes"] == 256 * c["flits"]
    # the same caller replayed on the object API: the same deliveries, and
    # every credit back at quiescence.  A consume scheduled at t before a
    # step at time now >= t has been processed by then (a step takes every
    # event at its time, in time order), which frees its slot.
    link = o.Link(prof)
    pending = {d: [i for i in range(n) if direction[i] == d] for d in (0, 1)}
    admitted = {0: 0, 1: 0}
    consumes = {0: [], 1: []}  # (time, steps taken when scheduled)
    steps = 0
    while True:
        for d in (0, 1):
            freed = sum(1 for t, k in consumes[d] if t <= link.now() and k < steps)
            while pending[d] and admitted[d] - freed < prof.max_accepted:
                i = pending[d].pop(0)
                link.enqueue(d, i + 1, max(int(ready[i]), link.now()))
                admitted[d] += 1
        if link.next_event_ns() is None:
            break
        delivered_now = link.step()
        steps += 1
        for d, rid, at in delivered_now:
            assert at == delivered[rid - 1]
            link.consume(d, rid, at + delay[d])
            consumes[d].append((at + delay[d], steps))
    assert not pending[0] and not pending[1]
    assert link.credits(REQUEST) == prof.initial_ar_granules
    assert link.credits(RETURN) == prof.initial_r_granules
    grants = {0: 0, 1: 0}
    for f in link.flits():
        grants[f["direction"]] += f["grant_granules"]
        assert f["grant_granules"] in (0, 1, 4, 8, 16, 32, 64, 128)
    # request flits return R credits, return flits AR credits
    assert grants[REQUEST] == 14 * int((direction == RETURN).sum())
    assert grants[RETURN] == 3 * int((direction == REQUEST).sum())
    link.close()


@pytest.mark.parametrize("gt,prop,direction,count", [
    (16, 10, REQUEST, 40), (8, 0, REQUEST, 17), (32, 7, RETURN, 9), (16, 100, RETURN, 30),
    (8, 3, REQUEST, 200)])
def test_back_to_back_flits_closed_form(gt, prop, direction, count):
    """With credits for every message and all of them ready at 0, the
    serializer never idles: message k (0-based) ends at granule s (k + 1) of
    the direction's granule stream (s = 3 per AR, 14 per R), rides flit
    f = ceil(s (k + 1) / 48) - 1, which leaves at f * ser, and is delivered
    at (f + 1) * ser + propagation."""
    size = 3 if direction == REQUEST else 14
    prof = o.link_profile(gt=gt, ar=max(3, 3 * count), r=max(14, 14 * count),
                          max_accepted=count, propagation_ns=prop)
    if direction == REQUEST and 3 * count > 65535 or direction == RETURN and 14 * count > 65535:
        pytest.skip("credits beyond the 16-bit counter")
    ser = 32 // gt
    delivered, counters = o.link_scenario(prof, [direction] * count, [0] * count, (0, 0))
    for k in range(count):
        f = -(-size * (k + 1) // 48) - 1
        assert int(delivered[k]) == (f + 1) * ser + prop, k
    assert counters[direction]["flits"] == -(-size * count // 48)
