"""Routed-expert trace events (trace_schema.json, as trace_collector.py
writes them) compiled into spans and records.  The fixture follows the
collector: per (token, layer) an event with the top-k experts and, per
expert in top-k order, its tensors (model_inventory.py:108-128) with page
bounds from the byte offsets and consecutive access-order sequences.  The
compiled records must equal a line-by-line expansion written out here; the
reference readers' rejections raise ValueError."""
from __future__ import annotations

import copy
import json

import numpy as np
import pytest

from hbfsim_amd import workloads as wl

PAGE = 16384
LINE = 128
SHARDS = {"model-00001.safetensors": 0x7000_0000_0000, "model-00002.safetensors": 0x7100_0000_0000}


def inventory(layers=3, experts=8, rng=None):
    """expert (layer, e) -> tensors [(name, shard, begin, end)], laid out
    back to back with odd sizes and alignments across two shards."""
    rng = rng or np.random.default_rng(0)
    inv, offset = {}, {k: 4096 + 8 for k in SHARDS}
    names = list(SHARDS)
    for layer in range(layers):
        for e in range(experts):
            tensors = []
            for kind in ("w13", "w2"):
                shard = names[(layer + e) % 2]
                size = int(rng.integers(1, 5 * PAGE))
                b = offset[shard]
                tensors.append((f"layers.{layer}.experts.{e}.{kind}", shard, b, b + size))
                offset[shard] = b + size + int(rng.integers(0, 300))
            inv[(layer, e)] = tensors
    return inv


def events_for(inv, routes, top_k=2):
    """routes[token][layer] = top-k ids -> schema-1 events, collector order."""
    out, seq = [], 0
    for token, layers in enumerate(routes):
        for layer, ids in enumerate(layers):
            begin = seq
            tensors = []
            for e in ids:
                for name, shard, b, end in inv[(layer, e)]:
                    tensors.append({"expert_id": e, "tensor": name, "tensor_kind": name[-3:],
                                    "source_shard": shard, "source_offset_begin": b,
                                    "source_offset_end": end, "tensor_bytes": end - b,
                                    "dtype": "bfloat16", "shape": [end - b],
                                    "page_begin": b // PAGE,
                                    "page_end": (end + PAGE - 1) // PAGE,
                                    "access_order_sequence": seq})
                    seq += 1
            out.append({"schema_version": 1, "run_id": "fixture", "request_id": "r0",
                        "sequence_id": 0, "prompt_id": 0, "phase": "decode",
                        "token_step": token, "layer_id": layer, "topk_expert_ids": list(ids),
                        "topk_weights": None, "expert_tensors": tensors,
                        "access_order_sequence_begin": begin, "access_order_sequence_end": seq,
                        "host_monotonic_timestamp_ns": 0, "gpu_event_timestamp_ns": None,
                        "previous_compute_gap_ns": None, "model_fingerprint": "0" * 64,
                        "environment_fingerprint": "0" * 64, "git_commit": "0" * 40})
    return out


def random_routes(rng, tokens, layers=3, experts=8, top_k=2):
    return [[[int(x) for x in rng.choice(experts, top_k, replace=False)] for _ in range(layers)]
            for _ in range(tokens)]


def expand(events, whole_pages=False):
    """Line-by-line record expansion: (addr, bytes, op) per line read."""
    rows = []
    for ev in events:
        for t in sorted(ev["expert_tensors"], key=lambda t: t["access_order_sequence"]):
            lo, hi = t["source_offset_begin"], t["source_offset_end"]
            if whole_pages:
                lo, hi = t["page_begin"] * PAGE, t["page_end"] * PAGE
            a = lo - lo % LINE
            while a < hi:
                rows.append((SHARDS[t["source_shard"]] + a, LINE, 0))
                a += LINE
    return rows


@pytest.mark.parametrize("whole_pages", [False, True])
def test_events_compile_to_line_reads(whole_pages):
    rng = np.random.default_rng(3)
    inv = inventory(rng=rng)
    events = events_for(inv, random_routes(rng, 5))
    lines = [json.dumps(e) for e in events]  # JSONL text and dicts both work
    base, first, op = wl.trace_event_spans(lines, SHARDS, PAGE, LINE, whole_pages=whole_pages)
    rec = wl.span_records(base, first, op, LINE, gap_ps=1000, issuers=4)
    want = expand(events, whole_pages)
    assert len(rec) == len(want)
    np.testing.assert_array_equal(rec[:, [0, 1, 3]], np.array(want, np.uint64))
    np.testing.assert_array_equal(rec[:, 2], (np.arange(len(rec)) // 4) * 1000)
    assert len(base) == sum(len(e["expert_tensors"]) for e in events)


def test_event_order_follows_access_sequence():
    """Tensors listed out of order inside an event compile in access order."""
    rng = np.random.default_rng(8)
    inv = inventory(rng=rng)
    events = events_for(inv, random_routes(rng, 2))
    shuffled = copy.deepcopy(events)
    for ev in shuffled:
        ev["expert_tensors"].reverse()
    a = wl.trace_event_spans(events, SHARDS, PAGE, LINE)
    b = wl.trace_event_spans(shuffled, SHARDS, PAGE, LINE)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("breakage", ["schema", "duplicate", "empty_topk", "pages", "gap",
                                      "foreign_expert", "shard", "no_events", "empty_range"])
def test_rejections(breakage):
    rng = np.random.default_rng(1)
    inv = inventory(rng=rng)
    events = events_for(inv, random_routes(rng, 2))
    ev = events[1]
    if breakage == "schema":
        ev["schema_version"] = 2
    elif breakage == "duplicate":
        ev["topk_expert_ids"] = [ev["topk_expert_ids"][0]] * 2
    elif breakage == "empty_topk":
        ev["topk_expert_ids"] = []
    elif breakage == "pages":
        ev["expert_tensors"][0]["page_end"] += 1
    elif breakage == "gap":
        for t in ev["expert_tensors"]:
            t["access_order_sequence"] += 1
        ev["access_order_sequence_begin"] += 1
        ev["access_order_sequence_end"] += 1
    elif breakage == "foreign_expert":
        ev["expert_tensors"][0]["expert_id"] = 99
    elif breakage == "shard":
        ev["expert_tensors"][0]["source_shard"] = "model-00009.safetensors"
    elif breakage == "no_events":
        events = []
    elif breakage == "empty_range":
        t = ev["expert_tensors"][0]
        t["source_offset_end"] = t["source_offset_begin"]
    with pytest.raises(ValueError):
        wl.trace_event_spans(events, SHARDS, PAGE, LINE)


@pytest.mark.gpu
def test_gpu_compiled_trace_matches_expansion_and_oracle():
    """The GPU span compiler's records of a trace equal the line expansion,
    and the engine times them bit-exactly against the oracle."""
    import torch

    import parity
    from test_gpu_parity import C2, check
    rng = np.random.default_rng(12)
    inv = inventory(layers=3, experts=8, rng=rng)
    events = events_for(inv, random_routes(rng, 40))
    base, first, op = wl.trace_event_spans(events, SHARDS, PAGE, LINE)
    rec = wl.gpu_span_records(base, first, op, LINE, gap_ps=2000, issuers=64)
    want = np.array(expand(events), np.uint64)
    got = rec.cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(got[:, [0, 1, 3]], want)
    torch.cuda.synchronize()
    ranges = [(b, 64 * 1024 * 1024, 1) for b in SHARDS.values()]
    p = parity.Pair(C2, ranges)
    try:
        (_, _, grep), _ = check(p, got.copy(), "routed-expert trace")
        assert grep["modeled"] == len(want)
        p.check_state()
    finally:
        p.close()
