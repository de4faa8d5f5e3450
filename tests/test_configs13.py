"""The workload builders of configs 1 (TinyLlama-1.1B weight streaming) and 3
(paged KV cache with appends), checked on the host against the
configurations' own arithmetic."""
from __future__ import annotations

import numpy as np

from hbfsim_amd import workloads as w


def test_tinyllama_step_reads_every_tensor_once():
    s = w.TINYLLAMA
    base, first, op = w.dense_spans(s)
    layout = s.layout()
    assert len(base) == len(layout) == 3 + 9 * s.layers  # embed, norm, lm_head
    total = sum(n for _, n in layout)
    assert 2.19e9 < total < 2.21e9                       # ~2.2 GB of bf16 weights
    assert int(first[-1]) == sum(-(-n // 128) for _, n in layout)
    assert not op.any()
    # tensors are disjoint and page aligned, and each span reads its tensor
    starts = np.array([b for b, _ in layout], np.uint64)
    assert (starts % np.uint64(s.page) == 0).all()
    ends = starts + np.array([n for _, n in layout], np.uint64)
    assert (ends[:-1] <= starts[1:]).all()
    np.testing.assert_array_equal(base, starts)
    # a 1.1B-parameter model: 22 x (4 attention + 3 MLP matrices + 2 norms) + embed, norm, head
    params = total // 2
    assert 1.09e9 < params < 1.11e9


def test_span_records_follow_spans():
    base = np.array([1 << 40, 5 << 40, 9 << 40], np.uint64)
    first = np.array([0, 3, 3, 7], np.uint64)            # an empty span in the middle
    op = np.array([0, 1, 1], np.uint32)
    rec = w.span_records(base, first, op, 128, 1000, 2)
    assert rec.shape == (7, 4)
    np.testing.assert_array_equal(rec[:, 0], [1 << 40, (1 << 40) + 128, (1 << 40) + 256,
                                              9 << 40, (9 << 40) + 128, (9 << 40) + 256,
                                              (9 << 40) + 384])
    np.testing.assert_array_equal(rec[:, 2], [0, 0, 1000, 1000, 2000, 2000, 3000])
    np.testing.assert_array_equal(rec[:, 3], [0, 0, 0, 1, 1, 1, 1])
    np.testing.assert_array_equal(w.span_records(base, first, op, 128, 1000, 2, 2, 3), rec[2:5])


def kv_expect(shape, step):
    lens = shape.lengths() + step
    appends = 2 * shape.layers * shape.seqs
    wlines = shape.token_bytes // shape.line
    # an append that ends on a page boundary programs the page
    per_page = shape.page // shape.token_bytes
    fills = int(((lens % per_page) == per_page - 1).sum()) * 2 * shape.layers
    reads = 2 * shape.layers * int(((lens + 1) * (shape.token_bytes // shape.line)).sum())
    return appends * wlines, fills, reads


def test_kv_steps_match_the_configuration():
    shape = w.PagedKvShape(layers=3, seqs=7, min_len=20, max_len=300, steps=4)
    tables = shape.tables()
    for step in range(shape.steps):
        base, first, op = w.kv_spans(shape, step, tables)
        rec = w.span_records(base, first, op, shape.line, shape.gap_ps, shape.issuers)
        writes, fills, reads = kv_expect(shape, step)
        assert int((rec[:, 3] == 1).sum()) == writes
        assert len(rec) - writes == reads
        # page-filling write lines: the last line of an append that ends a page
        wr = rec[rec[:, 3] == 1]
        ends = (wr[:, 0] + wr[:, 1]) % np.uint64(shape.page) == 0
        assert int(ends.sum()) == fills
        # every access stays inside its layer's pool of blocks
        lo = min(b for b, _, _ in w.kv_ranges(shape))
        hi = max(b + n for b, n, _ in w.kv_ranges(shape))
        assert (rec[:, 0] >= lo).all() and (rec[:, 0] + rec[:, 1] <= hi).all()


def test_kv_full_size_shape():
    s = w.PAGED_KV
    lens = s.lengths()
    assert lens.min() >= 1024 and lens.max() <= 32768 and len(lens) == 64
    # 2 x 32 pools of 16-token blocks, bf16 K and V for 8 heads x 128
    assert s.block_bytes == 16 * 8 * 128 * 2
    assert 2 * s.layers * s.pool_bytes() < 256 * 2**30  # fits the c3 profile
