"""pack_records (hbfsim_amd.engine): the packed 16-byte form of 32-byte
records, bit layout and refusals, on CPU tensors."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hbfsim_amd.engine import pack_records


def t(rows):
    return torch.from_numpy(np.array(rows, np.uint64).view(np.int64))


def test_layout():
    rec = t([[0x7000_0000_1234, 128, 5_000_000, 0], [(1 << 48) - 1, 65535, (1 << 56) - 1, 1]])
    out = pack_records(rec).numpy().view(np.uint64)
    assert out[0, 0] == 0x7000_0000_1234 | (128 << 48)
    assert out[0, 1] == 5_000_000
    assert out[1, 0] == (1 << 64) - 1
    assert out[1, 1] == ((1 << 56) - 1) | (1 << 56)


@pytest.mark.parametrize("col,value", [(0, 1 << 48), (1, 1 << 16), (2, 1 << 56), (3, 256),
                                       (0, (1 << 64) - 1)])
def test_refuses_records_that_do_not_fit(col, value):
    row = [0x1000, 64, 0, 0]
    row[col] = value
    with pytest.raises(ValueError):
        pack_records(t([row, [0x2000, 64, 0, 0]]))
