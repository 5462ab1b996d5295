"""Host table of cell-pattern token masks (sa_cell_tile_masks) for block masks whose blocks
are not 64 x 64 (sparse_attention_factory(BLOCK_M, BLOCK_N)), pinned by brute force."""
import ctypes
import random

import pytest
import torch

from sparseattnfunctions_amd import _lib


def _table(bm, bn):
    lib = _lib.load()
    n = ctypes.c_int64(0)
    assert lib.sa_cell_tile_masks(bm, bn, None, ctypes.byref(n)) == _lib.SA_OK
    t = torch.empty(n.value, 64, dtype=torch.int64)
    assert lib.sa_cell_tile_masks(bm, bn, t.data_ptr(), ctypes.byref(n)) == _lib.SA_OK
    return t


def _bits(word):
    w = int(word) & ((1 << 64) - 1)
    return [(w >> k) & 1 for k in range(64)]


@pytest.mark.parametrize("bm,bn", [(32, 32), (16, 64), (64, 16), (128, 32), (32, 256), (128, 128), (16, 16)])
def test_cell_tile_masks_brute_force(bm, bn):
    t = _table(bm, bn)
    cr = 64 // bm if bm < 64 else 1
    cc = 64 // bn if bn < 64 else 1
    assert t.shape == (1 << (cr * cc), 64)
    rng = random.Random(bm * 7 + bn)
    pats = range(t.shape[0]) if t.shape[0] <= 16 else [0, t.shape[0] - 1] + [rng.randrange(t.shape[0]) for _ in range(24)]
    for p in pats:
        for r in range(0, 64, 3 if t.shape[0] > 16 else 1):
            want = [(p >> ((r // min(bm, 64)) * cc + k // min(bn, 64))) & 1 for k in range(64)]
            assert _bits(t[p, r]) == want, (p, r)
    # the full pattern is every pair, the empty one none
    assert all(int(x) == -1 for x in t[-1]) and all(int(x) == 0 for x in t[0])


def test_cell_tile_masks_rejects_bad_sizes():
    lib = _lib.load()
    n = ctypes.c_int64(0)
    for bm, bn in [(8, 64), (64, 48), (2048, 64), (0, 64), (96, 64)]:
        assert lib.sa_cell_tile_masks(bm, bn, None, ctypes.byref(n)) == _lib.SA_ERR_INVALID
