"""The C ABI library loads, exports every symbol include/sa_api.h declares, and rejects bad
arguments before touching the GPU (no compute calls here; runs without a GPU)."""
import ctypes
import os
import re

import pytest

from sparseattnfunctions_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "sa_api.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.exported_names())


def test_every_declared_symbol_is_exported(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.sa_abi_version() == 2 == _lib.ABI_VERSION
    assert lib.sa_last_error() is not None


def test_null_pointers_rejected(lib):
    st = _lib.i64(0, 0, 0, 0)
    rc = lib.sa_mask_to_kv_list(None, st, 1, 1, 1, 1, None, 1, None, None)
    assert rc == _lib.SA_ERR_INVALID
    assert b"null" in lib.sa_last_error()
    s3 = _lib.i64(0, 0, 0)
    rc = lib.sa_block_sparse_fwd(None, s3, None, s3, None, s3, None, s3, 1, 1, 64, 64, 64,
                                 None, None, 1, None, None, 0.125, None, 0, None)
    assert rc == _lib.SA_ERR_INVALID


def test_bad_shapes_rejected(lib):
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    s3 = _lib.i64(0, 0, 0)
    args = [dummy, s3, dummy, s3, dummy, s3, dummy, s3]
    rc = lib.sa_block_sparse_fwd(*args, 1, 1, 64, 64, 96, dummy, dummy, 2, None, None, 0.125, None, 0, None)
    assert rc == _lib.SA_ERR_UNSUPPORTED and b"head_dim" in lib.sa_last_error()
    rc = lib.sa_block_sparse_fwd(*args, 0, 1, 64, 64, 64, dummy, dummy, 2, None, None, 0.125, None, 0, None)
    assert rc == _lib.SA_ERR_INVALID
    rc = lib.sa_block_sparse_fwd(*args, 1, 1, 64, 64, 64, dummy, dummy, 2, None, None, -1.0, None, 0, None)
    assert rc == _lib.SA_ERR_INVALID and b"sm_scale" in lib.sa_last_error()
    st = _lib.i64(0, 0, 0, 0)
    rc = lib.sa_mask_to_kv_list(dummy, st, 1, 1, 2, 5, dummy, 4, dummy, None)
    assert rc == _lib.SA_ERR_INVALID and b"max_cnt" in lib.sa_last_error()


def test_check_maps_codes_to_exceptions(lib):
    lib.sa_mask_to_kv_list(None, _lib.i64(0, 0, 0, 0), 1, 1, 1, 1, None, 1, None, None)
    with pytest.raises(ValueError):
        _lib.check(_lib.SA_ERR_INVALID, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.SA_ERR_UNSUPPORTED, "x")
    with pytest.raises(_lib.SAError):
        _lib.check(_lib.SA_ERR_HIP, "x")


def test_work_order_is_a_permutation(lib):
    import ctypes
    import torch
    for B, H, nqb, nt in [(2, 30, 278, 4), (1, 1, 1, 0), (1, 3, 5, 2), (2, 30, 705, 4)]:
        n = ctypes.c_int64(0)
        assert lib.sa_attn_work_order(B, H, nqb, nt, 8, None, ctypes.byref(n)) == 0
        assert n.value % 4 == 0 and n.value >= B * H * nqb
        order = torch.empty(n.value, dtype=torch.int32)
        assert lib.sa_attn_work_order(B, H, nqb, nt, 8, order.data_ptr(), ctypes.byref(n)) == 0
        items = order[order >= 0]
        assert torch.equal(items.sort().values, torch.arange(B * H * nqb, dtype=torch.int32))
        # Within each XCD (dispatch index % 8), text rows come before video rows.
        slots = torch.arange(n.value)
        for x in range(8):
            mine = order[((slots // 4) % 8) == x]
            mine = mine[mine >= 0]
            text = (mine % nqb) < nt
            if text.any() and (~text).any():
                assert text.nonzero().max() < (~text).nonzero().min()


def test_split_parts_query(lib):
    parts = ctypes.c_int(-1)
    assert lib.sa_attn_split_parts(0, 128, 64, ctypes.byref(parts)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_parts(4, 128, 96, ctypes.byref(parts)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_parts(4, 128, 64, None) == _lib.SA_ERR_INVALID
    # lists narrower than 64 positions are never split (no device query needed)
    assert lib.sa_attn_split_parts(4, 63, 64, ctypes.byref(parts)) == _lib.SA_OK and parts.value == 1
    # wide lists: 1 without a GPU (no device to size against), else >= 1
    assert lib.sa_attn_split_parts(4, 128, 64, ctypes.byref(parts)) == _lib.SA_OK and parts.value >= 1
