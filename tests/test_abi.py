"""The C ABI library loads, exports every symbol include/sa_api.h declares, and rejects bad
arguments before touching the GPU (no compute calls here; runs without a GPU)."""
import ctypes
import math
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
    assert lib.sa_abi_version() == 3 == _lib.ABI_VERSION
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
    assert lib.sa_attn_split_parts(0, 128, 64, 256, ctypes.byref(parts)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_parts(4, 128, 96, 256, ctypes.byref(parts)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_parts(4, 128, 64, 0, ctypes.byref(parts)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_parts(4, 128, 64, 256, None) == _lib.SA_ERR_INVALID

    def q(n, w, d, cus=256):
        assert lib.sa_attn_split_parts(n, w, d, cus, ctypes.byref(parts)) == _lib.SA_OK
        return parts.value

    # A pure function of its arguments: min(slots / n, width / 32, 16) parts while the blocks
    # fill at most half of the slots (256 CUs x 8 waves at head dim 64, x 4 at 128), lists of
    # at least 64 positions.
    assert q(4, 63, 64) == 1
    assert q(4, 128, 64) == 4 and q(4, 705, 64) == 16 and q(4, 705, 128) == 16
    assert q(384, 705, 64) == 5 and q(384, 705, 128) == 2
    assert q(1024, 705, 64) == 2 and q(1025, 705, 64) == 1 and q(513, 705, 128) == 1
    assert q(384, 705, 64, cus=32) == 1 and q(8, 705, 64, cus=32) == 16
    assert [q(384, 705, 64) for _ in range(3)] == [5, 5, 5]


def test_split_workspace_query(lib):
    n = ctypes.c_int64(-1)
    assert lib.sa_attn_split_workspace(10, 64, 4, ctypes.byref(n)) == _lib.SA_OK
    assert n.value == 10 * 4 * (64 * 64 + 128) * 4
    assert lib.sa_attn_split_workspace(10, 128, 16, ctypes.byref(n)) == _lib.SA_OK
    assert n.value == 10 * 16 * (64 * 128 + 128) * 4
    assert lib.sa_attn_split_workspace(10, 64, 1, ctypes.byref(n)) == _lib.SA_OK and n.value == 0
    for bad in [(0, 64, 2), (10, 96, 2), (10, 64, 0), (10, 64, 17)]:
        assert lib.sa_attn_split_workspace(*bad, ctypes.byref(n)) == _lib.SA_ERR_INVALID
    assert lib.sa_attn_split_workspace(10, 64, 2, None) == _lib.SA_ERR_INVALID


def test_split_launch_validates_workspace(lib):
    # Rejected before any GPU work: parts out of range, no workspace, a short or misaligned one.
    dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    s3 = _lib.i64(0, 0, 0)
    B, H, Lq, Lk, D = 1, 2, 64, 8192, 64
    need = ctypes.c_int64(0)
    assert lib.sa_attn_split_workspace(B * H, D, 4, ctypes.byref(need)) == _lib.SA_OK

    def call(parts, ws, nbytes):
        return lib.sa_block_sparse_fwd_split(dummy, s3, dummy, s3, dummy, s3, dummy, s3, B, H, Lq, Lk, D, dummy,
                                             dummy, Lk // 64, 0.125, None, 0, None, 0, parts, ws, nbytes, None)

    assert call(0, dummy, need.value) == _lib.SA_ERR_INVALID and b"parts" in lib.sa_last_error()
    assert call(17, dummy, 1 << 30) == _lib.SA_ERR_INVALID and b"parts" in lib.sa_last_error()
    assert call(4, None, need.value) == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
    assert call(4, dummy, need.value - 1) == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
    assert call(4, ctypes.c_void_p(4104), need.value) == _lib.SA_ERR_INVALID
    assert b"aligned" in lib.sa_last_error()


def test_k16_workspace_query(lib):
    # fp16 copy of k (256-byte aligned), one norm per 64-row key block, then (with_bias) the
    # bias times log2(e), 256-byte aligned.
    n = ctypes.c_int64(-1)
    B, H, Lk = 2, 30, 17776
    k16 = (B * H * Lk * 64 * 2 + 255) // 256 * 256
    norms = B * H * math.ceil(Lk / 64) * 4
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 64, 0, ctypes.byref(n)) == _lib.SA_OK
    assert n.value == k16 + norms
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 64, 1, ctypes.byref(n)) == _lib.SA_OK
    assert n.value == (k16 + norms + 255) // 256 * 256 + B * H * Lk * 4
    # head dim 128: plain lists only (the pair kernel), a 128-wide fp16 copy of k
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 128, 0, ctypes.byref(n)) == _lib.SA_OK
    assert n.value == (B * H * Lk * 128 * 2 + 255) // 256 * 256 + norms
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 128, 1, ctypes.byref(n)) == _lib.SA_ERR_UNSUPPORTED
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 96, 0, ctypes.byref(n)) == _lib.SA_ERR_UNSUPPORTED
    assert lib.sa_block_sparse_fwd_k16_workspace(0, H, Lk, 64, 0, ctypes.byref(n)) == _lib.SA_ERR_INVALID
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, 64, 0, None) == _lib.SA_ERR_INVALID


def test_k16_launches_validate_workspace(lib):
    # fp16-score entry points reject a missing, short or misaligned workspace, a bias without
    # strides and other head dims before any GPU work.
    dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    s3 = _lib.i64(0, 0, 0)
    B, H, Lq, Lk, D = 1, 2, 128, 1024, 64
    need, need_b = ctypes.c_int64(0), ctypes.c_int64(0)
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, D, 0, ctypes.byref(need)) == _lib.SA_OK
    assert lib.sa_block_sparse_fwd_k16_workspace(B, H, Lk, D, 1, ctypes.byref(need_b)) == _lib.SA_OK

    def fwd(prepared, ws, nbytes, bias=None, bias_strides=None, d=D):
        return lib.sa_block_sparse_fwd_k16(dummy, s3, dummy, s3, dummy, s3, dummy, s3, B, H, Lq, Lk, d, dummy, dummy,
                                           Lk // 64, bias, bias_strides, 0.125, None, 0, prepared, ws, nbytes, None)

    for prepared in (0, 1):
        assert fwd(prepared, None, need.value) == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
        assert fwd(prepared, dummy, need.value - 1) == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
        assert fwd(prepared, ctypes.c_void_p(4096 + 16), need.value) == _lib.SA_ERR_INVALID
        assert b"aligned" in lib.sa_last_error()
        # head dim 128 needs the 128-wide workspace and no key bias; other head dims are refused
        assert fwd(prepared, dummy, need.value, d=128) == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
        assert fwd(prepared, dummy, need_b.value * 2, d=128, bias=dummy,
                   bias_strides=_lib.i64(H * Lk, Lk)) == _lib.SA_ERR_UNSUPPORTED
        assert fwd(prepared, dummy, need_b.value * 2, d=96) == _lib.SA_ERR_UNSUPPORTED
        # a key bias needs its strides, and the larger workspace
        assert fwd(prepared, dummy, need_b.value, bias=dummy) == _lib.SA_ERR_INVALID
        assert fwd(prepared, dummy, need.value, bias=dummy, bias_strides=_lib.i64(0, 0)) == _lib.SA_ERR_INVALID
        assert b"key_bias" in lib.sa_last_error()
    assert lib.sa_block_sparse_fwd_k16_prepare(dummy, s3, B, H, Lk, D, dummy, need.value - 1, None) == _lib.SA_ERR_INVALID
    assert lib.sa_block_sparse_fwd_k16_prepare(dummy, s3, B, H, Lk, 128, dummy, need.value, None) == \
        _lib.SA_ERR_INVALID
    assert lib.sa_block_sparse_fwd_k16_prepare(dummy, s3, B, H, Lk, 96, dummy, need.value * 2, None) == \
        _lib.SA_ERR_UNSUPPORTED
    assert lib.sa_block_pool_k16(dummy, s3, dummy, s3, B, H, Lk, D, dummy, dummy, dummy, need.value - 1,
                                 None) == _lib.SA_ERR_INVALID
    assert lib.sa_block_pool_k16(dummy, s3, None, s3, B, H, Lk, D, dummy, dummy, dummy, need.value,
                                 None) == _lib.SA_ERR_INVALID


def test_library_allocates_no_device_memory():
    # The only device buffer the library owns is the fixed scratch array of the no-alloc
    # matching entry point; no source calls an allocator or changes a memory pool.
    csrc = os.path.join(os.path.dirname(HEADER), "..", "sparseattnfunctions_amd", "csrc")
    names = sorted(f for f in os.listdir(csrc) if f.endswith((".hip", ".h")))
    assert "attn_fwd.hip" in names
    pat = re.compile(r"\bhip(Malloc|Free|MemPool|ExtMalloc|HostMalloc|MallocManaged|DeviceSetMemPool)\w*")
    for f in names:
        hits = pat.findall(open(os.path.join(csrc, f)).read())
        assert not hits, (f, hits)


def test_tome_match_workspace_checks(lib):
    # Sizes and alignment of the caller's workspace are checked before any GPU work (the map
    # pointers are placeholders that the validation never dereferences).
    from sparseattnfunctions_amd._tome import _MapsStruct
    G, ns, nd, r, T = 2, 12240, 5310, 4000, 226
    N = ns + nd
    maps = _MapsStruct(G, N, T, ns, nd, r, T + N, T + N - r, *([4096] * 15))
    need = ctypes.c_int64(0)
    assert lib.sa_tome_match_workspace(G, ns, nd, ctypes.byref(need)) == 0
    splits = 14  # 42 dst tiles of 128 in splits of 3
    assert need.value == max(G * splits * ns * 8, G * ((ns + 255) // 256) * 256 * 8)
    metric = ctypes.c_void_p(4096)
    rc = lib.sa_tome_match(metric, 64, ctypes.byref(maps), ctypes.c_void_p(4096 + 8), need.value, None)
    assert rc == _lib.SA_ERR_INVALID and b"16-byte aligned" in lib.sa_last_error()
    rc = lib.sa_tome_match(metric, 64, ctypes.byref(maps), ctypes.c_void_p(4096), need.value - 1, None)
    assert rc == _lib.SA_ERR_INVALID and b"workspace" in lib.sa_last_error()
