"""Block-sparse attention forward on MI355X (drop-in for the reference module of this name).

Mirrors special_attentions/utils/block_sparse_attn_kernel.py of xiaolong-li1/SparseAttnFunctions:
  * `block_sparse_triton_fn(q, k, v, block_sparse_mask, sm_scale)` (:293) -- same arguments,
    same asserts (:226-231), output allocated like `torch.empty_like(q)` (:228), forward only
    (backward raises NotImplementedError, :278-281);
  * `sparse_attention_factory` (:283-291; any power-of-two BLOCK_M x BLOCK_N from 16 to 1024,
    mapped onto 64 x 64 tiles with token-level masks where a tile is cut),
    `get_sparse_attn_mask_from_topk` (:31-39) and
    `get_sparse_attn_mask_from_threshold` (:42-47).
The name keeps "triton" for source compatibility; the work runs in the HIP kernels of
libsa_hip.so (`sa_mask_to_kv_list` + `sa_block_sparse_fwd`), not Triton.

Inputs are bf16 or fp16 (all three the same), head_dim 64 or 128 as the reference asserts
(:231); P is rounded to the input dtype before P.V as the reference rounds it to v's (:107).
fp32 inputs run the fp32 kernel (`sa_block_sparse_fwd_f32`: fp32 MFMA, P kept in fp32, as the
reference's cast to v's dtype leaves it), head_dim 64 or 128.

Differences from the reference, by design:
  * a query block whose mask row is empty yields 0 instead of NaN (:201-203);
  * sm_scale must be > 0.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from .. import _lib
from .._kv import KVList, kv_list_from_mask

BLOCK = 64


def _prep_qkv(t: torch.Tensor, dtypes=(torch.bfloat16,)) -> torch.Tensor:
    """bf16 (or another of `dtypes`), last dim contiguous, 16-byte aligned rows (the kernel's
    vector loads)."""
    if t.dtype not in dtypes:
        raise TypeError(f"expected {' or '.join(str(d) for d in dtypes)} tensors, got {t.dtype}")
    per16 = 16 // t.element_size()  # elements per 16 bytes
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % per16 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


N_XCD = 8  # MI355X: workgroups are dealt round-robin to 8 XCDs, each with its own L2
# MI355X compute units. The key-range split is sized for this fixed count rather than the
# runtime's, so that a launch's parts, and with them its output bits, depend on its shape only.
N_CU = 256


def split_parts(n_items: int, max_cnt: int, D: int) -> int:
    """Key-range parts per query block (`sa_attn_split_parts`) for a plain launch of n_items
    query blocks over lists of width max_cnt: 1 means one wave per block."""
    parts = ctypes.c_int(0)
    _lib.check(_lib.load().sa_attn_split_parts(int(n_items), int(max_cnt), int(D), N_CU, ctypes.byref(parts)),
               "sa_attn_split_parts")
    return parts.value


def split_workspace_bytes(n_items: int, D: int, parts: int) -> int:
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().sa_attn_split_workspace(int(n_items), int(D), int(parts), ctypes.byref(n)),
               "sa_attn_split_workspace")
    return n.value


def k16_workspace_bytes(B: int, H: int, Lk: int, D: int, with_bias: bool = False) -> int:
    """Bytes of the fp16-score workspace (`sa_block_sparse_fwd_k16_workspace`): an fp16 copy of k,
    the largest squared key-row norm of each 64-row key block and, with_bias, the key bias times
    log2(e)."""
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().sa_block_sparse_fwd_k16_workspace(int(B), int(H), int(Lk), int(D), int(bool(with_bias)),
                                                              ctypes.byref(n)),
               "sa_block_sparse_fwd_k16_workspace")
    return n.value

# Gate of the fp16 scores (block_sparse_attention's default and prepare_fp16_keys): with False,
# every launch takes the bf16 operands.
FP16_SCORES = True
# Dense lists take fp16 scores by default from this many query blocks and key blocks.
DENSE_FP16_BLOCKS = 128


class FP16Keys:
    """The fp16 copy of k and its per-head key norms for `block_sparse_attention(..., k16=...)`
    (`sa_block_sparse_fwd_k16_prepare`), made on `stream`; `event` marks its completion."""

    def __init__(self, k: torch.Tensor, ws: torch.Tensor, stream, event):
        self.key = (k.data_ptr(), tuple(k.shape), tuple(k.stride()))
        self.ws, self.stream, self.event = ws, stream, event

    def matches(self, k: torch.Tensor) -> bool:
        return self.key == (k.data_ptr(), tuple(k.shape), tuple(k.stride()))


def fp16_keys_wanted(k: torch.Tensor) -> bool:
    """Whether block_sparse_attention's default takes fp16 scores with this k (bf16 [B,H,Lk,D],
    D = 64 or 128)."""
    return FP16_SCORES and k.is_cuda and k.dtype == torch.bfloat16 and k.dim() == 4 and k.shape[3] in (64, 128)


def prepare_fp16_keys(k: torch.Tensor) -> Optional[FP16Keys]:
    """Enqueues the fp16 copy of k (bf16 [B,H,Lk,D], D = 64 or 128) on the current stream; None
    for other dtypes or head dims (those launches take no fp16 scores)."""
    if not fp16_keys_wanted(k):
        return None
    k_in, k = k, _prep_qkv(k, (torch.bfloat16,))
    B, H, Lk, D = k.shape
    ws = torch.empty(k16_workspace_bytes(B, H, Lk, D), dtype=torch.uint8, device=k.device)
    stream = torch.cuda.current_stream(k.device)
    with torch.cuda.device(k.device):
        rc = _lib.load().sa_block_sparse_fwd_k16_prepare(k.data_ptr(), _lib.i64(*k.stride()[:3]), B, H, Lk, D,
                                                          ws.data_ptr(), ws.numel(), stream.cuda_stream)
    _lib.check(rc, "sa_block_sparse_fwd_k16_prepare")
    event = torch.cuda.Event()
    event.record(stream)
    return FP16Keys(k_in, ws, stream, event)


_ORDER_CACHE = {}


def work_order(B: int, H: int, nqb: int, n_text_blocks: int, device) -> torch.Tensor:
    """Device copy of the attention dispatch order (`sa_attn_work_order`), cached per shape."""
    key = (B, H, nqb, n_text_blocks, str(device))
    order = _ORDER_CACHE.get(key)
    if order is None:
        lib = _lib.load()
        n = ctypes.c_int64(0)
        _lib.check(lib.sa_attn_work_order(B, H, nqb, n_text_blocks, N_XCD, None, ctypes.byref(n)), "sa_attn_work_order")
        host = torch.empty(n.value, dtype=torch.int32)
        _lib.check(lib.sa_attn_work_order(B, H, nqb, n_text_blocks, N_XCD, host.data_ptr(), ctypes.byref(n)),
                   "sa_attn_work_order")
        order = host.to(device)
        _ORDER_CACHE[key] = order
    return order


def _row_map(rows, device):
    if rows is None:
        return None
    if rows.dim() != 1:
        raise ValueError("row maps must be 1-D int32 tensors")
    return rows.to(device=device, dtype=torch.int32).contiguous()


def block_sparse_attention(q, k, v, kv: KVList, sm_scale: float, key_bias=None, out=None,
                           n_text_blocks: int = 0, q_rows=None, o_rows=None, tile_masks=None, v_cols: int = None,
                           fp16_scores: Optional[bool] = None, k16: Optional[FP16Keys] = None):
    """out = block-sparse softmax(q k^T * sm_scale [+ key_bias]) v over the blocks of `kv`.

    q [B,H,Lq,D], k/v [B,H,Lk,D] on the GPU, bf16 or fp16 (one dtype), D = 64 or 128, or fp32
    (plain lists only: fp32 MFMA, P kept in fp32 as the reference's kernel does);
    key_bias optional fp32 [B,H,Lk] (any strides with a contiguous key axis, stride 0 to
    broadcast). `n_text_blocks` only affects scheduling (those block rows are dispatched
    first).

    Layout remapping inside the kernel (no copies): with `q_rows` (int32 [n]) the attention
    runs over n logical query rows, row i reading q's row q_rows[i] (zeros outside q); with
    `o_rows` (int32 [n]) logical row i is written to out row o_rows[i] (dropped outside
    out). `tile_masks` = (kv_slot [rows, max_cnt] int32, masks uint64 [slots, 64],
    lists_shared) adds token-level masks inside cut blocks.

    `v_cols=32` (bf16, head dim 64, no row maps or tile masks): only v's first 32 columns
    enter P.V and the output is [B,H,Lq,32] (`sa_block_sparse_fwd_v32`; segment-indicator v).

    fp16 scores (`sa_block_sparse_fwd_k16`; plain or key-bias bf16 lists at head dim 64, plain
    ones at 128, no row maps, tile masks or key-range parts): an fp16 copy of k (exact for 2^-17 <= |k| < 65504)
    and q scaled by sm_scale*log2(e) into fp16 inside the kernel, so the softmax takes no
    multiply per score. A query block takes them only when max|q_i*sm_scale*log2(e)| *
    max|k_j| <= 32 (row norms; it bounds every exp2-domain score), which limits each score's
    change to about 2^-6; other blocks use the bf16 operands (`sa_block_sparse_fwd`, the
    arithmetic of every other mode). The fp16 copy of k costs one pass over k (about 2.8 ns
    per key block and head at C2 sizes, against about 0.03 ns saved per tile), which pays from
    about 100 tiles per key block: by default (`fp16_scores=None`) a launch takes fp16 scores
    when `k16` holds keys already made for this k (`prepare_fp16_keys`, or the pooling pass of
    the mask builders, `with_fp16_keys`; possibly on another stream, whose event this call's
    stream waits for) or when the lists are dense over at least DENSE_FP16_BLOCKS query and key
    blocks at head dim 64 (at 128 the pair kernel runs as fast on bf16 scores, 1.119 against
    1.116 ms on the C2 lists); fp16_scores=True makes the copy here, False never. FP16_SCORES = False turns the
    mode off everywhere.
    """
    _lib.require_gpu(q, k, v)
    types = (torch.bfloat16, torch.float16, torch.float32)
    k_in = k
    q, k, v = _prep_qkv(q, types), _prep_qkv(k, types), _prep_qkv(v, types)
    if not q.dtype == k.dtype == v.dtype:
        raise TypeError(f"q, k, v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    fp16 = q.dtype == torch.float16
    fp32 = q.dtype == torch.float32
    if fp32 and (key_bias is not None or q_rows is not None or o_rows is not None or tile_masks is not None):
        raise NotImplementedError("fp32 inputs: plain block lists only (no key_bias, row maps or tile masks)")
    B, H, Lsrc, D = q.shape
    q_rows, o_rows = _row_map(q_rows, q.device), _row_map(o_rows, q.device)
    Lq = q_rows.numel() if q_rows is not None else (o_rows.numel() if o_rows is not None else Lsrc)
    if q_rows is None and o_rows is not None and o_rows.numel() != Lsrc:
        raise ValueError("o_rows without q_rows must have one entry per q row")
    if q_rows is not None and o_rows is not None and o_rows.numel() != Lq:
        raise ValueError("q_rows and o_rows must have the same length")
    Lk = k.shape[2]
    if k.shape != (B, H, Lk, D) or v.shape != (B, H, Lk, D):
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if v_cols not in (None, D):
        if v_cols != 32 or D != 64 or q.dtype != torch.bfloat16 or q_rows is not None or o_rows is not None \
                or tile_masks is not None:
            raise NotImplementedError("v_cols=32: bf16, head dim 64, plain or key-bias lists only")
    Dout = D if v_cols is None else v_cols
    lists_shared = tile_masks is not None and tile_masks[2]
    want_rows = (1 if lists_shared else B * H) * math.ceil(Lq / BLOCK)
    if kv.rows != want_rows:
        raise ValueError(f"kv list has {kv.rows} rows, expected {want_rows}")
    if out is None:
        out = torch.empty_like(q) if o_rows is not None else torch.empty(B, H, Lq, Dout, dtype=q.dtype,
                                                                          device=q.device)
    elif out.shape[:2] != (B, H) or out.shape[3] != Dout or (o_rows is None and out.shape[2] != Lq):
        raise ValueError(f"out has shape {tuple(out.shape)}")
    bias_ptr, bias_strides = None, None
    if key_bias is not None:
        if key_bias.dtype != torch.float32 or key_bias.shape[-1] != Lk or key_bias.stride(-1) != 1:
            raise ValueError("key_bias must be fp32 [B,H,Lk] with a contiguous key axis")
        key_bias = key_bias.expand(B, H, Lk)
        bias_ptr, bias_strides = key_bias.data_ptr(), _lib.i64(key_bias.stride(0), key_bias.stride(1))
    lib = _lib.load()
    nqb = math.ceil(Lq / BLOCK)
    parts = 1
    if not fp32 and key_bias is None and tile_masks is None and Dout == D:
        parts = split_parts(B * H * nqb, kv.max_cnt, D)
    if parts > 1:
        # Few query blocks over long lists: key-range parts, their partials in a workspace
        # from the caching allocator on this stream (the kernels use it in stream order).
        ws = torch.empty(split_workspace_bytes(B * H * nqb, D, parts), dtype=torch.uint8, device=q.device)
        fn = "sa_block_sparse_fwd_split_f16" if fp16 else "sa_block_sparse_fwd_split"
        with torch.cuda.device(q.device):
            rc = getattr(lib, fn)(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                v.data_ptr(), _lib.i64(*v.stride()[:3]), out.data_ptr(), _lib.i64(*out.stride()[:3]),
                B, H, Lq, Lk, D, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, float(sm_scale),
                _lib.ptr(q_rows), Lsrc, _lib.ptr(o_rows), out.shape[2], parts, ws.data_ptr(), ws.numel(),
                _lib.stream_of(q))
        _lib.check(rc, fn)
        return out
    order = work_order(B, H, nqb, n_text_blocks, q.device)
    if q_rows is not None or o_rows is not None or tile_masks is not None:
        kv_slot, masks = (tile_masks[0], tile_masks[1]) if tile_masks is not None else (None, None)
        fn = "sa_block_sparse_fwd_mapped_f16" if fp16 else "sa_block_sparse_fwd_mapped"
        with torch.cuda.device(q.device):
            rc = getattr(lib, fn)(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                v.data_ptr(), _lib.i64(*v.stride()[:3]), out.data_ptr(), _lib.i64(*out.stride()[:3]),
                B, H, Lq, Lk, D, kv.idx.data_ptr(), kv.cnt.data_ptr(), _lib.ptr(kv_slot), kv.max_cnt,
                int(bool(lists_shared)), _lib.ptr(masks), bias_ptr, bias_strides, float(sm_scale),
                _lib.ptr(q_rows), Lsrc, _lib.ptr(o_rows), out.shape[2], order.data_ptr(), order.numel(),
                _lib.stream_of(q))
        _lib.check(rc, fn)
        return out
    if Dout == 32 and D == 64:
        with torch.cuda.device(q.device):
            rc = lib.sa_block_sparse_fwd_v32(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                v.data_ptr(), _lib.i64(*v.stride()[:3]), out.data_ptr(), _lib.i64(*out.stride()[:3]),
                B, H, Lq, Lk, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, bias_ptr, bias_strides,
                float(sm_scale), order.data_ptr(), order.numel(), _lib.stream_of(q))
        _lib.check(rc, "sa_block_sparse_fwd_v32")
        return out
    if fp16_scores is None:
        fp16_scores = k16 is not None or (D == 64 and kv.dense and min(kv.nqb, kv.nkb) >= DENSE_FP16_BLOCKS)
    fp16_scores = fp16_scores and FP16_SCORES
    if fp16_scores and not fp16 and not fp32 and (D == 64 or (D == 128 and key_bias is None)):
        # fp16 scores (`sa_block_sparse_fwd_k16`): an fp16 copy of k, and q scaled into the exp2
        # domain in fp16 inside the kernel, so the softmax needs no multiply per score; query
        # blocks whose score bound fails run on the bf16 operands.
        stream = torch.cuda.current_stream(q.device)
        if k16 is not None:
            if not k16.matches(k_in):
                raise ValueError("k16 was prepared for another k")
            if key_bias is not None:
                raise ValueError("k16 with key_bias: the prepared workspace holds no bias (pass fp16_scores=True)")
            stream.wait_event(k16.event)
            if k16.stream != stream:
                k16.ws.record_stream(stream)
            ws, prepared = k16.ws, 1
        else:
            ws = torch.empty(k16_workspace_bytes(B, H, Lk, D, with_bias=key_bias is not None), dtype=torch.uint8,
                             device=q.device)
            prepared = 0
        with torch.cuda.device(q.device):
            rc = lib.sa_block_sparse_fwd_k16(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                v.data_ptr(), _lib.i64(*v.stride()[:3]), out.data_ptr(), _lib.i64(*out.stride()[:3]),
                B, H, Lq, Lk, D, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, bias_ptr, bias_strides,
                float(sm_scale), order.data_ptr(), order.numel(), prepared, ws.data_ptr(), ws.numel(),
                stream.cuda_stream)
        _lib.check(rc, "sa_block_sparse_fwd_k16")
        return out
    fn = "sa_block_sparse_fwd_f16" if fp16 else ("sa_block_sparse_fwd_f32" if fp32 else "sa_block_sparse_fwd")
    with torch.cuda.device(q.device):
        rc = getattr(lib, fn)(
            q.data_ptr(), _lib.i64(*q.stride()[:3]),
            k.data_ptr(), _lib.i64(*k.stride()[:3]),
            v.data_ptr(), _lib.i64(*v.stride()[:3]),
            out.data_ptr(), _lib.i64(*out.stride()[:3]),
            B, H, Lq, Lk, D,
            kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt,
            bias_ptr, bias_strides, float(sm_scale),
            order.data_ptr(), order.numel(),
            _lib.stream_of(q),
        )
    _lib.check(rc, fn)
    return out


_CELL_MASKS = {}


def cell_tile_masks(block_m: int, block_n: int, device) -> torch.Tensor:
    """Device table of the 64 x 64 token masks of every cell pattern (`sa_cell_tile_masks`),
    cached per block shape."""
    key = (block_m, block_n, str(device))
    t = _CELL_MASKS.get(key)
    if t is None:
        lib = _lib.load()
        n = ctypes.c_int64(0)
        _lib.check(lib.sa_cell_tile_masks(block_m, block_n, None, ctypes.byref(n)), "sa_cell_tile_masks")
        host = torch.empty(n.value, 64, dtype=torch.int64)
        _lib.check(lib.sa_cell_tile_masks(block_m, block_n, host.data_ptr(), ctypes.byref(n)), "sa_cell_tile_masks")
        t = _CELL_MASKS[key] = host.to(device)
    return t


def cell_kv_list(mask: torch.Tensor, B: int, H: int, Lq: int, Lk: int, block_m: int, block_n: int):
    """(KVList of 64 x 64 tiles, kv_slot or None) for a block mask of block_m x block_n cells
    (`sa_mask_cells_to_kv_list`)."""
    _lib.require_gpu(mask)
    nM, nN = math.ceil(Lq / block_m), math.ceil(Lk / block_n)
    if mask.dim() != 4 or mask.shape[-2] < nM or mask.shape[-1] < nN:
        raise ValueError(f"block mask of shape {tuple(mask.shape)} for {nM} x {nN} blocks of {block_m} x {block_n}")
    m = mask.to(torch.bool).expand(B, H, mask.shape[-2], mask.shape[-1]).view(torch.uint8)
    nqb, nkb = math.ceil(Lq / BLOCK), math.ceil(Lk / BLOCK)
    kv = KVList.empty(B, H, nqb, nkb, mask.device)
    slot = None if (block_m >= BLOCK and block_n >= BLOCK) else torch.empty_like(kv.idx)
    with torch.cuda.device(mask.device):
        _lib.check(_lib.load().sa_mask_cells_to_kv_list(
            m.data_ptr(), _lib.i64(*m.stride()), B, H, Lq, Lk, block_m, block_n, kv.idx.data_ptr(), _lib.ptr(slot),
            kv.max_cnt, kv.cnt.data_ptr(), _lib.stream_of(m)), "sa_mask_cells_to_kv_list")
    return kv, slot


def _forward(ctx, q, k, v, block_sparse_mask, sm_scale, BLOCK_M=64, BLOCK_N=64, num_warps=None,
             num_stages=1, out=None):
    """Reference host wrapper semantics (block_sparse_attn_kernel.py:211-265). BLOCK_M x BLOCK_N
    other than 64 x 64 (powers of two, 16..1024): mask row m covers query rows m*BLOCK_M..,
    column n keys n*BLOCK_N.. (:139-155); the kernel runs 64 x 64 tiles, a tile cut by the mask
    with token-level masks (`sa_mask_cells_to_kv_list`)."""
    assert q.shape[-1] == k.shape[-1] == v.shape[-1]
    assert k.shape[2] == v.shape[2]
    assert q.shape[-1] in [64, 128]
    B, H, Lq, _ = q.shape
    Lk = k.shape[2]
    if BLOCK_M == BLOCK and BLOCK_N == BLOCK:
        kv = kv_list_from_mask(block_sparse_mask, B, H, math.ceil(Lq / BLOCK), math.ceil(Lk / BLOCK))
        return block_sparse_attention(q, k, v, kv, sm_scale, out=out)
    kv, slot = cell_kv_list(block_sparse_mask, B, H, Lq, Lk, int(BLOCK_M), int(BLOCK_N))
    if slot is None:
        return block_sparse_attention(q, k, v, kv, sm_scale, out=out)
    if q.dtype == torch.float32:
        raise NotImplementedError("fp32 inputs with blocks smaller than 64: the fp32 kernel has no token masks")
    return block_sparse_attention(q, k, v, kv, sm_scale, out=out,
                                  tile_masks=(slot, cell_tile_masks(int(BLOCK_M), int(BLOCK_N), q.device), False))


class _sparse_attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, block_sparse_dense, sm_scale):
        return _forward(ctx, q, k, v, block_sparse_dense, sm_scale)

    @staticmethod
    def backward(ctx, do):
        raise NotImplementedError("It does not support gradient propagation yet")


def sparse_attention_factory(BLOCK_M=64, BLOCK_N=64, **kwargs):
    class _sparse_attention_config(_sparse_attention):
        @staticmethod
        def forward(ctx, q, k, v, block_sparse_dense, sm_scale):
            return _forward(ctx, q, k, v, block_sparse_dense, sm_scale, BLOCK_M, BLOCK_N, **kwargs)

    return _sparse_attention_config.apply


block_sparse_triton_fn = _sparse_attention.apply


def get_sparse_attn_mask_from_topk(x, topk, use_dense_for_last_block=False):
    """Per-row top-k block mask (reference :31-39: `torch.topk` over the last axis, then
    `scatter_` into a bool [bsz, heads, n, n] mask; with `use_dense_for_last_block` the last
    two rows are set dense).

    The selection runs in `topk_kernel` (`sa_block_topk_kv_list` in its `scores_in` mode, no
    text blocks, no local window): the kept set of each row is the first `topk` columns in
    (score descending, column ascending) order. Scores are compared in fp32; bf16/fp16 inputs
    convert exactly, so the order is the input's. torch leaves the order of tied scores
    unspecified; here the lowest column wins. `x` is [bsz, heads, n, m] with m <= n and
    m <= 1024; columns m..n-1 of the mask stay False, as the reference's scatter leaves them.
    """
    from ..block_masks import topk_kv_list

    if x.dim() != 4:
        raise ValueError(f"get_sparse_attn_mask_from_topk: x must be 4-D, got {tuple(x.shape)}")
    bsz, num_head, n, m = x.shape
    topk = int(topk)
    if topk < 0 or topk > m:
        raise RuntimeError(f"selected index k out of range (topk={topk}, {m} columns)")
    if m > n:
        raise ValueError(f"get_sparse_attn_mask_from_topk: {m} columns > {n} rows (the mask is [n, n])")
    _lib.require_gpu(x)
    if not x.is_floating_point():
        raise TypeError(f"get_sparse_attn_mask_from_topk: floating-point scores expected, got {x.dtype}")
    dense_mask = torch.zeros(bsz, num_head, n, n, dtype=torch.bool, device=x.device)
    if topk > 0 and n > 0:
        _, sel = topk_kv_list(None, None, bsz, num_head, topk, 0,
                              scores_in=x.to(torch.float32).reshape(bsz * num_head, n, m), return_mask=True)
        dense_mask[..., :m] = sel
    if use_dense_for_last_block:
        dense_mask[:, :, -2:, :] = True
    return dense_mask


def get_sparse_attn_mask_from_threshold(x, threshold, use_dense_for_last_block=False):
    """Threshold block mask with lower-triangular restriction (reference :42-47)."""
    dense_mask = x > threshold
    if use_dense_for_last_block:
        dense_mask[:, :, -2:, :] = True
    dense_mask.tril_()
    return dense_mask


def is_hip() -> bool:
    """The reference's backend probe (Triton's active target is "hip" on ROCm): this build runs
    on HIP only."""
    return True
