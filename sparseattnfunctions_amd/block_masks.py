"""Block-mask construction on the GPU: mean-pooled block scores, per-row top-k, unions.

Every function here launches HIP kernels of libsa_hip.so; PyTorch only allocates the
outputs. Rules follow the reference's mask builders:
  * top-k per score row + scatter (utils/block_sparse_attn_kernel.py:31-39) with
    `k = int(nb * ratio)` (SparseGen_Plus.py:31,57);
  * text block rows and columns forced dense (SparseGen_Plus.py:81-82);
  * block scores from block means of q and k (the deterministic replacement of the sampled
    estimator, utils/mask_related.py:40-81).
Ties in the top-k break to the lowest key-block index (torch.topk leaves them unspecified).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._kv import KVList


def _prep(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"expected bfloat16, got {t.dtype}")
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def pool_blocks(q: torch.Tensor, k: Optional[torch.Tensor] = None, block: int = 64,
                k16_ws: Optional[torch.Tensor] = None):
    """Block means: bf16 [B,H,L,64] -> fp32 [B*H, ceil(L/block), 64] (for q and k). With
    `k16_ws` (block 64, uint8 of block_sparse_attn_kernel.k16_workspace_bytes bytes), the k
    pass also writes the fp16-score workspace of block_sparse_attention (`sa_block_pool_k16`)."""
    _lib.require_gpu(q, k)
    q = _prep(q)
    B, H, L, D = q.shape
    nb = math.ceil(L / block)
    qp = torch.empty(B * H, nb, D, dtype=torch.float32, device=q.device)
    kp = None
    if k is not None:
        k = _prep(k)
        if k.shape != q.shape:
            raise ValueError("pool_blocks: q and k must have the same shape")
        kp = torch.empty_like(qp)
    lib = _lib.load()
    if k16_ws is not None:
        if k is None or block != 64:
            raise ValueError("pool_blocks: k16_ws needs k and 64-token blocks")
        with torch.cuda.device(q.device):
            rc = lib.sa_block_pool_k16(q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                                       B, H, L, D, qp.data_ptr(), kp.data_ptr(), k16_ws.data_ptr(), k16_ws.numel(),
                                       _lib.stream_of(q))
        _lib.check(rc, "sa_block_pool_k16")
        return qp, kp
    with torch.cuda.device(q.device):
        rc = lib.sa_block_pool(
            q.data_ptr(), _lib.i64(*q.stride()[:3]),
            _lib.ptr(k), _lib.i64(*k.stride()[:3]) if k is not None else None,
            B, H, L, D, block, qp.data_ptr(), _lib.ptr(kp), _lib.stream_of(q),
        )
    _lib.check(rc, "sa_block_pool")
    return qp, kp


def topk_kv_list(q_pooled, k_pooled, B: int, H: int, topk: int, n_text_blocks: int,
                 local_bitmap: Optional[torch.Tensor] = None, scores_in: Optional[torch.Tensor] = None,
                 return_mask: bool = False, return_scores: bool = False):
    """Top-k (+ text, + local) selection -> KVList; optionally the dense uint8 mask and the
    fp32 scores ([B, H, nqb, nkb])."""
    if scores_in is not None:
        _lib.require_gpu(scores_in)
        scores_in = scores_in.to(torch.float32).contiguous()
        nqb, nkb = scores_in.shape[-2:]
        D = 0
        dev = scores_in.device
    else:
        _lib.require_gpu(q_pooled, k_pooled)
        nqb, D = q_pooled.shape[1], q_pooled.shape[2]
        nkb = k_pooled.shape[1]
        dev = q_pooled.device
    kv = KVList.empty(B, H, nqb, nkb, dev)
    mask = torch.empty(B, H, nqb, nkb, dtype=torch.uint8, device=dev) if return_mask else None
    scores = torch.empty(B, H, nqb, nkb, dtype=torch.float32, device=dev) if return_scores else None
    loc = None
    if local_bitmap is not None:
        if tuple(local_bitmap.shape) != (nqb, nkb):
            raise ValueError(f"local bitmap {tuple(local_bitmap.shape)} != ({nqb}, {nkb})")
        loc = local_bitmap.to(device=dev, dtype=torch.uint8).contiguous()
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.sa_block_topk_kv_list(
            _lib.ptr(q_pooled), _lib.ptr(k_pooled), _lib.ptr(scores_in), B * H, nqb, nkb, D,
            int(topk), int(n_text_blocks), _lib.ptr(loc), kv.idx.data_ptr(), kv.max_cnt,
            kv.cnt.data_ptr(), _lib.ptr(mask), _lib.ptr(scores),
            torch.cuda.current_stream(dev).cuda_stream,
        )
    _lib.check(rc, "sa_block_topk_kv_list")
    out = [kv]
    if return_mask:
        out.append(mask.bool())
    if return_scores:
        out.append(scores)
    return out[0] if len(out) == 1 else tuple(out)


def meanpool_topk_kv_list(q, k, topk: int, n_text_blocks: int, block: int = 64,
                          local_bitmap: Optional[torch.Tensor] = None, with_fp16_keys: bool = False, **kw):
    """q, k bf16 [B,H,L,64] -> kv lists of the mean-pool top-k rule (config 2; with a
    local bitmap, the combined rule of config 3). With `with_fp16_keys`, returns (kv, k16):
    the fp16 keys of block_sparse_attention's fp16 scores, written by the pooling pass, which
    reads k anyway (`sa_block_pool_k16`; k16 is None when block_sparse_attention's default
    takes no fp16 scores or the blocks are not 64 tokens)."""
    from .utils.block_sparse_attn_kernel import FP16Keys, fp16_keys_wanted, k16_workspace_bytes
    B, H, L = q.shape[:3]
    ws = None
    if with_fp16_keys and block == 64 and k.shape[3] == 64 and fp16_keys_wanted(k):
        ws = torch.empty(k16_workspace_bytes(B, H, L, 64), dtype=torch.uint8, device=k.device)
    qp, kp = pool_blocks(q, k, block, k16_ws=ws)
    k16 = None
    if ws is not None:
        stream = torch.cuda.current_stream(k.device)
        event = torch.cuda.Event()
        event.record(stream)
        k16 = FP16Keys(k, ws, stream, event)
    kv = topk_kv_list(qp, kp, B, H, topk, n_text_blocks, local_bitmap=local_bitmap, **kw)
    return (kv, k16) if with_fp16_keys else kv


_LOCAL_CACHE = {}


def local_window_bitmap(geom, window=(1, 8, 8), device=None) -> torch.Tensor:
    """Static local 3-D window of the combined mask, uint8 [nb, nb] on `device`, cached per
    (geometry, window, device). Built on the host by `sa_local_window_bitmap`."""
    key = (geom, tuple(window), str(device))
    bm = _LOCAL_CACHE.get(key)
    if bm is None:
        nb = math.ceil(geom.L / geom.block)
        host = torch.empty(nb, nb, dtype=torch.uint8)
        dt, dh, dw = window
        rc = _lib.load().sa_local_window_bitmap(geom.L, geom.block, geom.text_len, geom.T, geom.Hp, geom.Wp,
                                                dt, dh, dw, host.data_ptr())
        _lib.check(rc, "sa_local_window_bitmap")
        bm = host.to(device) if device is not None else host
        _LOCAL_CACHE[key] = bm
    return bm


def local_window_bitmap_perm(geom, perm: torch.Tensor, window=(1, 8, 8), device=None) -> torch.Tensor:
    """The local window for a permuted token layout (`sa_local_window_bitmap_perm`): uint8
    [nb, nb] with position j holding natural token perm[j], blocks compared by the (t, h, w)
    of their centre tokens, and every row/column of a block with a text token set. Built on
    the host, cached per (geometry, permutation, window, device)."""
    perm = perm.to(device="cpu", dtype=torch.int32).contiguous()
    key = (geom, tuple(window), str(device), perm.numel(), hash(perm.numpy().tobytes()))
    bm = _LOCAL_CACHE.get(key)
    if bm is None:
        nb = math.ceil(geom.L / geom.block)
        if perm.numel() != geom.L:
            raise ValueError(f"permutation of {perm.numel()} tokens for L={geom.L}")
        host = torch.empty(nb, nb, dtype=torch.uint8)
        dt, dh, dw = window
        rc = _lib.load().sa_local_window_bitmap_perm(geom.L, geom.block, geom.text_len, geom.T, geom.Hp, geom.Wp,
                                                     dt, dh, dw, perm.data_ptr(), host.data_ptr())
        _lib.check(rc, "sa_local_window_bitmap_perm")
        bm = host.to(device) if device is not None else host
        _LOCAL_CACHE[key] = bm
    return bm
