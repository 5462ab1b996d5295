"""`BlockSparseAttention` processor of special_attentions/block_mask_attn.py (:5-29), on MI355X.

Called as `proc(q, k, v) -> out` with q, k, v bf16 [B, H, L, 64] on the GPU, text tokens
first then video in (t, h, w) order, exactly like the reference processor. The forward
builds the block mask of the mean-pool top-k rule on the GPU -- block means of q and k,
fp32 block scores, the top `int(nb * keep_ratio)` key blocks per query block, text block
rows and columns always kept (SparseGen_Plus.py:81-82) -- and runs the block-sparse
attention kernel on it.

Differences from the reference, by design:
  * `__call__` returns the output (the reference computes it and returns None, :26-29);
  * `forward` is the block-sparse path (the reference's `forward` is dense SDPA on a padded
    layout, :21-25); `forward_dense` runs the same kernel with every block kept;
  * `forward_backup` (:11-20) is the reference's frame-factored path: the frame-level mask
    of generate_attention_mask_frame_scope, the per-frame pad/truncate layout of
    preprocess_qkv, the first frame's inner block mask, their Kronecker fusion with dense text
    blocks, block-sparse attention and the inverse layout -- each a HIP kernel here (see
    utils/mask_related.py); it draws the same torch random numbers in the same order.
"""
from __future__ import annotations

import math

import torch

from ._kv import KVList, kv_list_from_mask
from .block_masks import meanpool_topk_kv_list
from .utils.block_sparse_attn_kernel import block_sparse_attention
from .workloads import COGVIDEOX_2B, Geometry, topk_count


def dense_kv_list(B: int, H: int, nqb: int, nkb: int, device) -> KVList:
    """Every key block for every query block (dense attention through the same kernel)."""
    idx = torch.arange(nkb, dtype=torch.int32, device=device).expand(B * H * nqb, nkb).contiguous()
    cnt = torch.full((B * H * nqb,), nkb, dtype=torch.int32, device=device)
    return KVList(idx, cnt, B, H, nqb, nkb, dense=True)


class BlockSparseAttention:
    def __init__(self, block_size: int = 64, keep_ratio: float = 0.2, geometry: Geometry = COGVIDEOX_2B,
                 sm_scale: float = 1 / 8):
        if block_size != 64:
            raise NotImplementedError("the MI355X kernel uses 64-token blocks")
        self.block_size = block_size
        self.sm_scale = sm_scale
        self.keep_ratio = keep_ratio
        self.geometry = geometry
        self.last_kv = None  # kv lists of the last call (sparsity statistics)

    def n_text_blocks(self) -> int:
        return math.ceil(self.geometry.text_len / self.block_size)

    def build_kv_list(self, q: torch.Tensor, k: torch.Tensor, with_fp16_keys: bool = False):
        """kv lists of the mean-pool top-k rule; with `with_fp16_keys`, (kv, fp16 keys made beside
        the top-k kernel) for block_sparse_attention(..., k16=...)."""
        nb = math.ceil(q.shape[2] / self.block_size)
        return meanpool_topk_kv_list(q, k, topk_count(self.keep_ratio, nb), self.n_text_blocks(),
                                     block=self.block_size, with_fp16_keys=with_fp16_keys)

    def forward(self, q, k, v):
        kv, k16 = self.build_kv_list(q, k, with_fp16_keys=True)
        self.last_kv = kv
        return block_sparse_attention(q, k, v, kv, self.sm_scale, n_text_blocks=self.n_text_blocks(), k16=k16)

    def forward_dense(self, q, k, v):
        B, H, L, _ = q.shape
        nb = math.ceil(L / self.block_size)
        return block_sparse_attention(q, k, v, dense_kv_list(B, H, nb, math.ceil(k.shape[2] / 64), q.device),
                                      self.sm_scale)

    def forward_backup(self, q, k, v, frame_draws=None, starts=None):
        """block_mask_attn.py:11-20: frame-level mask (generate_attention_mask_frame_scope),
        per-frame pad/truncate layout (preprocess_qkv), inner-frame mask of the first frame
        (get_inner_frame_mask, threshold 1), their fusion (get_block_mask), block-sparse
        attention on the processed layout and reverse_process_out. `frame_draws` / `starts`
        replace the two torch.randint draws (CPU: 60 first-frame positions; GPU: the (B, 13)
        truncation offsets) when given."""
        from .utils.mask_related import (generate_attention_mask_frame_scope, get_block_mask, get_inner_frame_mask,
                                         preprocess_qkv, reverse_process_out)

        outer = generate_attention_mask_frame_scope(q, k, draws=frame_draws)
        qp, kp, vp = preprocess_qkv(q, k, v, starts=starts)
        inner = get_inner_frame_mask(qp, kp)
        all_mask = get_block_mask(inner, outer)
        B, H = q.shape[:2]
        kv = kv_list_from_mask(all_mask, B, H, math.ceil(qp.shape[2] / 64), math.ceil(kp.shape[2] / 64))
        self.last_kv = kv
        out = block_sparse_attention(qp, kp, vp, kv, self.sm_scale)
        return reverse_process_out(out)

    def sparsity(self) -> float:
        """Fraction of skipped blocks in the last call."""
        kv = self.last_kv
        return 1.0 - kv.cnt.sum().item() / (kv.rows * kv.nkb)

    def __call__(self, q, k, v):
        return self.forward(q, k, v)
