"""Compacted per-row block lists ("kv lists") that drive the block-sparse attention kernel.

A kv list replaces the dense boolean block mask of the reference
(`block_mask bool[B, H, ceil(Lq/64), ceil(Lk/64)]`, utils/block_sparse_attn_kernel.py:141,155):
row r = (b*H + h)*nqb + m holds, ascending, the key-block indices that query block m of
head (b, h) attends to. It is built once per call on the GPU instead of every kernel
program re-reading the whole mask row.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class KVList:
    idx: torch.Tensor  # int32 [rows, max_cnt]
    cnt: torch.Tensor  # int32 [rows]
    B: int
    H: int
    nqb: int
    nkb: int
    dense: bool = False  # every row lists every key block (set by the dense-list builders)

    @property
    def rows(self) -> int:
        return self.cnt.numel()

    @property
    def max_cnt(self) -> int:
        return self.idx.shape[1]

    @staticmethod
    def empty(B: int, H: int, nqb: int, nkb: int, device) -> "KVList":
        rows = B * H * nqb
        return KVList(
            torch.empty(rows, nkb, dtype=torch.int32, device=device),
            torch.empty(rows, dtype=torch.int32, device=device),
            B, H, nqb, nkb,
        )

    def to_mask(self) -> torch.Tensor:
        """Dense bool [B, H, nqb, nkb] view of the lists (for inspection and tests)."""
        rows = self.rows
        pos = torch.arange(self.max_cnt, device=self.cnt.device)
        valid = pos[None, :] < self.cnt[:, None].long()
        mask = torch.zeros(rows, self.nkb + 1, dtype=torch.bool, device=self.cnt.device)
        idx = torch.where(valid, self.idx.long(), torch.full_like(self.idx.long(), self.nkb))
        mask.scatter_(1, idx, True)
        return mask[:, : self.nkb].reshape(self.B, self.H, self.nqb, self.nkb)

    def computed_pairs(self, Lq: int, Lk: int, block: int = 64) -> int:
        """Number of valid (query, key) pairs in the listed tiles (partial tiles counted at
        their valid size): the work unit of the effective-FLOP count."""
        nq = torch.clamp(Lq - torch.arange(self.nqb, device=self.cnt.device) * block, max=block)
        nk = torch.clamp(Lk - torch.arange(self.nkb, device=self.cnt.device) * block, max=block)
        mask = self.to_mask()
        per_row = (mask.to(torch.int64) * nk[None, None, None, :]).sum(-1)
        return int((per_row * nq[None, None, :]).sum().item())


def kv_list_from_mask(mask: torch.Tensor, B: int, H: int, nqb: int, nkb: int) -> KVList:
    """Dense block mask -> KVList on the GPU (`sa_mask_to_kv_list`).

    `mask` is any bool/integer tensor broadcastable to [B, H, >=nqb, >=nkb]; only rows
    [0, nqb) and columns [0, nkb) are read, as the reference kernel does (:155, :165).
    """
    _lib.require_gpu(mask)
    if mask.dim() != 4:
        raise ValueError(f"block mask must be 4-D [B,H,nqb,nkb], got {tuple(mask.shape)}")
    if mask.shape[-2] < nqb or mask.shape[-1] < nkb:
        raise ValueError(f"block mask {tuple(mask.shape)} smaller than the block grid ({nqb}, {nkb})")
    if mask.dtype == torch.bool:
        m8 = mask.view(torch.uint8)
    else:
        m8 = (mask != 0).view(torch.uint8)
    m8 = m8.expand(B, H, m8.shape[2], m8.shape[3])
    kv = KVList.empty(B, H, nqb, nkb, mask.device)
    lib = _lib.load()
    with torch.cuda.device(mask.device):
        rc = lib.sa_mask_to_kv_list(
            m8.data_ptr(), _lib.i64(*m8.stride()), B, H, nqb, nkb,
            kv.idx.data_ptr(), kv.max_cnt, kv.cnt.data_ptr(), _lib.stream_of(mask),
        )
    _lib.check(rc, "sa_mask_to_kv_list")
    return kv
