"""Token gather out[b, h, j] = x[b, h, idx[j]] on the GPU (`sa_gather_tokens`), used for the
layout permutations of the sliding-tile and the 1.5-5B rearranged attention."""
from __future__ import annotations

import torch

from . import _lib
from .utils.block_sparse_attn_kernel import _prep_qkv


def gather_tokens(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x bf16 or fp16 [B, H, L, D] (D a multiple of 8) on the GPU, idx int32 [L_out] on the same
    device -> [B, H, L_out, D]."""
    _lib.require_gpu(x, idx)
    x = _prep_qkv(x, (torch.bfloat16, torch.float16))
    idx = idx.to(torch.int32).contiguous()
    B, H, L, D = x.shape
    out = torch.empty(B, H, idx.numel(), D, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        rc = _lib.load().sa_gather_tokens(x.data_ptr(), _lib.i64(*x.stride()[:3]), B, H, L, D, idx.data_ptr(),
                                          idx.numel(), out.data_ptr(), _lib.i64(*out.stride()[:3]), _lib.stream_of(x))
    _lib.check(rc, "sa_gather_tokens")
    return out
