"""Dense block-masked attention on the CPU -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the reference's own correctness oracle for the block-sparse kernel
(special_attentions/utils/block_sparse_attn_kernel.py:326-334): expand the block mask to
token level with a Kronecker product, `masked_fill(~mask, -inf)`, softmax, then P.V.
Query block m uses mask row m, as the kernel does (:155). A row with no allowed key
returns 0 (the reference kernel divides by zero there, :201-203; the HIP kernel writes 0).
An optional additive key bias restates the proportional-attention `attn_mask` of
MergeAttention.py:33-48.

Pinned by tests/test_oracle_attention.py against: PyTorch's own SDPA on an all-ones mask,
a pure-Python brute force on tiny inputs, closed forms (single allowed key, identical
keys), and invariance to the order of key blocks.
"""
from __future__ import annotations

import torch


def expand_block_mask(block_mask: torch.Tensor, Lq: int, Lk: int, block: int = 64) -> torch.Tensor:
    """bool [..., nqb, nkb] -> bool [..., Lq, Lk] (torch.kron of the reference, :326-328)."""
    m = block_mask.to(torch.bool)
    m = m.repeat_interleave(block, dim=-2).repeat_interleave(block, dim=-1)
    return m[..., :Lq, :Lk]


def masked_attention(q, k, v, block_mask, sm_scale, key_bias=None, block: int = 64,
                     dtype=torch.float64, row_chunk: int = 2048, heads=None, token_mask=None, rows=None):
    """Dense-masked attention on CPU tensors; returns [B, H, Lq, D] in `dtype`.

    q [B,H,Lq,D], k/v [B,H,Lk,D] (any float dtype; converted to `dtype`);
    block_mask broadcastable to [B, H, >=ceil(Lq/block), >=ceil(Lk/block)];
    key_bias broadcastable to [B, H, Lk] or None. `heads` optionally restricts the
    computation to a list of (b, h) pairs (the rest of the output stays zero).
    `token_mask(rows)` optionally returns a bool [len(rows), Lk] token-level mask that is
    intersected with the block mask (flex_attention's mask_mod semantics).
    `rows` (int64 [n], ascending query indices) computes only those query rows and returns
    [B, H, n, D]; every row is computed as in the full call.
    """
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    nqb = -(-Lq // block)
    nkb = -(-Lk // block)
    bm = block_mask.to(torch.bool)
    bm = bm.expand(B, H, bm.shape[-2], bm.shape[-1])[..., :nqb, :nkb]
    sel = torch.arange(Lq) if rows is None else rows.to(torch.int64)
    out = torch.zeros(B, H, sel.numel(), D, dtype=dtype)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    for b, h in pairs:
        kk = k[b, h].to(dtype)
        vv = v[b, h].to(dtype)
        bias = None
        if key_bias is not None:
            bias = key_bias.expand(B, H, Lk)[b, h].to(dtype)
        for r0 in range(0, sel.numel(), row_chunk):
            r1 = min(sel.numel(), r0 + row_chunk)
            ridx = sel[r0:r1]
            qq = q[b, h, ridx].to(dtype)
            s = (qq @ kk.T) * sm_scale
            if bias is not None:
                s = s + bias[None, :]
            allowed = bm[b, h][ridx // block].repeat_interleave(block, dim=-1)[:, :Lk]
            if token_mask is not None:
                allowed = allowed & token_mask(ridx)
            s = s.masked_fill(~allowed, float("-inf"))
            empty = ~allowed.any(dim=-1)
            s[empty] = 0.0
            p = torch.softmax(s, dim=-1)
            o = p @ vv
            o[empty] = 0.0
            out[b, h, r0:r1] = o
    return out


def flops_of_mask(block_mask, Lq: int, Lk: int, D: int = 64, block: int = 64) -> int:
    """Effective FLOPs of the computed tiles: 4 * D * (valid q rows) * (valid k cols)."""
    B, H, nqb, nkb = block_mask.shape
    nq = torch.clamp(Lq - torch.arange(nqb) * block, max=block).to(torch.int64)
    nk = torch.clamp(Lk - torch.arange(nkb) * block, max=block).to(torch.int64)
    m = block_mask[..., :nqb, :nkb].to(torch.int64).cpu()
    return int(4 * D * ((m * nk[None, None, None, :]).sum(-1) * nq[None, None, :]).sum())
