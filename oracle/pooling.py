"""Dense attention with a 2-D max-pooled attention map on the CPU -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Restates attn_with_pooling (special_attentions/utils/attn_pooling_kernel.py:18-289) in
float64:
  P = softmax(q k^T * sm_scale), causal: keys c <= query r (:52-54); the key head of query
      head h is h // (H // H_kv) (:133-137, n_rep);
  out = P v;
  Po[i][j] = max over queries r of block i and keys c of block j of P[r][c]. The kernel
      keeps each row's block maxima of the scaled logits, R (:56-61). It turns them into
      probabilities with the row's final max and sum, exp2(R - m) / l (:80-103), and takes
      the maximum over the block's rows;
  Po[i][j] = 0 for j > i when causal (those entries are never written, :246);
  Po /= Po.sum(-1) (:285-287).
Only the L real rows take part in the maxima.

Pinned by tests/test_oracle_pooling.py against:
- closed forms for q = 0: P is uniform, so every Po row is uniform, and causal rows give
  Po[i][j] = 1 / (i + 1) for j <= i;
- a pure-Python brute force, with explicit exp and max loops, on tiny inputs with grouped
  key heads;
- PyTorch's SDPA for `out`.
"""
from __future__ import annotations

import torch


def pooled_attention(q, k, v, causal: bool, sm_scale: float, block_size: int, dtype=torch.float64):
    """(out [B,H,L,D], Po [B,H,nd,nd]) in `dtype`; k, v [B, H_kv, L, D] with H_kv | H."""
    B, H, L, D = q.shape
    rep = H // k.shape[1]
    q = q.to(dtype)
    k = k.to(dtype).repeat_interleave(rep, dim=1)
    v = v.to(dtype).repeat_interleave(rep, dim=1)
    s = q @ k.transpose(-1, -2) * sm_scale
    if causal:
        s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.softmax(s, dim=-1)
    out = p @ v
    nd = -(-L // block_size)
    pad = nd * block_size - L
    pp = torch.nn.functional.pad(p, (0, pad, 0, pad))  # probabilities >= 0: zero padding is inert
    po = pp.reshape(B, H, nd, block_size, nd, block_size).amax(dim=(3, 5))
    po = po / po.sum(dim=-1, keepdim=True)
    return out, po
