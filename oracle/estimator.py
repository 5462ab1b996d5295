"""Sampled block-score estimator on the CPU -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates calc_attn_block_sum_efficient (special_attentions/utils/mask_related.py:40-81) with
its helpers pad_to_multiple (:2-13) and random_sample_tokens (:14-37), in float64:
  * per 64-token block, the positions of the `num_keep` largest of the block's 64 draws in
    (draw descending, position ascending) order -- torch.topk(sorted=True) of :27 -- with
    positions past L standing for token L-1 (replicate padding, :12);
  * a = softmax_j(sq_i . sk_j / 8) over all sampled tokens of the head (:66-67);
  * pooled[I][J] = sum of a over the num_keep x num_keep cell (conv2d with a ones kernel and
    stride num_keep, :71-77).

Pinned by tests/test_oracle_estimator.py against: the reference's own formulation run with
torch ops (replicate pad + topk + gather, conv2d with a ones kernel), softmax row sums
(sum_J pooled[I][J] = num_keep), and the closed form for q = 0 (pooled = num_keep / nb).
The selection of transfer_attn_to_mask is in sa_oracle.c (oracle_energy_list).
"""
from __future__ import annotations

import torch


def sample_tokens(rand: torch.Tensor, L: int, num_keep: int) -> torch.Tensor:
    """rand [B, H, nb, 64] -> int64 token ids [B, H, nb * num_keep]."""
    B, H, nb, blk = rand.shape
    order = torch.sort(rand.float(), dim=-1, descending=True, stable=True).indices[..., :num_keep]
    tok = torch.arange(nb).view(1, 1, nb, 1) * blk + order
    return torch.clamp(tok, max=L - 1).reshape(B, H, nb * num_keep)


def sampled_block_scores(q, k, rand_q, rand_k, num_keep: int, heads=None) -> torch.Tensor:
    """float64 [B, H, nb, nb]; `heads` optionally restricts to a list of (b, h) (others 0)."""
    B, H, L, D = q.shape
    nb = -(-L // 64)
    tq = sample_tokens(rand_q, L, num_keep)
    tk = sample_tokens(rand_k, L, num_keep)
    out = torch.zeros(B, H, nb, nb, dtype=torch.float64)
    for b, h in heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]:
        sq = q[b, h].double()[tq[b, h]]
        sk = k[b, h].double()[tk[b, h]]
        a = torch.softmax(sq @ sk.T / 8, dim=-1)
        out[b, h] = a.reshape(nb, num_keep, nb, num_keep).sum(dim=(1, 3))
    return out
