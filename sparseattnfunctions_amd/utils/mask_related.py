"""Block-score estimator helpers of special_attentions/utils/mask_related.py (:2-81), on MI355X.

  * `pad_to_multiple(x, multiple)` (:2-13): replicate padding of the sequence axis;
  * `random_sample_tokens(x, block_size, sample_num)` (:14-37): per 64-token block, the tokens
    at the `sample_num` largest of 64 uniform draws, in draw order;
  * `calc_attn_block_sum_efficient(q, k, block_size, num_keep)` (:40-81): softmax(sq.sk^T/8)
    over the sampled tokens, summed over num_keep x num_keep cells.
The sampling and the scores run in the HIP kernels of libsa_hip.so; torch draws the uniform
numbers (torch.rand [B, H, nb, 64], q first, then k, as the reference).

Differences from the reference, by design:
  * block_size must be 64 and head_dim 64 (NotImplementedError otherwise);
  * the block scores are fp32 (the reference returns bf16 sums of bf16 probabilities);
  * `calc_attn_block_sum_efficient` takes num_keep 8 or 16;
  * ties among draws (probability ~0) keep the lower position first.
"""
from __future__ import annotations

import math

import torch

from .._gather import gather_tokens
from ..estimator import sample_block_tokens, sampled_block_scores


def _check_block(block_size: int) -> None:
    if block_size != 64:
        raise NotImplementedError("the MI355X estimator uses 64-token blocks")


def pad_to_multiple(x: torch.Tensor, multiple: int) -> torch.Tensor:
    """Pads dim 2 of [B, H, L, D] to a multiple of `multiple` by repeating the last token."""
    L = x.size(2)
    if L % multiple == 0:
        return x
    Lp = math.ceil(L / multiple) * multiple
    idx = torch.clamp(torch.arange(Lp, device=x.device, dtype=torch.int32), max=L - 1)
    return gather_tokens(x, idx)


def random_sample_tokens(x: torch.Tensor, block_size: int = 64, sample_num: int = 8,
                         generator=None) -> torch.Tensor:
    """x [B, H, L, D] with L a multiple of block_size -> sampled [B, H, num_blocks*sample_num, D]."""
    _check_block(block_size)
    B, H, L, D = x.shape
    if L % block_size:
        raise ValueError(f"random_sample_tokens: L={L} is not a multiple of {block_size}")
    nb = L // block_size
    xs, _, _, _ = sample_block_tokens(x, None, sample_num, generator=generator)
    return xs[:, : nb * sample_num].reshape(B, H, nb * sample_num, D)


def calc_attn_block_sum_efficient(q: torch.Tensor, k: torch.Tensor, block_size: int = 64, num_keep: int = 16,
                                  generator=None) -> torch.Tensor:
    """Sampled block scores, fp32 [B, H, nb, nb] with nb = ceil(L / 64)."""
    _check_block(block_size)
    return sampled_block_scores(q, k, num_keep, generator=generator)
