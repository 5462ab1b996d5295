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


# ---- per-frame pad / truncate layout (mask_related.py:87-187) -------------------------------

FRAME_LENGTH = 1350  # CogVideoX-2B latent frame: 30 x 45 patches
FRAME_NUM = 13


def _layout(L, text_length, frame_length, frame_num, stride):
    if L != text_length + frame_length * frame_num:
        raise ValueError(f"expected {text_length} + {frame_num} x {frame_length} tokens, got {L}")
    rem = frame_length % stride
    pad = stride - rem if rem else 0
    return rem, pad


def padded_layout_maps(L, text_length=226, frame_length=FRAME_LENGTH, frame_num=FRAME_NUM, stride=64,
                       device=None):
    """Row maps of the query side of preprocess_qkv / reverse_process_out for the row-mapped
    attention: logical row i of the padded layout [frames padded to a multiple of `stride` |
    text] reads token q_rows[i] (-1 = zero padding) and its output goes to token o_rows[i]."""
    rem, pad = _layout(L, text_length, frame_length, frame_num, stride)
    fp = frame_length + pad
    i = torch.arange(frame_num * fp + text_length)
    f, s = i // fp, i % fp
    video = i < frame_num * fp
    tok = torch.where(video, text_length + f * frame_length + s, i - frame_num * fp)
    tok = torch.where(video & (s >= frame_length), torch.full_like(tok, -1), tok).int()
    return tok.to(device), tok.to(device)


def preprocess_qkv(q, k, v, stride=64, text_length=226, starts=None):
    """[text | 13 frames] -> q with every frame zero-padded to a multiple of `stride` and k, v
    with every frame cut to a multiple of `stride` at a random offset (one offset per batch
    item and frame, shared by heads, k and v, drawn as torch.randint(0, rem + 1, (B, 13))),
    text moved to the end. Returns (q, k, v) in the new layouts."""
    B, H, L, D = q.shape
    rem, pad = _layout(L, text_length, FRAME_LENGTH, FRAME_NUM, stride)
    qmap, _ = padded_layout_maps(L, text_length, FRAME_LENGTH, FRAME_NUM, stride, q.device)
    qp = gather_tokens(q, qmap)
    if rem == 0:
        keep = torch.arange(FRAME_NUM * FRAME_LENGTH) + text_length
        kmap = torch.cat([keep, torch.arange(text_length)]).int().to(q.device)
        return qp, gather_tokens(k, kmap), gather_tokens(v, kmap)
    if starts is None:
        starts = torch.randint(0, rem + 1, (B, FRAME_NUM), device=q.device)
    keep_len = FRAME_LENGTH - rem
    starts = starts.to("cpu").long()
    ks, vs = [], []
    for b in range(B):
        frames = [text_length + f * FRAME_LENGTH + int(starts[b, f]) + torch.arange(keep_len) for f in range(FRAME_NUM)]
        kmap = torch.cat(frames + [torch.arange(text_length)]).int().to(q.device)
        ks.append(gather_tokens(k[b:b + 1], kmap))
        vs.append(gather_tokens(v[b:b + 1], kmap))
    return qp, torch.cat(ks), torch.cat(vs)


def reverse_process_out(out, text_length=226, original_length=FRAME_LENGTH):
    """Inverse of the query-side layout: [padded frames | text] -> [text | frames]."""
    B, H, Lp, D = out.shape
    stride = 64
    fp = -(-original_length // stride) * stride
    if Lp != FRAME_NUM * fp + text_length:
        raise ValueError(f"expected {FRAME_NUM} x {fp} + {text_length} rows, got {Lp}")
    j = torch.arange(text_length + FRAME_NUM * original_length)
    t = j - text_length
    src = torch.where(j < text_length, FRAME_NUM * fp + j, (t // original_length) * fp + t % original_length)
    return gather_tokens(out, src.int().to(out.device))
