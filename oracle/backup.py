"""Frame-factored block mask of the reference's backup path -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Restates in fp64 with torch CPU ops (special_attentions/utils/mask_related.py):
  frame_scope_map  the sampled frame-to-frame attention map of
                   generate_attention_mask_frame_scope (:194-218): text tokens plus
                   `sample_num` first-frame positions repeated in every frame, scores
                   q.k * scale with the bf16-rounded log(sample_num / S) on the text keys,
                   softmax, then the frame-pair cell sums divided by sample_num;
  inner_cell_sums  attn_reduced of get_inner_frame_mask (:344-361): softmax of the first
                   q_len queries over the first k_len keys (calc_attn, :339-342), summed over
                   stride x stride cells;
  kron_mask        get_block_mask (:397-404): frame mask (x) inner mask, then `pad` dense rows
                   and columns.
The energy cuts that follow them are oracle_energy_list modes 2 and 3 (sa_oracle.c).

Pinned by tests/test_oracle_backup.py: pure-Python brute force on tiny geometries (explicit
exp/sum loops; explicit index loops for the Kronecker layout), the uniform-attention closed
forms, and the row-sum invariant of the cell sums.
"""
from __future__ import annotations

import torch


def composition(sample_num: int, S: int) -> float:
    """log(sample_num / S) computed in fp32 and rounded to bf16, as the reference adds it
    (:210-212: torch.log of an fp32 tensor, then .to(q.dtype))."""
    return float(torch.log(torch.tensor(sample_num / S, dtype=torch.float32)).to(torch.bfloat16))


def sampled_index(draws, text_length: int, f: int, S: int) -> torch.Tensor:
    """Text tokens, then the first-frame positions `draws` repeated in every frame (:199-204)."""
    first = torch.as_tensor(draws).to(torch.int64) + text_length
    return torch.cat([torch.arange(text_length), (first.view(1, -1) + (torch.arange(f) * S).view(-1, 1)).view(-1)])


def frame_scope_map(q, k, draws, text_length=226, f=13, S=1350, sample_num=60, scale=1 / 8):
    """img2img_map [B, H, f, f] in fp64."""
    idx = sampled_index(draws, text_length, f, S)
    qs, ks = q[:, :, idx].double(), k[:, :, idx].double()
    s = qs @ ks.transpose(-1, -2) * scale
    s[..., :text_length] += composition(sample_num, S)
    p = torch.softmax(s, dim=-1)
    B, H = q.shape[:2]
    video = p[:, :, text_length:, text_length:]
    return video.reshape(B, H, f, sample_num, f, sample_num).sum(dim=(3, 5)) / sample_num


def inner_cell_sums(q, k, original_length=1350, stride=64):
    """attn_reduced [B, H, q_len/stride, k_len/stride] in fp64."""
    rem = original_length % stride
    q_len = original_length + (stride - rem) if rem else original_length
    k_len = original_length - rem if rem else original_length
    s = q[:, :, :q_len].double() @ k[:, :, :k_len].double().transpose(-1, -2) / 8
    p = torch.softmax(s, dim=-1)
    B, H = q.shape[:2]
    return p.reshape(B, H, q_len // stride, stride, k_len // stride, stride).sum(dim=(3, 5))


def kron_mask(inner, frame, pad=4) -> torch.Tensor:
    """fp32 0/1 [B, H, F*Ri + pad, F*Ci + pad]."""
    B, H, F, _ = frame.shape
    Ri, Ci = inner.shape[-2:]
    fr = frame.bool()[:, :, :, None, :, None]
    inn = inner.bool()[:, :, None, :, None, :]
    video = (fr & inn).reshape(B, H, F * Ri, F * Ci).float()
    out = torch.ones(B, H, F * Ri + pad, F * Ci + pad)
    out[:, :, : F * Ri, : F * Ci] = video
    return out
