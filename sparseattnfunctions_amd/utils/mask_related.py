"""Block-score estimator helpers of special_attentions/utils/mask_related.py (:2-81), on MI355X.

  * `pad_to_multiple(x, multiple)` (:2-13): replicate padding of the sequence axis;
  * `random_sample_tokens(x, block_size, sample_num)` (:14-37): per 64-token block, the tokens
    at the `sample_num` largest of 64 uniform draws, in draw order;
  * `calc_attn_block_sum_efficient(q, k, block_size, num_keep)` (:40-81): softmax(sq.sk^T/8)
    over the sampled tokens, summed over num_keep x num_keep cells;
  * `preprocess_qkv` / `reverse_process_out` (:87-187): the per-frame pad/truncate layout;
  * `generate_attention_mask_frame_scope` (:194-245), `calc_attn` / `get_inner_frame_mask`
    (:339-395) and `get_block_mask` (:397-404): the frame-factored block mask of
    block_mask_attn.forward_backup.
The sampling and the scores run in the HIP kernels of libsa_hip.so; torch draws the uniform
numbers (torch.rand [B, H, nb, 64], q first, then k, as the reference).

Differences from the reference, by design:
  * block_size must be 64 and head_dim 64 (NotImplementedError otherwise);
  * the block scores are fp32 (the reference returns bf16 sums of bf16 probabilities);
  * `calc_attn_block_sum_efficient` takes num_keep 8 or 16;
  * ties among draws (probability ~0) keep the lower position first;
  * the frame-scope and inner-frame masses are fp32 softmax masses rounded to bf16 per row
    and summed in fp32 (the reference keeps bf16 scores, softmax and sums), and the energy
    cuts compare against the fp32 sum in sorted order; calc_attn's softmax is fp32;
  * get_block_mask takes B and H from its inputs (the reference reshapes to (2, 30)).
"""
from __future__ import annotations

import math

import torch

from .. import _lib
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


# ---- frame-factored block mask of the backup path (mask_related.py:194-245, 339-404) --------

def generate_attention_mask_frame_scope(q, k, text_length=226, f=13, width=45, height=30, sample_num=60,
                                        scale_factor=1 / 8, base_threshold=0.9, draws=None):
    """Frame-level mask [B, H, f, f] (bool) of the reference (:194-245).

    Sampled attention: the text tokens plus `sample_num` first-frame positions repeated in every
    frame (`draws`, int [sample_num]; default `torch.randint(0, width*height, (sample_num,))`
    on the CPU generator, as the reference draws them, :200). Scores q.k * scale_factor with
    log(sample_num / (width*height)) (rounded to bf16, as the reference adds it) on the text
    keys; img2img[f1][f2] = the softmax mass of frame f1's sampled queries on frame f2's sampled
    keys, summed over the queries and divided by sample_num (:213-218). Per head, the f*f map
    is sorted descending and kept through the first entry whose cumulative sum reaches
    base_threshold of the total (:224-238).

    The masses come from the attention kernel with a 0/1 segment-indicator v (fp32 softmax,
    bf16 outputs; the reference rounds scores and softmax to bf16), summed by
    `sa_pattern_maps`; the cut runs in `sa_energy_kv_list` (mode 2).
    """
    from ..estimator import energy_mask

    img2img = frame_scope_map(q, k, text_length, f, width, height, sample_num, scale_factor, draws)
    B, H = q.shape[:2]
    return energy_mask(img2img.reshape(B * H, 1, f * f), "inclusive", base_threshold).reshape(B, H, f, f)


def frame_scope_map(q, k, text_length=226, f=13, width=45, height=30, sample_num=60, scale_factor=1 / 8,
                    draws=None):
    """img2img_map of generate_attention_mask_frame_scope (:199-218): fp32 [B, H, f, f]."""
    from ..partern_attention import ParternAttentionColVersion_V2, PatternGeometry

    S = width * height
    if draws is None:
        draws = torch.randint(0, S, (sample_num,))
    draws = torch.as_tensor(draws).to(device="cpu", dtype=torch.int64).reshape(-1)
    if draws.numel() != sample_num or int(draws.min()) < 0 or int(draws.max()) >= S:
        raise ValueError(f"draws must be {sample_num} positions in [0, {S})")
    g = PatternGeometry(frames=f, height=height, width=width, text_length=text_length, sample_num=sample_num)
    first = draws + text_length
    all_idxs = (first.view(1, -1) + (torch.arange(f) * S).view(-1, 1)).view(-1)
    index_k = torch.cat([torch.arange(text_length), all_idxs])
    img2img, _ = ParternAttentionColVersion_V2(g).get_weight_for_patch(q, k, index_k, sm_scale=scale_factor)
    return img2img


def calc_attn(q, k):
    """softmax(q k^T / 8) over the keys (:339-342): fp32 probabilities of `sa_sampled_probs`
    (scores and softmax in fp32), returned in q's dtype as the reference's."""
    from ..partern_attention import _compact, _pad32, _probs

    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    if D != 64 or k.shape[:2] != (B, H) or k.shape[3] != D:
        raise ValueError(f"calc_attn: q {tuple(q.shape)} and k {tuple(k.shape)} must be [B, H, L, 64]")
    qs = _compact(q, torch.arange(Lq), _pad32(Lq))
    ks = _compact(k, torch.arange(Lk), _pad32(Lk))
    P = torch.empty(B * H, Lq, Lk, dtype=torch.float32, device=q.device)
    _probs(qs, ks, Lq, Lk, 0, 0.0, 0, Lk, P, sm_scale=1 / 8)
    return P.view(B, H, Lq, Lk).to(q.dtype)


def inner_frame_cell_sums(q, k, original_length=FRAME_LENGTH, stride=64):
    """attn_reduced of get_inner_frame_mask (:348-361): the softmax of the first
    q_len = original_length rounded up to `stride` queries over the first k_len = rounded
    down keys, summed over stride x stride cells -> fp32 [B, H, q_len/stride, k_len/stride].
    Each query row's mass per key block is the attention kernel's output with a 0/1 key-block
    indicator as v (fp32 softmax, bf16 output); `sa_row_group_sums` adds the rows of a cell."""
    from ..block_mask_attn import dense_kv_list
    from .block_sparse_attn_kernel import block_sparse_attention

    if stride != 64:
        raise NotImplementedError("the MI355X kernels use 64-token blocks")
    rem = original_length % stride
    q_len = original_length + (stride - rem) if rem else original_length
    k_len = original_length - rem if rem else original_length
    B, H = q.shape[:2]
    if q.shape[2] < q_len or k.shape[2] < k_len:
        raise ValueError(f"need {q_len} query and {k_len} key tokens, got {q.shape[2]} and {k.shape[2]}")
    Qr, Kr = q_len // stride, k_len // stride
    if Kr > 64:
        raise NotImplementedError(f"{Kr} key blocks per frame (at most 64)")
    ind = torch.zeros(k_len, 64, dtype=torch.bfloat16)
    ind[torch.arange(k_len), torch.arange(k_len) // stride] = 1
    ind = ind.to(q.device).expand(B, H, k_len, 64)
    mass = block_sparse_attention(q[:, :, :q_len], k[:, :, :k_len], ind, dense_kv_list(B, H, Qr, Kr, q.device),
                                  1 / 8, v_cols=32 if Kr <= 32 and q.dtype == torch.bfloat16 else None)
    out = torch.empty(B, H, Qr, Kr, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        rc = _lib.load().sa_row_group_sums(mass.data_ptr(), _lib.i64(*mass.stride()[:3]), B, H, q_len, stride, 0, Kr,
                                           out.data_ptr(), _lib.stream_of(mass))
    _lib.check(rc, "sa_row_group_sums")
    return out


def get_inner_frame_mask(q, k, scope="row", original_length=FRAME_LENGTH, stride=64, threshold=1):
    """Block mask inside a frame (:344-395), from the first frame of the processed layout
    (q padded, k truncated per frame, preprocess_qkv): bool [B, H, q_len/stride, k_len/stride].
    scope "row": per query block, keep the key blocks through the first sorted position whose
    cumulative mass reaches threshold * the row's total (:363-376); scope "head": over the
    whole map, keep the sorted positions whose cumulative mass stays <= threshold * total, and
    the last (:378-391). The totals are the sequential fp32 sums in sorted order (the
    reference also compares against `attn_reduced.sum(-1)` in bf16 for the row scope)."""
    from ..estimator import energy_mask

    assert 0 < threshold <= 1, "Threshold需在(0,1]范围内"
    cells = inner_frame_cell_sums(q, k, original_length, stride)
    B, H, Qr, Kr = cells.shape
    if scope == "row":
        return energy_mask(cells.reshape(B * H, Qr, Kr), "inclusive", threshold).reshape(B, H, Qr, Kr)
    if scope == "head":
        return energy_mask(cells.reshape(B * H, 1, Qr * Kr), "cumulative", threshold).reshape(B, H, Qr, Kr)
    raise ValueError(f"scope must be 'row' or 'head', got {scope!r}")


def get_block_mask(inner_frame_mask, frame_mask, padding=4):
    """Block mask of the processed layout (:397-404): entry (a*Ri + d, c*Ci + e) = frame_mask[a, c]
    and inner_frame_mask[d, e] (the reference's einsum 'bhac,bhde->bhadce' reshaped), then
    `padding` dense text rows and columns (pad(value=1)). fp32 0/1 [B, H, F*Ri + padding,
    F*Ci + padding] (`sa_kron_block_mask`); B and H come from the masks (the reference fixes
    them at 2 and 30)."""
    _lib.require_gpu(inner_frame_mask, frame_mask)
    B, H, F, F2 = frame_mask.shape
    Ri, Ci = inner_frame_mask.shape[-2:]
    if F != F2 or tuple(inner_frame_mask.shape[:2]) != (B, H):
        raise ValueError(f"frame mask {tuple(frame_mask.shape)} / inner mask {tuple(inner_frame_mask.shape)}")
    fm = (frame_mask != 0).to(torch.uint8).contiguous()
    im = (inner_frame_mask != 0).to(torch.uint8).contiguous()
    out = torch.empty(B, H, F * Ri + padding, F * Ci + padding, dtype=torch.float32, device=fm.device)
    with torch.cuda.device(fm.device):
        rc = _lib.load().sa_kron_block_mask(fm.data_ptr(), im.data_ptr(), B * H, F, Ri, Ci, int(padding),
                                            out.data_ptr(), _lib.stream_of(fm))
    _lib.check(rc, "sa_kron_block_mask")
    return out
