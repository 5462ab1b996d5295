"""Pins the estimator oracles: sampled block scores (oracle/estimator.py) and the energy /
adaptive top-k selection (oracle_energy_list in oracle/sa_oracle.c)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import estimator, native


def _rand(shape, seed):
    return torch.rand(shape, generator=torch.Generator().manual_seed(seed))


def _bf16(shape, seed, scale=1.0):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * scale).to(torch.bfloat16)


# ---- sampling and sampled block scores ------------------------------------------------------

@pytest.mark.parametrize("L,S", [(128, 8), (300, 8), (257, 16)])
def test_sampled_tokens_match_pad_topk_gather(L, S):
    # The reference's formulation: replicate-pad to a multiple of 64, topk(sorted) of the
    # draws per block, gather (utils/mask_related.py:2-37).
    B, H, D = 1, 2, 64
    x = _bf16((B, H, L, D), 1)
    nb = math.ceil(L / 64)
    rand = _rand((B, H, nb, 64), 2)
    Lp = nb * 64
    xp = F.pad(x.float(), (0, 0, 0, Lp - L), mode="replicate") if Lp != L else x.float()
    idx = torch.topk(rand, S, dim=3).indices
    want = torch.gather(xp.view(B, H, nb, 64, D), 3, idx[..., None].expand(-1, -1, -1, -1, D)).reshape(B, H, nb * S, D)
    tok = estimator.sample_tokens(rand, L, S)
    got = torch.stack([x[0, h].float()[tok[0, h]] for h in range(H)])[None]
    assert torch.equal(got, want)


@pytest.mark.parametrize("S", [8, 16])
def test_pooled_scores_match_conv2d_sum(S):
    # The reference pools with conv2d(ones(S, S), stride=S) (:71-77).
    B, H, L = 1, 2, 200
    q, k = _bf16((B, H, L, 64), 3), _bf16((B, H, L, 64), 4)
    nb = math.ceil(L / 64)
    rq, rk = _rand((B, H, nb, 64), 5), _rand((B, H, nb, 64), 6)
    got = estimator.sampled_block_scores(q, k, rq, rk, S)
    tq, tk = estimator.sample_tokens(rq, L, S), estimator.sample_tokens(rk, L, S)
    for h in range(H):
        a = torch.softmax(q[0, h].double()[tq[0, h]] @ k[0, h].double()[tk[0, h]].T / 8, dim=-1)
        pooled = F.conv2d(a[None, None], torch.ones(1, 1, S, S, dtype=torch.float64), stride=S)[0, 0]
        assert torch.allclose(got[0, h], pooled, rtol=1e-12, atol=1e-14)


def test_pooled_rows_sum_to_num_keep():
    B, H, L, S = 2, 2, 500, 8
    q, k = _bf16((B, H, L, 64), 7, 3.0), _bf16((B, H, L, 64), 8, 3.0)
    nb = math.ceil(L / 64)
    got = estimator.sampled_block_scores(q, k, _rand((B, H, nb, 64), 9), _rand((B, H, nb, 64), 10), S)
    assert torch.allclose(got.sum(-1), torch.full((B, H, nb), float(S), dtype=torch.float64), atol=1e-10)


def test_pooled_uniform_when_q_is_zero():
    B, H, L, S = 1, 1, 320, 8
    q = torch.zeros(B, H, L, 64, dtype=torch.bfloat16)
    k = _bf16((B, H, L, 64), 11)
    nb = 5
    got = estimator.sampled_block_scores(q, k, _rand((B, H, nb, 64), 12), _rand((B, H, nb, 64), 13), S)
    assert torch.allclose(got, torch.full_like(got, S / nb), atol=1e-12)


# ---- energy / adaptive top-k selection ------------------------------------------------------

def _reference_ops(scores, mode, thr, min_keep, max_keep, init_k, n_text=4):
    """transfer_attn_to_mask (SparseGen_Plus.py:12-84) with torch's CPU ops in fp32: stable
    descending sort, cumsum, argmax of the threshold mask, where, clamp, scatter."""
    BH, nqb, n = scores.shape
    s = scores.float()
    srt, ind = torch.sort(s, dim=-1, descending=True, stable=True)
    cum = torch.cumsum(srt, dim=-1)
    total = cum[..., -1:]
    if mode == 0:
        hit = cum >= thr * total
        kk = torch.argmax(hit.int(), dim=-1)
        uns = (cum[..., -1:] < thr * total).squeeze(-1)
        kk = torch.where(uns, torch.full_like(kk, n), kk)
        kk = torch.clamp(torch.clamp(kk, max=n), min=min_keep, max=max_keep)
    elif mode == 2:
        # generate_attention_mask_frame_scope / get_inner_frame_mask "row" (mask_related.py
        # :224-232, 366-376): cum >= threshold, last forced, argmax, ranks <= k.
        over = cum >= thr * total
        over[..., -1] = True
        kk = torch.argmax(over.int(), dim=-1) + 1
        kk = torch.clamp(kk, min=min_keep, max=max_keep)
    elif mode == 3:
        # get_inner_frame_mask "head" (mask_related.py:378-391): cum <= threshold, last forced.
        sel = cum <= thr * total
        sel[..., -1] = True
        mask = torch.zeros_like(sel).scatter_(-1, ind, sel)
        mask[:, :n_text] = True
        mask[:, :, :n_text] = True
        return mask
    else:
        cur_k = torch.full((BH, nqb), init_k, dtype=torch.int64)
        cur = cum.gather(-1, (cur_k - 1)[..., None]).squeeze(-1)
        upd = (~(cur >= 0.6 * total.squeeze(-1))) & (cur_k < n)
        upd1 = (~(cur >= 0.9 * total.squeeze(-1))) & (cur_k < n)
        cur_k[upd] = torch.clamp(cur_k[upd] * 3, max=n)
        cur_k[upd1] = torch.clamp(cur_k[upd1] // 3 * 2, max=n)
        kk = cur_k
    keep = torch.arange(n).view(1, 1, n) < kk[..., None]
    mask = torch.zeros_like(keep).scatter_(-1, ind, keep)
    mask[:, :n_text] = True
    mask[:, :, :n_text] = True
    return mask


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("n,seed", [(5, 0), (64, 1), (65, 2), (278, 3), (700, 4)])
def test_energy_oracle_matches_reference_ops(mode, n, seed):
    BH, nqb = 3, 7
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(BH, nqb, n, generator=g) ** 4  # skewed, as attention energies are
    scores[0, 1] = 1.0  # a row of ties
    scores[1, 2, : n // 2] = 0.25  # half ties
    thr = [0.9, 0.95, 0.98][seed % 3]
    min_keep, max_keep = max(1, int(n * 0.1)), max(1, int(n * 0.8))
    init_k = max(1, int(n * 0.2))
    _, _, got = native.energy_list(scores, mode, thr, min_keep, max_keep, init_k, 4)
    want = _reference_ops(scores, mode, thr, min_keep, max_keep, init_k)
    assert torch.equal(got.bool().reshape(BH, nqb, n), want)


def test_energy_hand_cases():
    # Equal scores: cum[j] = j + 1, total = 10, target 9.5 -> first j with j + 1 >= 9.5 is 9,
    # so 9 columns are kept (the crossing column is not); text blocks off.
    s = torch.ones(1, 1, 10)
    _, cnt, m = native.energy_list(s, 0, 0.95, 1, 10, 1, 0)
    assert cnt.item() == 9 and m.sum().item() == 9 and m[0, 9] == 0  # ties keep low columns
    # A dominant column crossing the threshold alone: k = 0, raised to min_keep = 2.
    s = torch.tensor([[[0.1, 5.0, 0.2, 0.05]]])
    _, cnt, m = native.energy_list(s, 0, 0.5, 2, 4, 1, 0)
    assert m[0].tolist() == [0, 1, 1, 0]
    # max_keep caps: threshold 1.0 needs all 4 -> clamp to 3, dropping the smallest.
    _, cnt, m = native.energy_list(s, 0, 1.0, 1, 3, 1, 0)
    assert m[0].tolist() == [1, 1, 1, 0]
    # topk: init 1 holds 5/5.35 >= 0.9 of the energy -> stays 1.
    _, cnt, m = native.energy_list(s, 1, 0.0, 1, 4, 1, 0)
    assert m[0].tolist() == [0, 1, 0, 0]
    # topk: flat row of 9, init 2 holds 2/9 < 0.6 -> 6, then < 0.9 -> 6 // 3 * 2 = 4.
    _, cnt, m = native.energy_list(torch.ones(1, 1, 9), 1, 0.0, 1, 9, 2, 0)
    assert cnt.item() == 4 and m[0].tolist() == [1, 1, 1, 1, 0, 0, 0, 0, 0]
    # text rows and columns: scores 1..6, cum 6, 11, ... reaches 0.5 * 21 at j = 1 -> column 5.
    s = torch.arange(1.0, 7.0).expand(1, 3, 6).contiguous()
    _, cnt, m = native.energy_list(s, 0, 0.5, 1, 6, 1, 2)
    m = m.reshape(3, 6)
    assert m[0].all() and m[1].all() and m[2].tolist() == [1, 1, 0, 0, 0, 1]


def test_energy_inclusive_and_cumulative_hand_cases():
    # Equal scores, cum[j] = j + 1, total 10. Mode 2 keeps through the crossing: 0.95 -> j = 9
    # (all 10); 0.5 -> j = 4 (5 kept). Mode 3 keeps cum <= target plus the last rank:
    # 0.5 -> ranks 0..4 and rank 9 (ties: ranks follow the column order).
    s = torch.ones(1, 1, 10)
    assert native.energy_list(s, 2, 0.95, 0, 10, 1, 0)[1].item() == 10
    _, cnt, m = native.energy_list(s, 2, 0.5, 0, 10, 1, 0)
    assert cnt.item() == 5 and m[0].tolist() == [1] * 5 + [0] * 5
    _, cnt, m = native.energy_list(s, 3, 0.5, 0, 10, 1, 0)
    assert m[0].tolist() == [1] * 5 + [0] * 4 + [1]
    # Threshold 1 (the reference's get_inner_frame_mask default): mode 2 keeps every column
    # up to the last one that still raises the sum; a zero tail is dropped.
    s = torch.tensor([[[0.0, 3.0, 0.5, 0.0, 1.5]]])
    _, cnt, m = native.energy_list(s, 2, 1.0, 0, 5, 1, 0)
    assert m[0].tolist() == [0, 1, 1, 0, 1]
    # A dominant column alone crosses 0.5: mode 2 keeps it; mode 3 keeps nothing below the
    # target but the forced last rank (the smallest score).
    s = torch.tensor([[[0.1, 5.0, 0.2, 0.05]]])
    assert native.energy_list(s, 2, 0.5, 0, 4, 1, 0)[2][0].tolist() == [0, 1, 0, 0]
    assert native.energy_list(s, 3, 0.5, 0, 4, 1, 0)[2][0].tolist() == [0, 0, 0, 1]


def test_energy_prefix_property():
    # Before clamping, the kept prefix is the longest one whose energy stays below the target.
    g = torch.Generator().manual_seed(5)
    s = torch.rand(1, 40, 200, generator=g) ** 3
    idx, cnt, m = native.energy_list(s, 0, 0.9, 1, 200, 1, 0)
    for r in range(40):
        srt = torch.sort(s[0, r], descending=True).values.double()
        k = cnt[r].item()
        total = srt.sum().item()
        assert srt[:k].sum().item() < 0.9 * total * (1 + 1e-6)
        assert srt[: k + 1].sum().item() >= 0.9 * total * (1 - 1e-6)
