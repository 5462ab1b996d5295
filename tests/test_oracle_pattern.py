"""Pins the pattern-attention oracle (oracle/pattern.py) with closed forms and hand cases."""
import math

import torch

from oracle import pattern

F, H_, W_, T = 11, 4, 5, 8
S = H_ * W_
L = T + F * S


def _rand(shape, seed, scale=1.0):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * scale


def test_maps_closed_form_for_uniform_attention():
    # q = 0: every score is 0; the text keys carry exp(log(ns/S)) = ns/S each.
    ns = 6
    q = torch.zeros(1, 2, L, 64, dtype=torch.float64)
    k = _rand((1, 2, L, 64), 1)
    p = torch.randperm(S, generator=torch.Generator().manual_seed(2))[:ns]
    i2i, i2t = pattern.weight_for_patch(q, k, p, F, S, T)
    z = T * ns / S + F * ns
    assert torch.allclose(i2i, torch.full_like(i2i, ns / z), atol=1e-12)
    assert torch.allclose(i2t, torch.full_like(i2t, T * ns / S / z), atol=1e-12)
    # map rows: the text share plus the frame shares sum to one
    assert torch.allclose(i2i.sum(-1, keepdim=True) + i2t, torch.ones_like(i2t), atol=1e-12)


def test_maps_rows_sum_to_one():
    ns = 7
    q, k = _rand((2, 3, L, 64), 3, 0.5), _rand((2, 3, L, 64), 4, 0.5)
    p = torch.randperm(S, generator=torch.Generator().manual_seed(5))[:ns]
    i2i, i2t = pattern.weight_for_patch(q, k, p, F, S, T)
    assert torch.allclose(i2i.sum(-1, keepdim=True) + i2t, torch.ones_like(i2t), atol=1e-12)


def test_constrained_mod_factor_cases():
    # (a) every head within [lo, hi]: unchanged (no clamp either)
    m = torch.tensor([0.5, 1.0, 1.5, 1.0], dtype=torch.float64).view(1, 1, 4, 1).repeat(1, 2, 1, 1)
    assert torch.equal(pattern.constrained_mod_factor(m, 0.1, 10.0), m)
    # (b) one head above hi: both heads are remapped affinely onto [max(min, lo), min(max, hi)]
    #     and rescaled to keep their sums; then clamped.
    m2 = m.clone()
    m2[0, 1] = torch.tensor([0.5, 4.0, 20.0, 3.5], dtype=torch.float64).view(4, 1)
    out = pattern.constrained_mod_factor(m2, 0.1, 10.0)
    x = m2[0, 1, :, 0]
    scaled = (x - 0.5) / 19.5 * (10.0 - 0.5) + 0.5
    want = torch.clamp(scaled * (x.sum() / scaled.sum()), 0.1, 10.0)
    assert torch.allclose(out[0, 1, :, 0], want, atol=1e-12)
    assert torch.allclose(out[0, 0], m2[0, 0], atol=1e-12)  # in-range head: identity map
    # (c) a flat head keeps its values (then clamped) when another head triggers adjustment
    m3 = torch.cat([torch.full((1, 1, 4, 1), 20.0, dtype=torch.float64), m2[:, 1:]], dim=1)
    out3 = pattern.constrained_mod_factor(m3, 0.1, 10.0)
    assert torch.all(out3[0, 0] == 10.0)


def test_uniform_attention_forward_closed_form():
    # q = 0 and every v row equal to c: every attention average is c, so the output is
    # text rows: c; video rows: (sum_i img2img[f][i] * s_i + img2text[f] * mft) * c with
    # s_i = 1 (modify factors of uniform masses are 1, or masses / map with map = mass share).
    ns = 5
    B, H = 1, 2
    q = torch.zeros(B, H, L, 64, dtype=torch.float64)
    k = _rand((B, H, L, 64), 6)
    c = _rand((64,), 7)
    v = c.expand(B, H, L, 64).clone()
    p = torch.randperm(S, generator=torch.Generator().manual_seed(8))[:ns]
    out, parts = pattern.pattern_v2(q, k, v, p, F, S, T, return_parts=True)
    assert torch.allclose(out[:, :, :T], c.expand(B, H, T, 64), atol=1e-12)
    i2i, i2t = parts["i2i"], parts["i2t"]
    z = T * ns / S + F * ns
    # masses of uniform first-frame rows: frame share S / L; map[0][i] = ns / z
    s_case_b = (S / L) / (ns / z)
    s = torch.where(parts["cases"], torch.full_like(i2t[..., 0], s_case_b), torch.ones_like(i2t[..., 0]))
    coef = (i2i * s.unsqueeze(-2)).sum(-1) + i2t[..., 0]                      # [B,H,F]
    want = coef.view(B, H, F, 1, 1) * c.view(1, 1, 1, 1, 64)
    assert torch.allclose(out[:, :, T:].view(B, H, F, S, 64), want.expand(B, H, F, S, 64), atol=1e-10)


def test_similarity_of_identical_frames_is_one_and_uniform_is_not_sparse():
    ns = 6
    B, H = 1, 2
    qf, kf = _rand((B, H, S, 64), 9, 0.5), _rand((B, H, S, 64), 10, 0.5)
    q = torch.cat([_rand((B, H, T, 64), 11, 0.5)] + [qf] * F, dim=2)
    k = torch.cat([_rand((B, H, T, 64), 12, 0.5)] + [kf] * F, dim=2)
    p = torch.randperm(S, generator=torch.Generator().manual_seed(13))[:ns]
    _, col = pattern.judge_similarity(q, k, p, F, S, T)
    assert torch.allclose(col, torch.ones_like(col), atol=1e-12)
    sp, share = pattern.judge_sparsity(torch.zeros_like(q), k, p, S, T)
    n = k[:, :, ::3].shape[2]
    assert not sp.any() and torch.allclose(share, torch.full_like(share, int(n * 0.2) / n), atol=1e-12)
