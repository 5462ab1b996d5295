"""Pins the pattern-attention oracle (oracle/pattern.py) with closed forms and hand cases."""
import math

import pytest
import torch

from oracle import pattern

F, H_, W_, T = 11, 4, 5, 8
S = H_ * W_
L = T + F * S


def _rand(shape, seed, scale=1.0):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * scale


@pytest.mark.parametrize("ns,S_,want", [(500, 4080, -2.09375), (6, 20, -1.203125), (3, 6, -0.69140625)])
def test_composition_is_bf16_rounded(ns, S_, want):
    # log(ns / S) rounded to bf16 (8 significant bits): log(500/4080) = -2.09924 -> -2.09375.
    assert pattern.composition(ns, S_) == want
    assert abs(want - math.log(ns / S_)) < 2 ** -7


def test_maps_closed_form_for_uniform_attention():
    # q = 0: every score is 0; the text keys carry exp(c) each, c = log(6/20) in bf16.
    ns = 6
    q = torch.zeros(1, 2, L, 64, dtype=torch.float64)
    k = _rand((1, 2, L, 64), 1)
    p = torch.randperm(S, generator=torch.Generator().manual_seed(2))[:ns]
    i2i, i2t = pattern.weight_for_patch(q, k, p, F, S, T)
    z = T * math.exp(-1.203125) + F * ns
    assert torch.allclose(i2i, torch.full_like(i2i, ns / z), atol=1e-12)
    assert torch.allclose(i2t, torch.full_like(i2t, T * math.exp(-1.203125) / z), atol=1e-12)
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
    z = T * math.exp(pattern.composition(ns, S)) + F * ns
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


# ---- directed construction ------------------------------------------------------------------
# F frames of S = 2 x 3 tokens after T = 3 text tokens, ns = 3 samples at positions P.
# Keys: text e_30; frame i, position s: e_i + t_s e_20. Queries: text 0; frame f, position s:
# 8a e_(f+1 mod F) + 8 g_f e_20 (+ 8 beta_s e_30 on frame 0). Values: text e_40; frame i,
# position s: (1 + t_s) e_(41+i). Scaled scores are then a [key frame = f+1] + g_f t_s on
# frame keys and beta_s [f = 0] on text keys, so every softmax reduces to scalar sums.
DF, DT = 5, 3
DS = 6
DL = DT + DF * DS
DA = 2.5
DG = [0.3, -0.2, 0.5, 0.1, -0.4]
DTS = [0.0, 0.4, 0.8, 1.2, 1.6, 2.0]
DBETA = [0.0, 0.3, -0.2, 0.5, 0.1, -0.3]
DP = [0, 2, 5]
DC = -0.69140625  # log(3/6) in bf16


def _directed():
    q = torch.zeros(1, 1, DL, 64, dtype=torch.float64)
    k = torch.zeros_like(q)
    v = torch.zeros_like(q)
    k[0, 0, :DT, 30] = 1
    v[0, 0, :DT, 40] = 1
    for f in range(DF):
        for s in range(DS):
            r = DT + f * DS + s
            q[0, 0, r, (f + 1) % DF] = 8 * DA
            q[0, 0, r, 20] = 8 * DG[f]
            if f == 0:
                q[0, 0, r, 30] = 8 * DBETA[s]
            k[0, 0, r, f] = 1
            k[0, 0, r, 20] = DTS[s]
            v[0, 0, r, 41 + f] = 1 + DTS[s]
    return q, k, v


def _sum_exp(g, pos):
    return sum(math.exp(g * DTS[s]) for s in pos)


def _mean_t(g):  # within-frame softmax mean of t over all positions
    return sum(DTS[s] * math.exp(g * DTS[s]) for s in range(DS)) / _sum_exp(g, range(DS))


def _directed_maps():
    i2i = [[0.0] * DF for _ in range(DF)]
    i2t = [0.0] * DF
    ns = len(DP)
    for f in range(DF):
        for s in DP:
            b = DBETA[s] if f == 0 else 0.0
            z = DT * math.exp(b + DC) + (math.exp(DA) + DF - 1) * _sum_exp(DG[f], DP)
            for i in range(DF):
                i2i[f][i] += math.exp(DA * (i == (f + 1) % DF)) * _sum_exp(DG[f], DP) / z / ns
            i2t[f] += DT * math.exp(b + DC) / z / ns
    return i2i, i2t


def test_directed_maps_closed_form():
    q, k, _ = _directed()
    i2i, i2t = pattern.weight_for_patch(q, k, torch.tensor(DP), DF, DS, DT)
    w_i2i, w_i2t = _directed_maps()
    assert torch.allclose(i2i[0, 0], torch.tensor(w_i2i, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(i2t[0, 0, :, 0], torch.tensor(w_i2t, dtype=torch.float64), atol=1e-12)
    assert i2i[0, 0, 0, 1] > 0.5 and i2i[0, 0, 1, 0] < 0.1  # not symmetric: orientation is pinned


def test_directed_forward_closed_form():
    q, k, v = _directed()
    out = pattern.pattern_v2(q, k, v, torch.tensor(DP), DF, DS, DT)[0, 0]
    i2i, i2t = _directed_maps()
    # first-frame rows over every key (no bias): text mass T e^beta_r / Z_r, frame i mass
    # e^(a [i = 1]) sum_s e^(g_0 t_s) / Z_r
    e0 = _sum_exp(DG[0], range(DS))
    zr = [DT * math.exp(DBETA[r]) + (math.exp(DA) + DF - 1) * e0 for r in range(DS)]
    mu = [(1 / z) / (sum(1 / y for y in zr) / DS) for z in zr]           # every frame's factor
    tm = [math.exp(DBETA[r]) / zr[r] for r in range(DS)]
    mft = [x / (sum(tm) / DS) for x in tm]
    assert min(mu) > 0.05 and max(mu) < 100 and min(mft) > 0.01 and max(mft) < 100  # no adjustment
    assert i2i[0][1] >= 0.1 and all(i2i[0][i] < 0.1 for i in range(DF) if i != 1)
    want = torch.zeros(DL, 64, dtype=torch.float64)
    want[:DT, 40] = DT / DL                                              # q = 0: mean of every v row
    for i in range(DF):
        want[:DT, 41 + i] = sum(1 + t for t in DTS) / DL
    for f1 in range(DF):
        for r in range(DS):
            row = DT + f1 * DS + r
            for i in range(DF):
                if i2i[0][i] >= 0.1:   # first-frame masses of frame i over img2img_map[0][i]
                    o = math.exp(DA * (i == 1)) * e0 / zr[r] / i2i[0][i] * (1 + _mean_t(DG[0]))
                else:                  # queries of frame argmax_f img2img_map[f][i] = i - 1
                    o = mu[r] * (1 + _mean_t(DG[(i - 1) % DF]))
                want[row, 41 + i] = i2i[f1][i] * o
            want[row, 40] = i2t[f1] * mft[r]
    assert torch.allclose(out, want, atol=1e-12), (out - want).abs().max()


def test_directed_similarity_closed_form():
    # Patterns are rank 1: P[(f1,s1)][(f2,s2)] = e^(a [f2 = f1+1]) e^(g_f1 t_s2) / Z(f1, s1), so
    # cos(X_f1f2, X_f3f2) = cos(1/Z(f1,.), 1/Z(f3,.)) * cos(e^(g_f1 t), e^(g_f3 t)) over the
    # samples, for every key frame f2; col_sim is its mean over (f1, f3).
    q, k, _ = _directed()
    _, col = pattern.judge_similarity(q, k, torch.tensor(DP), DF, DS, DT)

    def cos(x, y):
        return sum(a * b for a, b in zip(x, y)) / math.sqrt(sum(a * a for a in x) * sum(b * b for b in y))
    u, w = [], []
    for f in range(DF):
        z = [DT * math.exp((DBETA[s] if f == 0 else 0.0) + DC) + (math.exp(DA) + DF - 1) * _sum_exp(DG[f], DP)
             for s in DP]
        u.append([1 / x for x in z])
        w.append([math.exp(DG[f] * DTS[s]) for s in DP])
    want = sum(cos(u[a], u[b]) * cos(w[a], w[b]) for a in range(DF) for b in range(DF)) / DF ** 2
    assert abs(col.item() - want) < 1e-12
    assert want < 0.999


def test_directed_sparsity_closed_form():
    # First-frame queries against keys 0, 3, 6, ...: text keys score beta_s, frame-i keys
    # a [i = 1] + g_0 t_pos; share = mean over the sampled rows of the top int(0.2 n) mass.
    q, k, _ = _directed()
    idx_q = torch.tensor([1, 4, 5])
    _, share = pattern.judge_sparsity(q, k, idx_q, DS, DT)
    keys = range(0, DL, 3)
    n = len(keys)
    total = 0.0
    for s in idx_q.tolist():
        logits = []
        for j in keys:
            if j < DT:
                logits.append(DBETA[s])
            else:
                fi, pos = divmod(j - DT, DS)
                logits.append(DA * (fi == 1) + DG[0] * DTS[pos])
        e = sorted((math.exp(x) for x in logits), reverse=True)
        total += sum(e[: int(n * 0.2)]) / sum(e)
    assert abs(share.item() - total / 3) < 1e-12
