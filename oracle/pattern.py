"""Frame-pattern attention and head routing on the CPU -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Restates, in float64 with the random sample positions passed in, the reference's
  * ParternAttentionColVersion_V2.get_weight_for_patch / forward (partern_attention.py:318-456),
  * constrained_mod_factor (:262-315),
  * judge_sparsity / judge_similarity / unified_judge (:468-521),
for a geometry of `frames` frames of height x width tokens after `text` text tokens, with
`ns` sampled positions per frame.

Pinned by tests/test_oracle_pattern.py against: the bf16 values of the text-key bias;
closed forms for uniform attention (every map entry ns/z, every modify factor 1); closed
forms for a directed construction in which every quantity of the forward and of both judges
reduces to scalars (frame f's queries boost the keys of frame f+1 and carry a per-frame slope
on a position channel; v is one direction per frame): the orientation of the maps, the
query frame chosen per key frame, both frame cases, the per-row modify factors, the final
mix, the rank-1 cosine of the similarity judge and the every-third-key share of the
sparsity judge; the reference's op chain for constrained_mod_factor on hand-made factors;
and invariants (map rows sum to 1 with the text share; identical frames give similarity 1).
"""
from __future__ import annotations

import torch


def _softmax(x):
    return torch.softmax(x, dim=-1)


def composition(ns, S):
    """The bias of the sampled text keys: log(ns / S) computed in fp32 and rounded to the
    inputs' dtype, bf16 (partern_attention.py:34-35, 343 and 497: composition.to(q.dtype))."""
    return float(torch.log(torch.tensor(ns / S, dtype=torch.float32)).to(torch.bfloat16))


def index_k(p, frames, S, text):
    """Sampled key/query tokens: the text tokens, then position p of every frame."""
    allf = (p.view(1, -1) + torch.arange(frames).view(-1, 1) * S + text).reshape(-1)
    return torch.cat([torch.arange(text), allf])


def weight_for_patch(q, k, p, frames, S, text):
    """(img2img_map [B,H,F,F], img2text_map [B,H,F,1]) of get_weight_for_patch (:321-358)."""
    ns = p.numel()
    idx = index_k(p, frames, S, text)
    qs, ks = q.double()[:, :, idx], k.double()[:, :, idx]
    out = qs @ ks.transpose(-1, -2) / 8
    out[..., :text] += composition(ns, S)
    out = _softmax(out)
    B, H = q.shape[:2]
    i2t = out[:, :, text:, :text].reshape(B, H, frames, ns * text).sum(-1, keepdim=True) / ns
    blocks = out[:, :, text:, text:].reshape(B, H, frames, ns, frames, ns)
    i2i = blocks.sum(dim=(3, 5)) / ns
    return i2i, i2t


def constrained_mod_factor(m, lo, hi):
    """:262-315 (m [B,H,L,1]); the adjustment decision is taken over every head at once."""
    osum = m.sum(dim=(-2, -1), keepdim=True)
    cmin = m.min(dim=-2, keepdim=True)[0]
    cmax = m.max(dim=-2, keepdim=True)[0]
    if not torch.logical_or(cmin < lo, cmax > hi).any():
        return m
    tmin = torch.where(cmin < lo, torch.full_like(cmin, lo), cmin)
    tmax = torch.where(cmax > hi, torch.full_like(cmax, hi), cmax)
    rng = cmax - cmin
    flat = rng < 1e-6
    rng = torch.where(flat, torch.ones_like(rng), rng)
    scaled = (m - cmin) / rng * (tmax - tmin) + tmin
    final = scaled * (osum / scaled.sum(dim=(-2, -1), keepdim=True))
    final = torch.where(flat, m, final)
    return torch.clamp(final, lo, hi)


def pattern_v2(q, k, v, p, frames, S, text, return_parts=False):
    """ParternAttentionColVersion_V2.forward (:377-453) in float64; returns [B,H,L,D]."""
    q, k, v = q.double(), k.double(), v.double()
    B, H, L, D = q.shape
    T, F = text, frames
    text_out = _softmax(q[:, :, :T] @ k.transpose(-1, -2) / 8) @ v
    ffa = _softmax(q[:, :, T:T + S] @ k.transpose(-1, -2) / 8)                    # [B,H,S,L]
    ida = _softmax(q[:, :, T:] @ k[:, :, :T].transpose(-1, -2) / 8)               # [B,H,F*S,T]
    i2i, i2t = weight_for_patch(q, k, p, F, S, T)
    a = ffa[..., :T].sum(-1, keepdim=True)
    mft = constrained_mod_factor(a / a.mean(dim=[-1, -2], keepdim=True), 0.01, 100)
    sel = torch.argmax(i2i, dim=-2)                                                # [B,H,F]
    vis, cases, mfs = [], [], []
    for i in range(F):
        ks = slice(T + i * S, T + (i + 1) * S)
        qsel = torch.stack([torch.stack([q[b, h, T + sel[b, h, i] * S: T + (sel[b, h, i] + 1) * S]
                                         for h in range(H)]) for b in range(B)])
        att = _softmax(qsel @ k[:, :, ks].transpose(-1, -2) / 8)
        blk = ffa[..., ks]
        tmp = blk.sum(-1, keepdim=True)
        mf = constrained_mod_factor(tmp / tmp.mean(dim=[-1, -2], keepdim=True), 0.05, 100)
        m0 = i2i[:, :, 0:1, i:i + 1]
        use = torch.where(m0 < 0.1, att * mf, blk / m0)
        vis.append(use @ v[:, :, ks])
        cases.append((m0 >= 0.1).view(B, H))
        mfs.append(mf)
    vmat = torch.stack(vis, dim=2)                                                 # [B,H,F,S,D]
    out_img = torch.einsum("bhfi,bhisd->bhfsd", i2i, vmat).reshape(B, H, F * S, D)
    fixed = ida.reshape(B, H, F, S, T) * mft.view(B, H, 1, S, 1)
    out_text = (i2t.view(B, H, F, 1, 1) * fixed).reshape(B, H, F * S, T) @ v[:, :, :T]
    out = torch.cat([text_out, out_img + out_text], dim=2)
    if return_parts:
        return out, dict(i2i=i2i, i2t=i2t, sel=sel, cases=torch.stack(cases, -1), mft=mft, mfs=mfs, ffa_blocks=None)
    return out


def judge_sparsity(q, k, idx_q, S, text, keep=0.2, thr=0.9):
    """(:468-476): sampled first-frame queries vs every third key; a head is sparse when the
    mean (over queries) share of its top `keep` keys exceeds `thr`. Returns (bool [B,H], share)."""
    qs = q.double()[:, :, idx_q + text]
    ks = k.double()[:, :, ::3]
    att = _softmax(qs @ ks.transpose(-1, -2) / 8)
    srt = att.sort(dim=-1, descending=True)[0].mean(dim=-2)
    share = srt[:, :, : int(ks.shape[2] * keep)].sum(-1)
    return share > thr, share


def judge_similarity(q, k, p, frames, S, text, thr=0.9):
    """(:477-514): cosine similarity of the sampled frame-pair attention patterns; a head is
    self-similar when the mean similarity of patterns sharing a key frame exceeds `thr`.
    Returns (bool [B,H], col_sim)."""
    ns = p.numel()
    idx = index_k(p, frames, S, text)
    qs, ks = q.double()[:, :, idx], k.double()[:, :, idx]
    out = qs @ ks.transpose(-1, -2) / 8
    out[..., :text] += composition(ns, S)
    out = _softmax(out)
    B, H = q.shape[:2]
    F = frames
    pat = out[:, :, text:, text:].reshape(B, H, F, ns, F, ns).permute(0, 1, 2, 4, 3, 5).reshape(B, H, F * F, ns * ns)
    pat = pat / pat.norm(dim=-1, keepdim=True)
    sim = pat @ pat.transpose(-1, -2)                                              # [(f1 f2), (f3 f4)]
    sim = sim.reshape(B, H, F, F, F, F).permute(0, 1, 3, 5, 2, 4).reshape(B, H, F, F, F * F).mean(-1)
    col = torch.diagonal(sim, dim1=-2, dim2=-1).mean(-1)
    return col > thr, col


def unified_judge(q, k, idx_sparse, p_sim1, p_sim2, frames, S, text):
    sp, _ = judge_sparsity(q, k, idx_sparse, S, text)
    s1, _ = judge_similarity(q, k, p_sim1, frames, S, text)
    s2, _ = judge_similarity(q, k, p_sim2, frames, S, text)
    return (~sp) & s1 & s2
