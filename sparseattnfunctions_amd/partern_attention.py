"""Frame-pattern attention and head routing of special_attentions/partern_attention.py, on MI355X.

  * `ParternAttentionColVersion_V2` (:318-456): text rows attend everything; every video
    frame's output is a mix, weighted by a sampled frame-to-frame map, of per-key-frame
    attention outputs computed once from a representative query frame, plus a video-to-text
    term scaled by first-frame text masses.
  * `constrained_mod_factor` (:262-315), `get_indexs` (:17-31).
  * `judge_sparsity`, `judge_similarity`, `unified_judge` (:463-521): whether a head suits
    the pattern approximation.

The geometry defaults to the reference's 1.5-5B constants (11 frames of 48 x 85 tokens after
224 text tokens, 500 sampled positions per frame); `PatternGeometry` makes it a parameter.
Sampled positions are drawn with `torch.randperm` on the CPU generator in the reference's
order. Every tensor computation runs in HIP kernels of libsa_hip.so: the attention-shaped
parts in the block-sparse attention kernel (a 0/1 segment-indicator V turns its output into
per-segment probability masses), the rest in the kernels of csrc/pattern.hip and
csrc/judge.hip.

Differences from the reference, by design: probabilities and masses are fp32 inside the
kernels and rounded to bf16 only where the attention kernel writes its output (the reference
keeps bf16 scores and softmax throughout); `ParternAttentionRowVersion` and the first
`ParternAttentionColVersion` are not provided (`CombinedAttn` uses only the V2 class).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._gather import gather_tokens
from ._kv import KVList
from .block_mask_attn import dense_kv_list
from .utils.block_sparse_attn_kernel import _prep_qkv, block_sparse_attention


@dataclass(frozen=True)
class PatternGeometry:
    frames: int = 11
    height: int = 48
    width: int = 85
    text_length: int = 224
    sample_num: int = 500

    @property
    def S(self) -> int:
        return self.height * self.width

    @property
    def L(self) -> int:
        return self.text_length + self.frames * self.S


DEFAULT = PatternGeometry()
f, width, height, text_length, sample_num, dim = 11, 85, 48, 224, 500, 64
scale_factor = 1 / 8
# The reference's module tensors (partern_attention.py:34-35).
sample_rate = torch.tensor(sample_num / (width * height))
composition = torch.log(sample_rate).view(1, 1, 1, 1)

_CACHE = {}
OVERLAP_TEXT = True  # text and video-to-text rows on a second stream (see forward)
OVERLAP_JUDGE = True  # sparsity judge on a second stream (see unified_judge)


def _side_stream(device):
    return _lib.side_stream(device)


def _cached(key, make):
    t = _CACHE.get(key)
    if t is None:
        t = make()
        _CACHE[key] = t
    return t


def _dense(B, H, nq, nk, device) -> KVList:
    return _cached(("dense", B, H, nq, nk, str(device)),
                   lambda: dense_kv_list(B, H, math.ceil(nq / 64), math.ceil(nk / 64), device))


def _indicator(seg_of_key: torch.Tensor, device):
    """bf16 [Lk, 64]: 1 at column seg_of_key[j] of row j (a 0/1 segment-indicator V)."""
    ind = torch.zeros(seg_of_key.numel(), 64, dtype=torch.bfloat16)
    ind[torch.arange(seg_of_key.numel()), seg_of_key] = 1
    return ind.to(device)


def _mass_cols(g: PatternGeometry):
    """Output columns of the segment-mass attention: 32 (only v's first 32 columns enter P.V)
    when the 1 + frames segments fit, else all 64."""
    return 32 if 1 + g.frames <= 32 else None


def _frame_indicator(g: PatternGeometry, device):
    def make():
        j = torch.arange(g.L)
        return _indicator(torch.where(j < g.text_length, 0, 1 + (j - g.text_length) // g.S), device)
    return _cached(("ind", g, str(device)), make)


def _sample_indicator(g: PatternGeometry, device):
    def make():
        j = torch.arange(g.text_length + g.frames * g.sample_num)
        return _indicator(torch.where(j < g.text_length, 0, 1 + (j - g.text_length) // g.sample_num), device)
    return _cached(("sind", g, str(device)), make)


def composition_bias(geometry: PatternGeometry = DEFAULT) -> float:
    """Bias of the sampled text keys: log(sample_num / S) in fp32, rounded to bf16 as the
    reference adds it (partern_attention.py:34-35, 343, 497: composition.to(q.dtype))."""
    g = geometry
    return float(torch.log(torch.tensor(g.sample_num / g.S, dtype=torch.float32)).to(torch.bfloat16))


def get_indexs(geometry: PatternGeometry = DEFAULT):
    """(all_idxs, index_k): `sample_num` random positions of the first frame repeated in every
    frame (torch.randperm on the CPU generator), and the same with the text tokens first."""
    g = geometry
    first = torch.randperm(g.S)[: g.sample_num] + g.text_length
    all_idxs = (first.view(1, -1) + (torch.arange(g.frames) * g.S).view(-1, 1)).view(-1)
    return all_idxs, torch.cat([torch.arange(g.text_length), all_idxs])


def _bcast(t, B, H):
    return t.expand(B, H, *t.shape)


class ParternAttentionColVersion_V2:
    def __init__(self, geometry: PatternGeometry = DEFAULT):
        self.geometry = geometry
        self.last_plan = None  # maps and choices of the last call (inspection and tests)

    def _check(self, q, k, v):
        _lib.require_gpu(q, k, v)
        g = self.geometry
        if q.shape[2] != g.L or k.shape != q.shape or v.shape != q.shape or q.shape[3] != 64:
            raise ValueError(f"expected q, k, v of shape [B, H, {g.L}, 64], got {tuple(q.shape)}")
        return _prep_qkv(q), _prep_qkv(k), _prep_qkv(v)

    def sampled_masses(self, q, k, index_k, sm_scale: float = scale_factor):
        """Segment masses of the sampled attention (get_weight_for_patch, :321-358): for every
        sampled video row, the softmax mass (with log(ns/S) added to text keys) on the text
        keys (column 0) and on each frame's samples (column 1 + f). bf16 [B, H, F*ns, 32] (64 columns
        for more than 31 frames)."""
        g = self.geometry
        B, H = q.shape[:2]
        idx = index_k.to(device=q.device, dtype=torch.int32)
        qs, ks = gather_tokens(q, idx), gather_tokens(k, idx)
        nk = idx.numel()
        bias = _cached(("bias", g, str(q.device)), lambda: torch.where(
            torch.arange(nk, device=q.device) < g.text_length, composition_bias(g), 0.0).float())
        return block_sparse_attention(qs[:, :, g.text_length:], ks, _bcast(_sample_indicator(g, q.device), B, H),
                                      _dense(B, H, g.frames * g.sample_num, nk, q.device), sm_scale,
                                      key_bias=_bcast(bias, B, H), v_cols=_mass_cols(g))

    def forward(self, q, k, v, index_k=None):
        q, k, v = self._check(q, k, v)
        g = self.geometry
        T, S, F, ns = g.text_length, g.S, g.frames, g.sample_num
        B, H, L, D = q.shape
        dev = q.device
        if index_k is None:
            _, index_k = get_indexs(g)
        out = torch.empty_like(q)
        # Video rows over the text keys (img2text_detailed_attention @ v_text; many short,
        # latency-bound blocks) and the text rows, launched on a second stream (default
        # priority) so that they run alongside the compute-bound launches below; joined before
        # the final mix.
        main = torch.cuda.current_stream(dev)
        # Every cached list the side stream reads is built (on a first call: by kernels on the
        # main stream) before the side stream waits for the main one.
        text_kv = _dense(B, H, F * S, T, dev)
        text_rows_kv = _dense(B, H, T, L, dev)
        side = _side_stream(dev) if OVERLAP_TEXT else main
        side.wait_stream(main)
        with torch.cuda.stream(side):
            o_text = block_sparse_attention(q[:, :, T:], k[:, :, :T], v[:, :, :T], text_kv, scale_factor)
            # Text rows over every key (the reference's SDPA, :442).
            block_sparse_attention(q[:, :, :T], k, v, text_rows_kv, scale_factor, out=out[:, :, :T])
        # First-frame rows over every key: per-segment masses (text, frame i).
        ff_mass = block_sparse_attention(q[:, :, T:T + S], k, _bcast(_frame_indicator(g, dev), B, H),
                                         _dense(B, H, S, L, dev), scale_factor, v_cols=_mass_cols(g))
        map_mass = self.sampled_masses(q, k, index_k)
        BH = B * H
        f32 = dict(dtype=torch.float32, device=dev)
        i2i, i2t = self._maps(map_mass)
        stats = torch.empty(BH, 1 + F, 3, **f32)
        fac = torch.empty(BH, 1 + F, 4, **f32)
        case = torch.empty(BH, F, dtype=torch.int32, device=dev)
        inv0 = torch.empty(BH, F, **f32)
        q_idx = torch.empty(BH, F * S, dtype=torch.int32, device=dev)
        lib = _lib.load()
        stream = _lib.stream_of(q)
        with torch.cuda.device(dev):
            _lib.check(lib.sa_pattern_plan(
                ff_mass.data_ptr(), _lib.i64(*ff_mass.stride()[:3]), i2i.data_ptr(), B, H, F, S, T,
                0.01, 100.0, 0.05, 100.0, 0.1, stats.data_ptr(), fac.data_ptr(), case.data_ptr(), inv0.data_ptr(),
                q_idx.data_ptr(), stream), "sa_pattern_plan")
            q_sel = torch.empty(B, H, F * S, D, dtype=q.dtype, device=dev)
            _lib.check(lib.sa_gather_tokens_heads(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), B, H, L, D, q_idx.data_ptr(), F * S, q_sel.data_ptr(),
                _lib.i64(*q_sel.stride()[:3]), stream), "sa_gather_tokens_heads")
        o_frames = torch.empty(B, H, F * S, D, dtype=q.dtype, device=dev)
        # Frame i's selected rows over frame i's keys, for every frame in one launch: (b, h) as
        # the batch index and the frame as the head index of [B*H, F, S, D] views. Inputs whose
        # batch and head axes do not merge into one stride (a slice of a tensor's heads) take
        # one launch per frame.
        if all(x.stride(0) == H * x.stride(1) or B == 1 for x in (k, v)):
            block_sparse_attention(q_sel.view(B * H, F, S, D), k[:, :, T:T + F * S].reshape(B * H, F, S, D),
                                   v[:, :, T:T + F * S].reshape(B * H, F, S, D), _dense(B * H, F, S, S, dev),
                                   scale_factor, out=o_frames.view(B * H, F, S, D))
        else:
            frame_kv = _dense(B, H, S, S, dev)
            for i in range(F):
                rows = slice(i * S, (i + 1) * S)
                keys = slice(T + i * S, T + (i + 1) * S)
                block_sparse_attention(q_sel[:, :, rows], k[:, :, keys], v[:, :, keys], frame_kv, scale_factor,
                                       out=o_frames[:, :, rows])
        main.wait_stream(side)
        o_text.record_stream(main)
        with torch.cuda.device(dev):
            _lib.check(lib.sa_pattern_combine(
                o_frames.data_ptr(), _lib.i64(*o_frames.stride()[:3]), o_text.data_ptr(),
                _lib.i64(*o_text.stride()[:3]), ff_mass.data_ptr(), _lib.i64(*ff_mass.stride()[:3]),
                i2t.data_ptr(), i2i.data_ptr(), fac.data_ptr(), case.data_ptr(), inv0.data_ptr(), B, H, F, S, T,
                0.01, 100.0, 0.05, 100.0, out.data_ptr(), _lib.i64(*out.stride()[:3]), stream),
                "sa_pattern_combine")
        self.last_plan = dict(img2text=i2t, img2img=i2i, frame_case=case.view(B, H, F), fac=fac.view(B, H, 1 + F, 4))
        return out

    def _maps(self, mass):
        g = self.geometry
        B, H = mass.shape[:2]
        i2t = torch.empty(B, H, g.frames, 1, dtype=torch.float32, device=mass.device)
        i2i = torch.empty(B, H, g.frames, g.frames, dtype=torch.float32, device=mass.device)
        with torch.cuda.device(mass.device):
            _lib.check(_lib.load().sa_pattern_maps(mass.data_ptr(), _lib.i64(*mass.stride()[:3]), B, H, g.frames,
                                                   g.sample_num, i2t.data_ptr(), i2i.data_ptr(),
                                                   _lib.stream_of(mass)), "sa_pattern_maps")
        return i2i, i2t

    def get_weight_for_patch(self, q, k, index_k=None, sm_scale: float = scale_factor):
        """(img2img_map [B,H,F,F], img2text_map [B,H,F,1]) fp32."""
        q, k, _ = self._check(q, k, k)
        if index_k is None:
            _, index_k = get_indexs(self.geometry)
        return self._maps(self.sampled_masses(q, k, index_k, sm_scale))

    def __call__(self, *args, **kwds):
        return self.forward(*args, **kwds)


def constrained_mod_factor(modify_factor, min_threshold=0.01, max_threshold=50.0):
    """partern_attention.py:262-315 on the GPU (`sa_constrained_mod_factor`): modify_factor
    [B, H, L, 1] fp32 (other float dtypes are converted); unchanged when every head lies within
    [min_threshold, max_threshold], else each head is mapped affinely onto the clipped range,
    rescaled to its original sum and clamped. Computed in fp32 and returned in the input's
    dtype and shape. Where the reference returns `modify_factor` itself (no head out of range)
    this returns a new tensor of equal values: the decision stays on the GPU, with no host
    synchronisation."""
    _lib.require_gpu(modify_factor)
    if modify_factor.dim() != 4 or modify_factor.shape[-1] != 1:
        raise ValueError(f"modify_factor must be [B, H, L, 1], got {tuple(modify_factor.shape)}")
    B, H, L, _ = modify_factor.shape
    x = modify_factor.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    stats = torch.empty(B * H, 3, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().sa_constrained_mod_factor(x.data_ptr(), B * H, L, float(min_threshold),
                                                         float(max_threshold), stats.data_ptr(), out.data_ptr(),
                                                         _lib.stream_of(x)), "sa_constrained_mod_factor")
    return out if modify_factor.dtype == torch.float32 else out.to(modify_factor.dtype)


def get_softmax(q, k):
    """softmax(q k^T * scale_factor) over the keys (partern_attention.py:463-467): fp32
    probabilities (`sa_sampled_probs`) in q's dtype."""
    from .utils.mask_related import calc_attn

    return calc_attn(q, k)


# ---- head routing (partern_attention.py:463-521) ---------------------------------------------

SPARSE_KEEP, SPARSE_THR, SIM_THR = 0.2, 0.9, 0.9
_HEAD_CHUNK_BYTES = 4 << 30  # probability workspace per chunk of heads
_GRAM_CHUNK = 8              # sample positions per Gram partial (kGramChunk in judge.hip)


def _pad32(n: int) -> int:
    return -(-n // 32) * 32


def _compact(x, idx, n_pad):
    """Rows idx of x (bf16 [B,H,L,64]) as a contiguous [B*H, n_pad, 64] buffer, zero padded."""
    full = torch.full((n_pad,), -1, dtype=torch.int32)
    full[: idx.numel()] = idx.to(torch.int32)
    B, H = x.shape[:2]
    return gather_tokens(x, full.to(x.device)).reshape(B * H, n_pad, 64)


def _probs(qs, ks, rows, keys, n_bias, bias, c_lo, c_hi, P, sm_scale: float = scale_factor):
    BH = qs.shape[0]
    with torch.cuda.device(qs.device):
        _lib.check(_lib.load().sa_sampled_probs(
            qs.data_ptr(), ks.data_ptr(), BH, rows, qs.shape[1], keys, ks.shape[1], sm_scale, n_bias, bias,
            c_lo, c_hi, P.data_ptr(), P.stride(0), P.stride(1), _lib.stream_of(qs)), "sa_sampled_probs")


def _chunks(BH, bytes_per_head):
    step = max(1, _HEAD_CHUNK_BYTES // max(1, bytes_per_head))
    return [(h0, min(BH, h0 + step)) for h0 in range(0, BH, step)]


def _sparsity_rows(q, k, g: PatternGeometry, idx_q):
    """Per sampled first-frame query: mass of its top 20 % keys among every third token."""
    B, H = q.shape[:2]
    ns = idx_q.numel()
    keys = torch.arange(0, g.L, 3)
    n = keys.numel()
    qs, ks = _compact(q, idx_q + g.text_length, _pad32(ns)), _compact(k, keys, _pad32(n))
    K = int(n * SPARSE_KEEP)
    share = torch.empty(B * H, ns, dtype=torch.float32, device=q.device)
    # rows padded to whole 128-byte lines
    for h0, h1 in _chunks(B * H, ns * _pad32(n) * 4):
        P = torch.empty(h1 - h0, ns, _pad32(n), dtype=torch.float32, device=q.device)
        _probs(qs[h0:h1], ks[h0:h1], ns, n, 0, 0.0, 0, n, P)
        with torch.cuda.device(q.device):
            _lib.check(_lib.load().sa_topk_share(P.data_ptr(), P.stride(0), P.stride(1), h1 - h0, ns, n, K,
                                                 share[h0:h1].data_ptr(), _lib.stream_of(q)), "sa_topk_share")
    return share


def _similarity_inputs(q, k, g: PatternGeometry, index_k):
    T, F, ns = g.text_length, g.frames, g.sample_num
    nv = F * ns
    qs = _compact(q, index_k[T:], _pad32(nv))
    ks = _compact(k, index_k, _pad32(T + nv))
    B, H = q.shape[:2]
    G = torch.empty(B * H, F, -(-ns // _GRAM_CHUNK), F * (F + 1) // 2, dtype=torch.float32, device=q.device)
    return qs, ks, G


def _similarity_gram(q, k, g: PatternGeometry, index_k):
    """Gram partials [B*H, F, ceil(ns/8), F(F+1)/2] of the sampled frame-pair attention patterns,
    computed without writing the probabilities (one fused kernel)."""
    T, F, ns = g.text_length, g.frames, g.sample_num
    qs, ks, G = _similarity_inputs(q, k, g, index_k)
    with torch.cuda.device(q.device):
        _lib.check(_lib.load().sa_pattern_sim_gram(
            qs.data_ptr(), ks.data_ptr(), qs.shape[0], F, ns, T, qs.shape[1], ks.shape[1], scale_factor,
            composition_bias(g), G.data_ptr(), _lib.stream_of(q)), "sa_pattern_sim_gram")
    return G


def _similarity_gram_via_probs(q, k, g: PatternGeometry, index_k):
    """The same partials through the written probabilities (sa_sampled_probs + sa_pattern_gram)."""
    T, F, ns = g.text_length, g.frames, g.sample_num
    nv = F * ns
    qs, ks, G = _similarity_inputs(q, k, g, index_k)
    BH = qs.shape[0]
    for h0, h1 in _chunks(BH, nv * _pad32(nv) * 4):
        P = torch.empty(h1 - h0, nv, _pad32(nv), dtype=torch.float32, device=q.device)
        _probs(qs[h0:h1], ks[h0:h1], nv, T + nv, T, composition_bias(g), T, T + nv, P)
        with torch.cuda.device(q.device):
            _lib.check(_lib.load().sa_pattern_gram(P.data_ptr(), P.stride(0), P.stride(1), h1 - h0, F, ns,
                                                   G[h0:h1].data_ptr(), _lib.stream_of(q)), "sa_pattern_gram")
    return G


def _finish(share, G1, G2, BH, rows, F, ns, device):
    f32 = dict(dtype=torch.float32, device=device)
    sm, c1, c2 = torch.empty(BH, **f32), torch.empty(BH, **f32), torch.empty(BH, **f32)
    use = torch.empty(BH, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        _lib.check(_lib.load().sa_pattern_judge_finish(
            _lib.ptr(share), _lib.ptr(G1), _lib.ptr(G2), BH, rows, F, ns, SPARSE_THR, SIM_THR, sm.data_ptr(),
            c1.data_ptr(), c2.data_ptr(), use.data_ptr(), torch.cuda.current_stream(device).cuda_stream),
            "sa_pattern_judge_finish")
    return sm, c1, c2, use


def judge_sparsity(q, k, geometry: PatternGeometry = DEFAULT, idx_q=None, return_share=False):
    """True for heads whose sampled first-frame queries put > 90 % of their mass on the top
    20 % of (every third) key (:468-476). idx_q: first-frame positions (default: a randperm)."""
    g = geometry
    q, k = _prep_qkv(q), _prep_qkv(k)
    _lib.require_gpu(q, k)
    if idx_q is None:
        idx_q = torch.randperm(g.S)[: g.sample_num]
    B, H = q.shape[:2]
    share = _sparsity_rows(q, k, g, idx_q)
    sm, _, _, _ = _finish(share, None, None, B * H, idx_q.numel(), g.frames, g.sample_num, q.device)
    sparse = (sm > SPARSE_THR).view(B, H)
    return (sparse, sm.view(B, H)) if return_share else sparse


def judge_similarity(q, k, geometry: PatternGeometry = DEFAULT, index_k=None, return_sim=False):
    """True for heads whose sampled frame-pair attention patterns sharing a key frame have a
    mean cosine similarity > 0.9 (:477-514)."""
    g = geometry
    q, k = _prep_qkv(q), _prep_qkv(k)
    _lib.require_gpu(q, k)
    if index_k is None:
        _, index_k = get_indexs(g)
    B, H = q.shape[:2]
    G = _similarity_gram(q, k, g, index_k)
    _, c1, _, _ = _finish(None, G, None, B * H, 1, g.frames, g.sample_num, q.device)
    sim = (c1 > SIM_THR).view(B, H)
    return (sim, c1.view(B, H)) if return_sim else sim


def unified_judge(q, k, geometry: PatternGeometry = DEFAULT, draws=None):
    """Heads routed to the pattern attention: not sparse and self-similar twice (:516-521).
    draws = (idx_q, index_k1, index_k2) overrides the three randperm draws."""
    g = geometry
    q, k = _prep_qkv(q), _prep_qkv(k)
    _lib.require_gpu(q, k)
    if draws is None:
        idx_q = torch.randperm(g.S)[: g.sample_num]
        _, ik1 = get_indexs(g)
        _, ik2 = get_indexs(g)
    else:
        idx_q, ik1, ik2 = draws
    B, H = q.shape[:2]
    # The sparsity judge (written probabilities and a latency-bound top-k pass) runs on a
    # second stream (default priority) beside the two similarity judges (exp2/VALU-bound).
    main = torch.cuda.current_stream(q.device)
    side = _side_stream(q.device) if OVERLAP_JUDGE else main
    side.wait_stream(main)
    with torch.cuda.stream(side):
        share = _sparsity_rows(q, k, g, idx_q)
    G1 = _similarity_gram(q, k, g, ik1)
    G2 = _similarity_gram(q, k, g, ik2)
    main.wait_stream(side)
    share.record_stream(main)
    sm, c1, c2, use = _finish(share, G1, G2, B * H, idx_q.numel(), g.frames, g.sample_num, q.device)
    return use.view(B, H).bool()
