"""`CombinedAttn` processor of special_attentions/combined_attn.py (:7-101), on MI355X.

Keeps the reference API -- `CombinedAttn(warmup_epoch=5)`, `__call__(q, k, v,
use_rearranger=False)`, the per-call counter `ct` with `layer_num` calls per denoising step
and dense attention during the first `warmup_epoch` steps (:42-46) -- and computes the
combined block mask of the MI355X build on the GPU:

    keep(qb, kb) = local 3-D window (+-1 latent frame, +-8 patch rows/cols between block
                   centre tokens, a static bitmap cached per geometry)
                 U global top-k of the mean-pooled block scores (k = int(0.10 * nb))
                 U text block rows and columns,

then runs the block-sparse attention kernel on it.

`CombinedAttn(head_routing=True)` is the reference's own 1.5-5B body instead
(combined_attn.py:42-101): after the warm-up steps, `unified_judge` (partern_attention.py:
516-521) routes each head either to the frame-pattern attention (`ParternAttentionColVersion_V2`,
at most 48 heads per call as the reference does) or to SparseGen_Plus's block-sparse
attention, optionally through the 1.5-5B token permutation (`use_rearranger=True`); the
routing needs one host synchronisation per call (the count of pattern heads), as in the
reference. Selected heads are copied with torch's index_select/index_copy_.
`rearranger` / `recover` are the reference's 1.5-5B token permutations (combined_attn.py:
17-41), as GPU gathers. Without head routing, `use_rearranger=True` (1.5-5B geometry) applies
the combined rule in the rearranged layout, as the reference's block-sparse heads are
estimated there: block means of the permuted q and k for the global top-k, the local window
between the original (t, h, w) of the permuted blocks' centre tokens, the blocks holding text
(last in that layout) dense; the output is recovered to the natural order.
"""
from __future__ import annotations

import math

import torch

from ._gather import gather_tokens
from .block_mask_attn import dense_kv_list
from .block_masks import local_window_bitmap, local_window_bitmap_perm, meanpool_topk_kv_list
from .utils.block_sparse_attn_kernel import block_sparse_attention
from .workloads import COGVIDEOX_2B, Geometry, topk_count


# The reference's 1.5-5B permutation (combined_attn.py:17-41): 224 text tokens first, then
# 11 x 48 x 85 video tokens in (t, h, w) order. Frames 0-8 are cut into 3 x 4 x 5 cubes and
# frames 9-10 into 2 x 6 x 5 cubes (frame, row, column sizes); the output lists the cubes of
# each chunk in (frame group, row group, column group) order with each cube's tokens in
# (frame, row, column) order, chunk 1 then chunk 2, then the text tokens.
_R_TEXT, _R_T, _R_H, _R_W = 224, 11, 48, 85
_R_CHUNKS = ((0, 3, 3, 12, 4, 17, 5), (9, 1, 2, 8, 6, 17, 5))  # first frame, fgroups, f, rgroups, r, cgroups, c


def rearranger_permutation() -> torch.Tensor:
    """int32 [L]: output token j of `rearranger` is input token perm[j] (CPU tensor)."""
    parts = []
    for t0, nfg, nf, nrg, nr, ncg, nc in _R_CHUNKS:
        t = torch.arange(nfg * nf).reshape(nfg, 1, 1, nf, 1, 1) + t0
        h = torch.arange(nrg * nr).reshape(1, nrg, 1, 1, nr, 1)
        w = torch.arange(ncg * nc).reshape(1, 1, ncg, 1, 1, nc)
        # dims: (frame group, row group, column group, frame, row, column) of each cube token
        tok = (t.reshape(nfg, 1, 1, nf, 1, 1) * _R_H + h) * _R_W + w
        tok = tok.expand(nfg, nrg, ncg, nf, nr, nc)
        parts.append(_R_TEXT + tok.reshape(-1))
    parts.append(torch.arange(_R_TEXT))
    return torch.cat(parts).to(torch.int32)


_PERM_CACHE = {}


def _perms(device):
    key = str(device)
    if key not in _PERM_CACHE:
        perm = rearranger_permutation()
        inv = torch.empty_like(perm)
        inv[perm.long()] = torch.arange(perm.numel(), dtype=torch.int32)
        _PERM_CACHE[key] = (perm.to(device), inv.to(device))
    return _PERM_CACHE[key]


class CombinedAttn:
    def __init__(self, warmup_epoch: int = 5, geometry: Geometry = COGVIDEOX_2B, global_ratio: float = 0.10,
                 window=(1, 8, 8), layer_num: int = 42, timestep: int = 50, sm_scale: float = None,
                 head_routing: bool = False, pattern_geometry=None, verbose: bool = False):
        self.layer_num = layer_num
        self.timestep = timestep
        self.counter = 0
        self.ct = 0
        self.warmup_epoch = warmup_epoch
        self.geometry = geometry
        self.global_ratio = global_ratio
        self.window = tuple(window)
        self.sm_scale = sm_scale
        self.last_kv = None
        # head_routing: the reference's 1.5-5B body (combined_attn.py:42-101): unified_judge
        # routes each head to the frame-pattern attention or to SparseGen_Plus's block-sparse
        # attention (dense during its warm-up).
        self.head_routing = head_routing
        self.verbose = verbose
        self.last_routing = None
        if head_routing:
            from .partern_attention import DEFAULT, ParternAttentionColVersion_V2
            from .SparseGen_Plus import BlockSparseAttention
            self.pat_attn = ParternAttentionColVersion_V2(pattern_geometry or DEFAULT)
            self.block_sparse_attention = BlockSparseAttention(block_size=64, layernum=layer_num, timestep=timestep,
                                                               num_samples=4, warmup_epoch=warmup_epoch,
                                                               verbose=verbose)

    def n_text_blocks(self) -> int:
        return math.ceil(self.geometry.text_len / self.geometry.block)

    def build_kv_list(self, q, k, with_fp16_keys: bool = False):
        """Combined-rule kv lists; with `with_fp16_keys`, (kv, fp16 keys made beside the top-k
        kernel) for block_sparse_attention(..., k16=...)."""
        L = q.shape[2]
        if L != self.geometry.L:
            raise ValueError(f"sequence length {L} does not match the geometry (L={self.geometry.L})")
        nb = math.ceil(L / 64)
        local = local_window_bitmap(self.geometry, self.window, q.device)
        return meanpool_topk_kv_list(q, k, topk_count(self.global_ratio, nb), self.n_text_blocks(),
                                     local_bitmap=local, with_fp16_keys=with_fp16_keys)

    @staticmethod
    def rearranger(q, k, v):
        """The 1.5-5B token permutation of q, k, v (L = 224 + 11*48*85): video cubes first,
        text last (combined_attn.py:17-31). Returns permuted copies."""
        L = _R_TEXT + _R_T * _R_H * _R_W
        if q.shape[2] != L or k.shape[2] != L or v.shape[2] != L:
            raise ValueError(f"rearranger expects the 1.5-5B sequence length {L}, got {q.shape[2]}")
        perm, _ = _perms(q.device)
        return tuple(gather_tokens(x, perm) for x in (q, k, v))

    @staticmethod
    def recover(out):
        """Inverse of `rearranger` for the attention output (combined_attn.py:32-40)."""
        L = _R_TEXT + _R_T * _R_H * _R_W
        if out.shape[2] != L:
            raise ValueError(f"recover expects the 1.5-5B sequence length {L}, got {out.shape[2]}")
        _, inv = _perms(out.device)
        return gather_tokens(out, inv)

    def _scale(self, q):
        return self.sm_scale if self.sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])

    def _pattern_heads(self, qs, ks, vs):
        # The reference runs the pattern attention on at most 48 selected heads at a time
        # (combined_attn.py:56-79); its modify-factor decision is taken per such call.
        outs = [self.pat_attn(qs[:, h:h + 48], ks[:, h:h + 48], vs[:, h:h + 48]) for h in range(0, qs.shape[1], 48)]
        return torch.cat(outs, dim=1)

    def _routed(self, q, k, v, use_rearranger):
        from .partern_attention import unified_judge
        if self.ct // self.layer_num < self.warmup_epoch:
            self.ct += 1
            return self.block_sparse_attention(q, k, v)
        self.ct += 1
        use = unified_judge(q, k, self.pat_attn.geometry)
        self.last_routing = use
        n_sel = int(use.sum().item())
        if n_sel == 0:
            return self.block_sparse_attention(q, k, v)
        B, H, L, D = q.shape
        flat = [x.reshape(B * H, L, D) for x in (q, k, v)]
        sel = use.reshape(-1).nonzero().squeeze(1)
        rest = (~use).reshape(-1).nonzero().squeeze(1)
        self.counter += n_sel
        pat = self._pattern_heads(*(x.index_select(0, sel).unsqueeze(0) for x in flat))
        parts = [pat[0]]
        if rest.numel() == 0:
            self.counter += n_sel
            self.block_sparse_attention.counter += 1
        else:
            qr, kr, vr = (x.index_select(0, rest).unsqueeze(0) for x in flat)
            if use_rearranger:
                qr, kr, vr = self.rearranger(qr, kr, vr)
            o = self.block_sparse_attention(qr, kr, vr)
            if use_rearranger:
                o = self.recover(o)
            parts.append(o[0])
        # Heads back in their order (the reference's out[use_pattern] = ... assignments,
        # combined_attn.py:50-97) as one gather from [pattern heads; other heads]: a zeroed
        # output with two index_copy_ scatters took 0.75 against 0.62 ms at 96 x 45 104 x 64.
        order = torch.cat([sel, rest])
        inv = torch.empty_like(order)
        inv[order] = torch.arange(order.numel(), device=order.device)
        out = torch.cat(parts).index_select(0, inv)
        if self.verbose:
            print("counter:", self.counter, "now increment:", n_sel)
        return out.view(B, H, L, D)

    def build_kv_list_rearranged(self, qr, kr):
        """Combined-rule kv lists in the rearranged layout (qr, kr from `rearranger`)."""
        g = self.geometry
        if (g.text_len, g.T, g.Hp, g.Wp) != (_R_TEXT, _R_T, _R_H, _R_W):
            raise ValueError("use_rearranger needs the 1.5-5B geometry (224 text + 11 x 48 x 85 video tokens)")
        nb = math.ceil(qr.shape[2] / 64)
        perm, _ = _perms("cpu")
        local = local_window_bitmap_perm(g, perm, self.window, qr.device)
        return meanpool_topk_kv_list(qr, kr, topk_count(self.global_ratio, nb), 0, local_bitmap=local)

    def __call__(self, q, k, v, use_rearranger: bool = False):
        if self.head_routing:
            return self._routed(q, k, v, use_rearranger)
        warm = self.ct // self.layer_num < self.warmup_epoch
        if use_rearranger:
            self.ct += 1
            qr, kr, vr = self.rearranger(q, k, v)
            B, H, L, _ = q.shape
            nb = math.ceil(L / 64)
            kv = dense_kv_list(B, H, nb, nb, q.device) if warm else self.build_kv_list_rearranged(qr, kr)
            self.last_kv = kv
            return self.recover(block_sparse_attention(qr, kr, vr, kv, self._scale(q)))
        self.ct += 1
        if warm:
            B, H, L, _ = q.shape
            nb = math.ceil(L / 64)
            kv = dense_kv_list(B, H, nb, math.ceil(k.shape[2] / 64), q.device)
        else:
            # bf16 scores: these lists (31-46 blocks of 278) earn less in the tile loop than the
            # fp16 copy of k costs the pooling pass
            kv = self.build_kv_list(q, k)
        self.last_kv = kv
        return block_sparse_attention(q, k, v, kv, self._scale(q), n_text_blocks=self.n_text_blocks())

    def sparsity(self) -> float:
        kv = self.last_kv
        return 1.0 - kv.cnt.sum().item() / (kv.rows * kv.nkb)
