"""`SildingTileAttention` processor of special_attentions/SildingTileAttention.py (:107-149).

The reference permutes the video tokens into 13x3x3 tiles (:111-131), runs
`flex_attention` with a BlockMask built from `sta_mask_3d` (:18-106) and permutes the
output back (:135-143). Here k and v are copied into the tile-major order by a
token-gather kernel, while the queries are read and the outputs written through the same
permutation by the attention kernel itself (row maps, `sa_block_sparse_fwd_mapped`). The
mask is compiled once per configuration (on the host, `sa_sta_block_masks`) into 64x64
block lists shared by every head, with a bitmask for each block a tile boundary cuts
through; the block-sparse kernel applies those bitmasks element-wise, so the result is the
same token-level mask as flex_attention's.

Difference by design: `preprocess` returns permuted copies instead of writing the
permutation into the caller's q, k, v (the reference mutates its inputs in place, :128-130).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._gather import gather_tokens as _gather
from ._kv import KVList
from .utils.block_sparse_attn_kernel import block_sparse_attention

config = {
    "kernel_size": (1, 9, 9),
    "tile_size": (13, 3, 3),
    "img_size": (13, 30, 45),
    "text_length": 226,
}


def generate_sta_mask(canvas_twh, kernel_twh, tile_twh, text_length):
    """The reference's mask_mod (SildingTileAttention.py:18-87) on the tile-major layout, as a
    torch function of (b, h, q_idx, kv_idx) index tensors (for inspection and tests)."""
    canvas_t, canvas_h, canvas_w = canvas_twh
    kernel_t, kernel_h, kernel_w = kernel_twh
    tile_t, tile_h, tile_w = tile_twh
    total = tile_t * tile_h * tile_w
    nt, nh, nw = canvas_t // tile_t, canvas_h // tile_h, canvas_w // tile_w

    def tile_of(idx):
        tid = torch.div(idx - text_length, total, rounding_mode="floor")
        return (torch.div(tid, nh * nw, rounding_mode="floor"),
                torch.div(tid % (nh * nw), nw, rounding_mode="floor"), tid % nw)

    def sta_mask_3d(b, h, q_idx, kv_idx):
        qt, qx, qy = tile_of(q_idx)
        kt, kx, ky = tile_of(kv_idx)
        ct = qt.clamp(kernel_t // 2, (nt - 1) - kernel_t // 2)
        cx = qx.clamp(kernel_h // 2, (nh - 1) - kernel_h // 2)
        cy = qy.clamp(kernel_w // 2, (nw - 1) - kernel_w // 2)
        window = ((ct - kt).abs() <= kernel_t // 2) & ((cx - kx).abs() <= kernel_h // 2) & \
                 ((cy - ky).abs() <= kernel_w // 2)
        image = (q_idx >= text_length) & (kv_idx >= text_length)
        return (image & window) | ((q_idx >= text_length) & (kv_idx < text_length)) | (q_idx < text_length)

    return sta_mask_3d


class StaLayout:
    """Device tables of one configuration: permutation, inverse, shared block lists, masks."""

    def __init__(self, kernel_size, tile_size, img_size, text_length, device):
        T, Hp, Wp = img_size
        self.L = text_length + T * Hp * Wp
        self.nb = math.ceil(self.L / 64)
        self.text_blocks = math.ceil(text_length / 64)
        lib = _lib.load()
        tile = (ctypes.c_int * 3)(*tile_size)
        kern = (ctypes.c_int * 3)(*kernel_size)
        perm = torch.empty(self.L, dtype=torch.int32)
        _lib.check(lib.sa_sta_permutation(text_length, T, Hp, Wp, tile, perm.data_ptr()), "sa_sta_permutation")
        n_slots = ctypes.c_int(0)
        _lib.check(lib.sa_sta_block_masks(text_length, T, Hp, Wp, tile, kern, None, None, None, None,
                                          ctypes.byref(n_slots)), "sa_sta_block_masks")
        nb = self.nb
        kv_idx = torch.zeros(nb, nb, dtype=torch.int32)
        kv_cnt = torch.zeros(nb, dtype=torch.int32)
        kv_slot = torch.full((nb, nb), -1, dtype=torch.int32)
        masks = torch.zeros(max(n_slots.value, 1), 64, dtype=torch.int64)
        _lib.check(lib.sa_sta_block_masks(text_length, T, Hp, Wp, tile, kern, kv_idx.data_ptr(), kv_cnt.data_ptr(),
                                          kv_slot.data_ptr(), masks.data_ptr(), ctypes.byref(n_slots)),
                   "sa_sta_block_masks")
        self.n_partial = n_slots.value
        self.perm = perm.to(device)
        self.inv = torch.empty_like(perm).scatter_(0, perm.long(), torch.arange(self.L, dtype=torch.int32)).to(device)
        self.kv_idx, self.kv_cnt, self.kv_slot, self.masks = (t.to(device) for t in (kv_idx, kv_cnt, kv_slot, masks))

    def density(self) -> float:
        return self.kv_cnt.sum().item() / (self.nb * self.nb)


_LAYOUTS = {}


def get_sliding_tile_attention_mask(kernel_size, tile_size, img_size, text_length, device):
    """Block lists + bitmasks of the sliding-tile mask (the reference builds a flex BlockMask
    here, SildingTileAttention.py:88-99), cached per configuration and device."""
    key = (tuple(kernel_size), tuple(tile_size), tuple(img_size), text_length, str(device))
    lay = _LAYOUTS.get(key)
    if lay is None:
        lay = StaLayout(kernel_size, tile_size, img_size, text_length, device)
        _LAYOUTS[key] = lay
    return lay


class SildingTileAttention:
    def __init__(self, config_=None):
        self.config = dict(config_ or config)
        self._layout = None

    @property
    def block_mask(self) -> StaLayout:
        return self._layout

    def _get_layout(self, device) -> StaLayout:
        c = self.config
        if self._layout is None or self._layout.perm.device != device:
            self._layout = get_sliding_tile_attention_mask(c["kernel_size"], c["tile_size"], c["img_size"],
                                                           c["text_length"], device)
        return self._layout

    def preprocess(self, q, k, v):
        lay = self._get_layout(q.device)
        return tuple(_gather(x, lay.perm) for x in (q, k, v))

    def process_out_back(self, out):
        return _gather(out, self._get_layout(out.device).inv)

    def attention(self, q, k, v, sm_scale=None):
        """Sliding-tile attention on inputs already in the tile-major layout."""
        lay = self._get_layout(q.device)
        B, H, L, D = q.shape
        if L != lay.L or k.shape != q.shape or v.shape != q.shape:
            raise ValueError(f"expected q, k, v of {lay.L} tokens for this configuration, got {tuple(q.shape)}")
        scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
        kv = KVList(lay.kv_idx, lay.kv_cnt, 1, 1, lay.nb, lay.nb)
        return block_sparse_attention(q, k, v, kv, scale, n_text_blocks=lay.text_blocks,
                                      tile_masks=(lay.kv_slot, lay.masks, True))

    def forward(self, q, k, v):
        """preprocess -> attention -> process_out_back, with the query permutation and the
        output's inverse permutation done by the attention kernel's loads and stores (row
        maps); only k and v are copied into the tile-major layout."""
        lay = self._get_layout(q.device)
        B, H, L, D = q.shape
        if L != lay.L or k.shape != q.shape or v.shape != q.shape:
            raise ValueError(f"expected q, k, v of {lay.L} tokens for this configuration, got {tuple(q.shape)}")
        kt, vt = _gather(k, lay.perm), _gather(v, lay.perm)
        kv = KVList(lay.kv_idx, lay.kv_cnt, 1, 1, lay.nb, lay.nb)
        return block_sparse_attention(q, kt, vt, kv, 1.0 / math.sqrt(D), n_text_blocks=lay.text_blocks,
                                      q_rows=lay.perm, o_rows=lay.perm,
                                      tile_masks=(lay.kv_slot, lay.masks, True))

    def __call__(self, *args, **kwds):
        return self.forward(*args, **kwds)
