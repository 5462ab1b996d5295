"""Sliding-tile attention layout and mask on the CPU -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Restates SildingTileAttention.py: the tile-major permutation "(nt tp nh hp nw wp) ->
(nt nh nw tp hp wp)" of the video tokens (:111-131) and the token mask sta_mask_3d
(:67-84: video pairs within the window of kernel-sized tiles around the query tile, the
centre clamped to the canvas; video -> text; text -> all). Pinned by
tests/test_oracle_sta.py against a pure-Python brute force on small grids.
"""
from __future__ import annotations

import torch


def permutation(text_len, img_size, tile_size) -> torch.Tensor:
    """perm[j] = natural token at tile-major position j (int64)."""
    T, Hp, Wp = img_size
    tt, th, tw = tile_size
    nt, nh, nw = T // tt, Hp // th, Wp // tw
    nat = torch.arange(T * Hp * Wp).reshape(nt, tt, nh, th, nw, tw)
    tile_major = nat.permute(0, 2, 4, 1, 3, 5).reshape(-1)
    return torch.cat([torch.arange(text_len), text_len + tile_major])


def token_mask(rows, L, text_len, img_size, tile_size, kernel_size) -> torch.Tensor:
    """bool [len(rows), L]: the sta_mask_3d of tile-major query positions `rows`."""
    T, Hp, Wp = img_size
    tt, th, tw = tile_size
    kt, kh, kw = kernel_size
    nt, nh, nw = T // tt, Hp // th, Wp // tw
    total = tt * th * tw

    def tile(idx):
        tid = torch.div(idx - text_len, total, rounding_mode="floor")
        return torch.div(tid, nh * nw, rounding_mode="floor"), torch.div(tid % (nh * nw), nw, rounding_mode="floor"), tid % nw

    q = rows[:, None]
    k = torch.arange(L)[None, :]
    qt, qh, qw = tile(q)
    ct = qt.clamp(kt // 2, nt - 1 - kt // 2)
    ch = qh.clamp(kh // 2, nh - 1 - kh // 2)
    cw = qw.clamp(kw // 2, nw - 1 - kw // 2)
    ktile, khh, kww = tile(k)
    win = ((ct - ktile).abs() <= kt // 2) & ((ch - khh).abs() <= kh // 2) & ((cw - kww).abs() <= kw // 2)
    return ((q >= text_len) & (k >= text_len) & win) | ((q >= text_len) & (k < text_len)) | (q < text_len)
