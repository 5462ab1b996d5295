"""Local window of the combined mask on a permuted token layout -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Restates the centre-token rule of the combined mask (the local part of the reference's local
windows, SildingTileAttention.py:18-87, SmartAttention.py:56-67, LocalGlobalAttention.py:
114-179) for a layout whose position j holds natural token perm[j] (as the 1.5-5B rearranger
of combined_attn.py:17-31 produces): block b is represented by natural token
perm[min(64b + 32, L - 1)]; two video blocks are in the window when their (t, h, w) differ by
at most (dt, dh, dw); rows and columns of blocks holding any text token are kept.

Pinned by tests/test_oracle_local.py: with the identity permutation it equals the C oracle's
bitmap (oracle_local_window) united with the text rows and columns, and a pure-Python brute
force on a tiny geometry with a random permutation.
"""
from __future__ import annotations

import torch


def local_window_perm(perm, L, block, text_len, T, Hp, Wp, dt, dh, dw) -> torch.Tensor:
    perm = torch.as_tensor(perm).to(torch.int64)
    nb = -(-L // block)
    centre = perm[torch.clamp(torch.arange(nb) * block + block // 2, max=L - 1)]
    video = centre >= text_len
    v = torch.clamp(centre - text_len, min=0)
    t, h, w = v // (Hp * Wp), (v // Wp) % Hp, v % Wp
    win = (video[:, None] & video[None, :] & ((t[:, None] - t[None, :]).abs() <= dt)
           & ((h[:, None] - h[None, :]).abs() <= dh) & ((w[:, None] - w[None, :]).abs() <= dw))
    has_text = torch.zeros(nb, dtype=torch.bool)
    has_text.scatter_(0, torch.arange(L)[perm < text_len] // block, True)
    return (win | has_text[:, None] | has_text[None, :]).to(torch.uint8)
