"""CogVideoX geometry and the synthetic inputs of the benchmark configurations.

Geometry follows the reference's hard-coded CogVideoX-2B layout: 226 text tokens first,
then 13 x 30 x 45 video tokens in row-major (t, h, w) order (MergeAttention.py:26,33-38;
SildingTileAttention.py:100-105), d = 64, 30 heads; CogVideoX1.5-5B is 224 text +
11 x 48 x 85 (partern_attention.py:10-16).

Inputs (the benchmark configurations): q, k = N(0,1) + amp * code(t, h, w) and v = N(0,1),
drawn on the CPU from one torch.Generator in the order q-noise, k-noise, v, then rounded to
bf16. code(t, h, w) is a unit-norm 64-d sinusoidal position code: dims 0-21 encode t,
22-43 encode h, 44-63 encode w, each axis as (sin, cos) pairs at frequencies
10000^(-2j/n_axis); the concatenation is L2-normalised. Text tokens get a zero code.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Tuple

import torch


@dataclass(frozen=True)
class Geometry:
    text_len: int = 226
    T: int = 13
    Hp: int = 30
    Wp: int = 45
    block: int = 64

    @property
    def frame(self) -> int:
        return self.Hp * self.Wp

    @property
    def n_video(self) -> int:
        return self.T * self.Hp * self.Wp

    @property
    def L(self) -> int:
        return self.text_len + self.n_video

    @property
    def nb(self) -> int:
        return math.ceil(self.L / self.block)

    @property
    def n_text_blocks(self) -> int:
        """Block rows/columns holding text tokens, forced dense (SparseGen_Plus.py:81-82)."""
        return math.ceil(self.text_len / self.block)


COGVIDEOX_2B = Geometry()
COGVIDEOX_15_5B = Geometry(text_len=224, T=11, Hp=48, Wp=85)

_AXIS_DIMS = (22, 22, 20)


def position_code(geom: Geometry, d: int = 64) -> torch.Tensor:
    """[L, d] fp32: zero rows for text, unit-norm sinusoidal (t, h, w) code for video."""
    assert d == sum(_AXIS_DIMS)
    n = torch.arange(geom.n_video, dtype=torch.float64)
    t = torch.div(n, geom.frame, rounding_mode="floor")
    h = torch.div(n - t * geom.frame, geom.Wp, rounding_mode="floor")
    w = n - t * geom.frame - h * geom.Wp
    parts = []
    for pos, nd in zip((t, h, w), _AXIS_DIMS):
        j = torch.arange(nd // 2, dtype=torch.float64)
        freq = torch.pow(10000.0, -2.0 * j / nd)
        ang = pos[:, None] * freq[None, :]
        pair = torch.stack((torch.sin(ang), torch.cos(ang)), dim=-1).reshape(-1, nd)
        parts.append(pair)
    code = torch.cat(parts, dim=1)
    code = code / code.norm(dim=1, keepdim=True)
    out = torch.zeros(geom.L, d, dtype=torch.float32)
    out[geom.text_len:] = code.to(torch.float32)
    return out


def cogvideox_qkv(seed: int, B: int = 2, H: int = 30, geom: Geometry = COGVIDEOX_2B, d: int = 64,
                  amp: float = 2.0, heads: Tuple[int, int] = None, device: str = "cpu") -> Tuple[torch.Tensor, ...]:
    """q, k, v bf16 [B, H, L, d] (configs 2-5), drawn on the CPU generator by default.

    `heads=(h0, h1)` returns only heads h0..h1-1 of the same draw (all heads are drawn so
    that the values do not depend on the slice). `device="cuda"` draws with that device's
    generator instead (same distribution, different values; used where the CPU draw of many
    layers would dominate the run time)."""
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (B, H, geom.L, d)
    code = position_code(geom, d).to(device)
    out = []
    for i in range(3):
        x = torch.randn(shape, generator=g, dtype=torch.float32, device=device)
        if i < 2:
            x.add_(code, alpha=amp)
        if heads is not None:
            x = x[:, heads[0]:heads[1]]
        out.append(x.to(torch.bfloat16))
    return tuple(out)


def config1_inputs():
    """Config 1: B=1, H=2, L=2048, d=64 fp32 q,k,v ~ N(0,1) (seed 0), and a block mask
    (seed 1) that keeps each row block's diagonal block plus each other block with
    probability 0.25."""
    g = torch.Generator(device="cpu").manual_seed(0)
    shape = (1, 2, 2048, 64)
    q = torch.randn(shape, generator=g)
    k = torch.randn(shape, generator=g)
    v = torch.randn(shape, generator=g)
    g1 = torch.Generator(device="cpu").manual_seed(1)
    nb = 2048 // 64
    mask = torch.rand((1, 2, nb, nb), generator=g1) < 0.25
    mask |= torch.eye(nb, dtype=torch.bool)[None, None]
    return q, k, v, mask, 1.0 / 8.0


def topk_count(ratio: float, nb: int) -> int:
    """Blocks kept per row for a keep ratio: `int(seq * ratio)` as the reference truncates
    (SparseGen_Plus.py:31,57)."""
    return int(nb * ratio) if ratio < 1 else int(ratio)
