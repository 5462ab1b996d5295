"""ToMe bipartite soft matching for video tokens (drop-in for utils/merge_unmerge.py).

`bipartite_soft_matching_video(metric, w, h, t, sx, sy, st, r, no_rand=False,
generator=None)` keeps the reference signature and returns `(merge, unmerge)` closures
(merge_unmerge.py:34-156); the module global `counter` holds the dst sizes
[B, num_dst, 1] int64 after each call (:33, :113-116), as MergeAttention reads it. The
matching, the maps and the merge/unmerge gathers run as HIP kernels (`sa_tome_*`).

Semantics and the deliberate differences:
  * partition: first frame all dst, one dst per (st, sy, sx) cell (random offset from
    `generator` unless `no_rand`), dst/src in ascending token order (a stable version of
    the reference's argsort, :82);
  * scores in fp32 (cosine of the fp32-normalised metric), never materialised; argmax ties
    go to the lowest dst, the edge order is a stable descending sort (torch leaves both
    unspecified);
  * closures take the tokens WITH the `text_len` (226) text tokens first, as the
    reference's 4-D path does (:120-122, :139-141): x [G, L, 64] (3-D, G = metric batch) or
    [b, h, L, 64] (4-D, b*h a multiple of G; consecutive heads share a group), and return
    the same rank; merged dst rows are fp32 means rounded once to bf16; only mode="mean".
"""
from __future__ import annotations

from typing import Callable, Tuple

import torch

from .. import _tome

counter = None


def do_nothing(x: torch.Tensor, mode: str = None):
    return x


def init_generator(device: torch.device, fallback: torch.Generator = None):
    """Reference helper (merge_unmerge.py:8-22): a generator seeded from the global RNG."""
    if device.type == "cpu":
        return torch.Generator(device="cpu").set_state(torch.get_rng_state())
    if device.type == "cuda":
        return torch.Generator(device=device).set_state(torch.cuda.get_rng_state())
    return init_generator(torch.device("cpu")) if fallback is None else fallback


def draw_cell_choice(t: int, h: int, w: int, sx: int, sy: int, st: int, generator: torch.Generator = None):
    """The dst offset of each (st, sy, sx) cell of frames 1..t-1, drawn as the reference draws
    it (merge_unmerge.py:69: `torch.randint(sy*sx*st, (tst, hsy, wsx, 1))` on the generator's
    device, the same values in the same order); int32 [tst, hsy, wsx] on the CPU."""
    tst, hsy, wsx = (t - 1) // st, h // sy, w // sx
    dev = generator.device if generator is not None else torch.device("cpu")
    return torch.randint(sy * sx * st, size=(tst, hsy, wsx, 1), device=dev, generator=generator).reshape(
        tst, hsy, wsx).to(device="cpu", dtype=torch.int32)


def bipartite_soft_matching_video(metric: torch.Tensor, w: int, h: int, t: int, sx: int, sy: int, st: int, r: int,
                                  no_rand: bool = False, generator: torch.Generator = None,
                                  text_len: int = 226) -> Tuple[Callable, Callable]:
    global counter
    G, N, C = metric.shape
    if r <= 0:
        return do_nothing, do_nothing
    if N != t * h * w:
        raise ValueError(f"metric has {N} tokens, expected t*h*w = {t * h * w}")
    choice = None if no_rand else draw_cell_choice(t, h, w, sx, sy, st, generator)
    a_idx, b_idx = _tome.partition(t, h, w, sx, sy, st, metric.device, cell_choice=choice)
    maps = _tome.match(_tome.normalize(metric), a_idx, b_idx, r, text_len)
    counter = maps.sizes.to(torch.int64).reshape(G, maps.n_dst, 1)

    def _as4(x):
        if x.dim() == 3:
            return x.unsqueeze(1), True
        return x, False

    def _group(x4):
        heads = x4.shape[0] * x4.shape[1]
        if heads % G:
            raise ValueError(f"{heads} heads do not split into {G} matching groups")
        return heads // G

    def merge(x: torch.Tensor, mode: str = "mean") -> torch.Tensor:
        if mode != "mean":
            raise NotImplementedError("only mode='mean' (the reference's default) is implemented")
        x4, squeeze = _as4(x)
        hpg = _group(x4)
        if x4.shape[1] % hpg:
            raise ValueError("heads of one matching group must belong to one batch item")
        out = _tome.merge(x4, maps, hpg)
        return out.squeeze(1) if squeeze else out

    def unmerge(x: torch.Tensor) -> torch.Tensor:
        x4, squeeze = _as4(x)
        out = _tome.unmerge(x4, maps, _group(x4))
        return out.squeeze(1) if squeeze else out

    merge.maps = unmerge.maps = maps
    return merge, unmerge
