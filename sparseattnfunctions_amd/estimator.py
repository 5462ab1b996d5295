"""The adaptive block-mask source of SparseGen_Plus on the GPU: sampled block scores and the
energy-threshold / adaptive top-k selection.

Every function launches HIP kernels of libsa_hip.so (`sa_sample_block_tokens`,
`sa_sampled_block_scores`, `sa_energy_kv_list`); PyTorch allocates the buffers and, like
the reference, draws the uniform numbers that pick the sampled tokens (`torch.rand` of shape
[B, H, nb, 64], first for q then for k, utils/mask_related.py:26).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._kv import KVList
from .block_masks import _prep

BLOCK = 64
MODES = {"energy": 0, "topk": 1}
# Selection rules of the backup block mask (utils/mask_related.py:224-232, 366-391): "inclusive"
# keeps the sorted prefix through the first position reaching the threshold (the last one when
# none does); "cumulative" keeps the positions whose cumulative sum stays within it, plus the last.
CUT_MODES = {"inclusive": 2, "cumulative": 3}


def _ns_pad(nb: int, num_keep: int) -> int:
    return -(-nb * num_keep // 32) * 32


def _draws(B: int, H: int, nb: int, device, generator: Optional[torch.Generator]) -> torch.Tensor:
    return torch.rand(B, H, nb, BLOCK, device=device, generator=generator)


def sample_block_tokens(q: torch.Tensor, k: Optional[torch.Tensor] = None, num_keep: int = 8,
                        rand_q: Optional[torch.Tensor] = None, rand_k: Optional[torch.Tensor] = None,
                        generator: Optional[torch.Generator] = None):
    """Sampled tokens of every 64-token block (random_sample_tokens on the replicate-padded
    tensor, utils/mask_related.py:2-37).

    Returns (q_sampled, k_sampled, tok_q, tok_k): bf16 [B*H, ns_pad, 64] row buffers (rows past
    nb*num_keep unspecified; k_sampled None without k) and int32 [B*H, nb*num_keep] token ids.
    `rand_q`/`rand_k` (fp32 [B, H, nb, 64]) default to fresh `torch.rand` draws.
    """
    _lib.require_gpu(q, k)
    q = _prep(q)
    B, H, L, D = q.shape
    if k is not None:
        k = _prep(k)
        if k.shape != q.shape:
            raise ValueError("sample_block_tokens: q and k must have the same shape")
    nb = math.ceil(L / BLOCK)
    if rand_q is None:
        rand_q = _draws(B, H, nb, q.device, generator)
    if k is not None and rand_k is None:
        rand_k = _draws(B, H, nb, q.device, generator)
    for r in (rand_q, rand_k):
        if r is not None and tuple(r.shape) != (B, H, nb, BLOCK):
            raise ValueError(f"draws must have shape {(B, H, nb, BLOCK)}, got {tuple(r.shape)}")
    rand_q = rand_q.to(device=q.device, dtype=torch.float32).contiguous()
    if rand_k is not None:
        rand_k = rand_k.to(device=q.device, dtype=torch.float32).contiguous()
    ns_pad = _ns_pad(nb, num_keep)
    qs = torch.empty(B * H, ns_pad, D, dtype=torch.bfloat16, device=q.device)
    tq = torch.empty(B * H, nb * num_keep, dtype=torch.int32, device=q.device)
    ks = tk = None
    if k is not None:
        ks = torch.empty_like(qs)
        tk = torch.empty_like(tq)
    with torch.cuda.device(q.device):
        rc = _lib.load().sa_sample_block_tokens(
            rand_q.data_ptr(), q.data_ptr(), _lib.i64(*q.stride()[:3]),
            _lib.ptr(rand_k), _lib.ptr(k), _lib.i64(*k.stride()[:3]) if k is not None else None,
            B, H, L, D, int(num_keep), tq.data_ptr(), _lib.ptr(tk), qs.data_ptr(), _lib.ptr(ks), ns_pad,
            _lib.stream_of(q))
    _lib.check(rc, "sa_sample_block_tokens")
    return qs, ks, tq, tk


def sampled_block_scores(q: torch.Tensor, k: torch.Tensor, num_keep: int = 16,
                         rand_q: Optional[torch.Tensor] = None, rand_k: Optional[torch.Tensor] = None,
                         generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """Block scores of calc_attn_block_sum_efficient (utils/mask_related.py:40-81): softmax of
    the sampled q.k/8 summed over num_keep x num_keep cells. fp32 [B, H, nb, nb]."""
    B, H, L, _ = q.shape
    nb = math.ceil(L / BLOCK)
    qs, ks, _, _ = sample_block_tokens(q, k, num_keep, rand_q, rand_k, generator)
    pooled = torch.empty(B, H, nb, nb, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        rc = _lib.load().sa_sampled_block_scores(qs.data_ptr(), ks.data_ptr(), B * H, nb, int(num_keep),
                                                 qs.shape[1], pooled.data_ptr(), _lib.stream_of(q))
    _lib.check(rc, "sa_sampled_block_scores")
    return pooled


def retain_bounds(seq: int, min_retain_ratio: float, max_retain_ratio: float):
    """The reference's integer bounds: max(1, int(seq * ratio)) (SparseGen_Plus.py:57-58)."""
    return max(1, int(seq * min_retain_ratio)), max(1, int(seq * max_retain_ratio))


def initial_k(seq: int, init_k) -> int:
    """Starting k of the "topk" mode: seq * init_k when init_k < 1, truncated to an integer
    as torch.full(..., dtype=int64) does (SparseGen_Plus.py:31, 36)."""
    if init_k is None:
        raise ValueError("mode 'topk' needs an initial k (init_k)")
    k0 = seq * init_k if init_k < 1 else init_k
    return int(k0)


def energy_kv_list(scores: torch.Tensor, mode: str = "energy", init_k=None, max_retain_ratio: float = 0.7,
                   min_retain_ratio: float = 0.1, energy_threshold: float = 0.95, n_text_blocks: int = 4,
                   return_mask: bool = False):
    """Per-row selection of transfer_attn_to_mask (SparseGen_Plus.py:12-84) over fp32 block
    scores [B, H, nqb, nkb] -> KVList (and the dense bool mask when asked)."""
    _lib.require_gpu(scores)
    if scores.dim() != 4:
        raise ValueError(f"scores must be [B, H, nqb, nkb], got {tuple(scores.shape)}")
    if mode not in MODES:
        raise ValueError(f"Unsupported mode: {mode}")
    B, H, nqb, nkb = scores.shape
    seq = nkb
    min_keep, max_keep = retain_bounds(seq, min_retain_ratio, max_retain_ratio)
    k0 = initial_k(seq, init_k) if mode == "topk" else 1
    if mode == "topk" and not 1 <= k0 <= seq:
        raise ValueError(f"topk mode: initial k {k0} outside [1, {seq}]")
    s = scores.to(torch.float32).contiguous()
    kv = KVList.empty(B, H, nqb, nkb, s.device)
    mask = torch.empty(B, H, nqb, nkb, dtype=torch.uint8, device=s.device) if return_mask else None
    with torch.cuda.device(s.device):
        rc = _lib.load().sa_energy_kv_list(
            s.data_ptr(), B * H, nqb, nkb, MODES[mode], float(energy_threshold), min_keep, max_keep, k0,
            int(n_text_blocks), kv.idx.data_ptr(), kv.max_cnt, kv.cnt.data_ptr(), _lib.ptr(mask),
            _lib.stream_of(s))
    _lib.check(rc, "sa_energy_kv_list")
    return (kv, mask.bool()) if return_mask else kv


def energy_mask(scores: torch.Tensor, mode: str, threshold: float) -> torch.Tensor:
    """Energy cut of every row of fp32 scores [G, rows, n] (n <= 1024) on the GPU with the
    rules of CUT_MODES (`sa_energy_kv_list` modes 2 and 3, no clamping, no text blocks):
    bool [G, rows, n]. Ranks order (score descending, column ascending); the cumulative sums
    are sequential fp32 additions in rank order and the total is their last value."""
    _lib.require_gpu(scores)
    if scores.dim() != 3:
        raise ValueError(f"scores must be [G, rows, n], got {tuple(scores.shape)}")
    if mode not in CUT_MODES:
        raise ValueError(f"Unsupported mode: {mode}")
    G, rows, n = scores.shape
    s = scores.to(torch.float32).contiguous()
    kv = KVList.empty(G, 1, rows, n, s.device)
    mask = torch.empty(G, rows, n, dtype=torch.uint8, device=s.device)
    with torch.cuda.device(s.device):
        rc = _lib.load().sa_energy_kv_list(
            s.data_ptr(), G, rows, n, CUT_MODES[mode], float(threshold), 0, n, 1, 0, kv.idx.data_ptr(), kv.max_cnt,
            kv.cnt.data_ptr(), mask.data_ptr(), _lib.stream_of(s))
    _lib.check(rc, "sa_energy_kv_list")
    return mask.bool()
