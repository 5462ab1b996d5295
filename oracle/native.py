"""ctypes wrapper of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

All functions take and return CPU torch tensors.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        L.oracle_block_pool.argtypes = [_P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _P]
        L.oracle_block_pool.restype = None
        L.oracle_block_score.argtypes = [_P, _P, _I]
        L.oracle_block_score.restype = ctypes.c_float
        L.oracle_block_topk.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P]
        L.oracle_block_topk.restype = None
        L.oracle_energy_list.argtypes = [_P, _I, _I, _I, _I, ctypes.c_float, _I, _I, _I, _I, _P, _I, _P, _P]
        L.oracle_energy_list.restype = None
        L.oracle_local_window.argtypes = [_I] * 9 + [_P]
        L.oracle_local_window.restype = None
        L.oracle_tome_partition.argtypes = [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]
        L.oracle_tome_partition.restype = None
        L.oracle_tome_metric.argtypes = [_P, _P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _P]
        L.oracle_tome_metric.restype = None
        L.oracle_tome_argmax.argtypes = [_P, _I, _I, _I, _P, _I, _P, _I, _P, _P]
        L.oracle_tome_argmax.restype = None
        L.oracle_tome_maps.argtypes = [_P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P]
        L.oracle_tome_maps.restype = None
        L.oracle_tome_match.argtypes = [_P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]
        L.oracle_tome_match.restype = None
        L.oracle_tome_merge.argtypes = [_P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _P, _P]
        L.oracle_tome_merge.restype = None
        _lib = L
    return _lib


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def block_pool(x: torch.Tensor, block: int = 64) -> torch.Tensor:
    """x bf16 [B,H,L,D] (CPU) -> fp32 [B*H, nb, D] block means."""
    assert x.dtype == torch.bfloat16 and x.stride(-1) == 1
    B, H, L, D = x.shape
    nb = -(-L // block)
    out = torch.empty(B * H, nb, D, dtype=torch.float32)
    lib().oracle_block_pool(_p(x.view(torch.int16)), x.stride(0), x.stride(1), x.stride(2), B, H, L, D, block, _p(out))
    return out


def block_topk(qp, kp, topk: int, n_text: int, local=None, scores_in=None, nqb=None, nkb=None):
    """Returns (kv_idx [rows, nkb], kv_cnt [rows], mask [rows, nkb] uint8, scores [rows, nkb])."""
    if scores_in is not None:
        BH, nqb, nkb = scores_in.shape
        D = 0
        scores_in = scores_in.contiguous().float()
    else:
        BH, nqb, D = qp.shape
        nkb = kp.shape[1]
        qp, kp = qp.contiguous(), kp.contiguous()
    rows = BH * nqb
    kv_idx = torch.full((rows, nkb), -1, dtype=torch.int32)
    kv_cnt = torch.empty(rows, dtype=torch.int32)
    mask = torch.empty(rows, nkb, dtype=torch.uint8)
    scores = torch.empty(rows, nkb, dtype=torch.float32)
    loc = None if local is None else local.to(torch.uint8).contiguous()
    lib().oracle_block_topk(_p(qp), _p(kp), _p(scores_in), BH, nqb, nkb, D, topk, n_text, _p(loc),
                            _p(kv_idx), nkb, _p(kv_cnt), _p(mask), _p(scores))
    return kv_idx, kv_cnt, mask, scores


def energy_list(scores, mode: int, threshold: float = 0.95, min_keep: int = 1, max_keep: int = 1 << 30,
                init_k: int = 1, n_text: int = 4):
    """scores fp32 [BH, nqb, nkb] -> (kv_idx [rows, nkb], kv_cnt [rows], mask uint8 [rows, nkb])."""
    BH, nqb, nkb = scores.shape
    scores = scores.contiguous().float()
    rows = BH * nqb
    kv_idx = torch.full((rows, nkb), -1, dtype=torch.int32)
    kv_cnt = torch.empty(rows, dtype=torch.int32)
    mask = torch.empty(rows, nkb, dtype=torch.uint8)
    lib().oracle_energy_list(_p(scores), BH, nqb, nkb, mode, threshold, min_keep, max_keep, init_k, n_text,
                             _p(kv_idx), nkb, _p(kv_cnt), _p(mask))
    return kv_idx, kv_cnt, mask


def local_window(geom, dt: int, dh: int, dw: int) -> torch.Tensor:
    """uint8 [nb, nb] local-window bitmap of a Geometry (text_len, T, Hp, Wp, block)."""
    nb = -(-geom.L // geom.block)
    out = torch.empty(nb, nb, dtype=torch.uint8)
    lib().oracle_local_window(geom.L, geom.block, geom.text_len, geom.T, geom.Hp, geom.Wp, dt, dh, dw, _p(out))
    return out


def tome_partition(T, Hp, Wp, sx, sy, st, choice=None):
    """(a_idx, b_idx) int32 tensors of the video-token partition."""
    N = T * Hp * Wp
    a = torch.empty(N, dtype=torch.int32)
    b = torch.empty(N, dtype=torch.int32)
    ns, nd = ctypes.c_int(0), ctypes.c_int(0)
    ch = None if choice is None else choice.to(torch.int32).contiguous()
    lib().oracle_tome_partition(T, Hp, Wp, sx, sy, st, _p(ch), _p(a), _p(b), ctypes.byref(ns), ctypes.byref(nd))
    return a[: ns.value].clone(), b[: nd.value].clone()


def tome_metric(k, v, text_len: int, mode: int) -> torch.Tensor:
    B, H, L, D = k.shape
    k = k.contiguous()
    v = v.contiguous() if v is not None else k
    N = L - text_len
    out = torch.empty((B, N, 64) if mode == 0 else (B * H, N, 130), dtype=torch.float32)
    lib().oracle_tome_metric(_p(k.view(torch.int16)), _p(v.view(torch.int16)), k.stride(0), k.stride(1), k.stride(2),
                             B, H, L, text_len, mode, _p(out))
    return out


def tome_match(metric, a_idx, b_idx, r: int, text_len: int):
    """Returns a dict of the maps (node_idx, node_max, edge, dst_idx, dst_cnt, row_of_token, key_bias)."""
    G, N, C = metric.shape
    ns, nd = a_idx.numel(), b_idx.numel()
    L = text_len + N
    out = dict(node_idx=torch.empty(G, ns, dtype=torch.int32), node_max=torch.empty(G, ns),
               edge=torch.empty(G, ns, dtype=torch.int32), dst_idx=torch.empty(G, max(r, 1), dtype=torch.int32),
               dst_cnt=torch.empty(G, nd, dtype=torch.int32), row_of_token=torch.empty(G, L, dtype=torch.int32),
               key_bias=torch.empty(G, L - r))
    lib().oracle_tome_match(_p(metric.contiguous()), G, N, C, _p(a_idx), _p(b_idx), ns, nd, r, text_len,
                            _p(out["node_idx"]), _p(out["node_max"]), _p(out["edge"]), _p(out["dst_idx"]),
                            _p(out["dst_cnt"]), _p(out["row_of_token"]), _p(out["key_bias"]))
    out["dst_idx"] = out["dst_idx"][:, :r]
    return out


def tome_merge(x, maps, a_idx, b_idx, r: int, text_len: int, heads_per_group: int) -> torch.Tensor:
    B, H, L, D = x.shape
    x = x.contiguous()
    N = L - text_len
    out = torch.empty(B, H, L - r, D, dtype=torch.bfloat16)
    dst = maps["dst_idx"].contiguous() if r > 0 else torch.zeros(1, 1, dtype=torch.int32)
    lib().oracle_tome_merge(_p(x.view(torch.int16)), x.stride(0), x.stride(1), x.stride(2), B, H, heads_per_group, N,
                            text_len, _p(a_idx), _p(b_idx), a_idx.numel(), b_idx.numel(), r, _p(maps["edge"]),
                            _p(dst), _p(out.view(torch.int16)))
    return out


def tome_unmerge(xm, maps, heads_per_group: int) -> torch.Tensor:
    B, H, Lm, D = xm.shape
    rot = maps["row_of_token"].long()
    g = torch.arange(B * H) // heads_per_group
    idx = rot[g].reshape(B, H, -1)
    return torch.gather(xm, 2, idx[..., None].expand(B, H, idx.shape[-1], D))


def tome_argmax(metric, a_subset, b_idx):
    """(node_idx, node_max) [G, len(a_subset)] for a subset of the srcs."""
    G, N, C = metric.shape
    n = a_subset.numel()
    idx = torch.empty(G, n, dtype=torch.int32)
    mx = torch.empty(G, n)
    lib().oracle_tome_argmax(_p(metric.contiguous()), G, N, C, _p(a_subset.contiguous()), n, _p(b_idx), b_idx.numel(),
                             _p(idx), _p(mx))
    return idx, mx


def tome_argmax_all(metric, a_idx, b_idx, threads: int = 0):
    """(node_idx, node_max) [G, n_src] for every src: `oracle_tome_argmax` on contiguous
    slices of the srcs in a thread pool (ctypes releases the GIL during the call; every src
    is computed independently, so the result does not depend on the split)."""
    from concurrent.futures import ThreadPoolExecutor

    lib()  # load once, before the threads call it
    G = metric.shape[0]
    n = a_idx.numel()
    metric = metric.contiguous()
    b_idx = b_idx.contiguous()
    nt = max(1, min(threads or (os.cpu_count() or 1), 32))
    bounds = [n * i // nt for i in range(nt + 1)]
    parts = [(bounds[i], bounds[i + 1]) for i in range(nt) if bounds[i + 1] > bounds[i]]
    with ThreadPoolExecutor(len(parts)) as ex:
        res = list(ex.map(lambda p: tome_argmax(metric, a_idx[p[0]:p[1]].contiguous(), b_idx), parts))
    idx = torch.cat([r[0] for r in res], dim=1) if res else torch.empty(G, 0, dtype=torch.int32)
    mx = torch.cat([r[1] for r in res], dim=1) if res else torch.empty(G, 0)
    return idx, mx


def tome_maps(node_max, node_idx, N, a_idx, b_idx, r: int, text_len: int):
    """Maps from given node_max/node_idx [G, n_src] (same dict as tome_match)."""
    G = node_max.shape[0]
    ns, nd = a_idx.numel(), b_idx.numel()
    L = text_len + N
    out = dict(node_idx=node_idx.contiguous(), node_max=node_max.contiguous(),
               edge=torch.empty(G, ns, dtype=torch.int32), dst_idx=torch.empty(G, max(r, 1), dtype=torch.int32),
               dst_cnt=torch.empty(G, nd, dtype=torch.int32), row_of_token=torch.empty(G, L, dtype=torch.int32),
               key_bias=torch.empty(G, L - r))
    lib().oracle_tome_maps(_p(out["node_max"]), _p(out["node_idx"]), G, N, _p(a_idx), _p(b_idx), ns, nd, r, text_len,
                           _p(out["edge"]), _p(out["dst_idx"]), _p(out["dst_cnt"]), _p(out["row_of_token"]),
                           _p(out["key_bias"]))
    out["dst_idx"] = out["dst_idx"][:, :r]
    return out
