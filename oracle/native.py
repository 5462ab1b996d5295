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
        L.oracle_local_window.argtypes = [_I] * 9 + [_P]
        L.oracle_local_window.restype = None
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


def local_window(geom, dt: int, dh: int, dw: int) -> torch.Tensor:
    """uint8 [nb, nb] local-window bitmap of a Geometry (text_len, T, Hp, Wp, block)."""
    nb = -(-geom.L // geom.block)
    out = torch.empty(nb, nb, dtype=torch.uint8)
    lib().oracle_local_window(geom.L, geom.block, geom.text_len, geom.T, geom.Hp, geom.Wp, dt, dh, dw, _p(out))
    return out
