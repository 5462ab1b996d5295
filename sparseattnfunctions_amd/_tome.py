"""Token merging on the GPU: partition, metric, matching maps, merge and unmerge.

Thin host layer over the `sa_tome_*` entry points of libsa_hip.so. All per-call buffers are
allocated here with PyTorch (device memory) and described to the library by a
`sa_tome_maps` struct of plain pointers.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

_I = ctypes.c_int
_P = ctypes.c_void_p


class _MapsStruct(ctypes.Structure):
    _fields_ = [(n, _I) for n in ("G", "N", "text_len", "n_src", "n_dst", "r", "L", "Lm")] + [
        (n, _P)
        for n in ("a_idx", "b_idx", "node_idx", "node_max", "rank", "edge", "dst_idx", "dst_cnt", "dst_cursor",
                  "dst_ptr", "members", "row_of_token", "key_bias", "merged_src", "member_rows")
    ]


_PART_CACHE = {}


def partition(T: int, Hp: int, Wp: int, sx: int, sy: int, st: int, device, cell_choice=None):
    """(a_idx, b_idx) int32 device tensors of the src/dst split (`sa_tome_partition`).
    Cached per geometry when `cell_choice` is None (the deterministic top-left rule)."""
    key = (T, Hp, Wp, sx, sy, st, str(device))
    if cell_choice is None and key in _PART_CACHE:
        return _PART_CACHE[key]
    lib = _lib.load()
    ns, nd = ctypes.c_int(0), ctypes.c_int(0)
    choice = None if cell_choice is None else cell_choice.to(device="cpu", dtype=torch.int32).contiguous()
    cptr = None if choice is None else choice.data_ptr()
    _lib.check(lib.sa_tome_partition(T, Hp, Wp, sx, sy, st, cptr, None, None, ctypes.byref(ns), ctypes.byref(nd)),
               "sa_tome_partition")
    a = torch.empty(max(ns.value, 1), dtype=torch.int32)
    b = torch.empty(nd.value, dtype=torch.int32)
    _lib.check(lib.sa_tome_partition(T, Hp, Wp, sx, sy, st, cptr, a.data_ptr(), b.data_ptr(), ctypes.byref(ns),
                                     ctypes.byref(nd)), "sa_tome_partition")
    out = (a[: ns.value].to(device), b.to(device))
    if cell_choice is None:
        _PART_CACHE[key] = out
    return out


def _bf16(t):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"expected bfloat16, got {t.dtype}")
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def metric_from_qkv(k, v=None, text_len: int = 226, mode: int = 0) -> torch.Tensor:
    """Normalised matching metric of the video tokens: mode 0 head-sum of k -> [B, N, 64];
    mode 1 per-head (k, |k|, v, |v|) -> [B*H, N, 130] (`sa_tome_metric`)."""
    _lib.require_gpu(k, v)
    k = _bf16(k)
    v = _bf16(v) if v is not None else None
    B, H, L, D = k.shape
    N = L - text_len
    out = torch.empty((B, N, 64) if mode == 0 else (B * H, N, 130), dtype=torch.float32, device=k.device)
    with torch.cuda.device(k.device):
        rc = _lib.load().sa_tome_metric(k.data_ptr(), _lib.i64(*k.stride()[:3]), _lib.ptr(v),
                                        _lib.i64(*v.stride()[:3]) if v is not None else None, B, H, L, D, text_len,
                                        mode, out.data_ptr(), _lib.stream_of(k))
    _lib.check(rc, "sa_tome_metric")
    return out


def normalize(metric: torch.Tensor) -> torch.Tensor:
    """Row-wise L2 normalisation of a [G, N, C] metric in fp32 (`sa_tome_normalize`)."""
    _lib.require_gpu(metric)
    x = metric.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    rows = x.numel() // x.shape[-1]
    with torch.cuda.device(x.device):
        rc = _lib.load().sa_tome_normalize(x.data_ptr(), rows, x.shape[-1], out.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "sa_tome_normalize")
    return out


class TomeMaps:
    """Device buffers of one matching (see sa_tome_maps in include/sa_api.h)."""

    def __init__(self, G, N, text_len, a_idx, b_idx, r, device):
        ns, nd = a_idx.numel(), b_idx.numel()
        L = text_len + N
        self.G, self.N, self.text_len, self.n_src, self.n_dst, self.r, self.L, self.Lm = G, N, text_len, ns, nd, r, L, L - r
        self.a_idx, self.b_idx = a_idx, b_idx
        i32 = dict(dtype=torch.int32, device=device)
        self.node_idx = torch.empty(G, max(ns, 1), **i32)
        self.node_max = torch.empty(G, max(ns, 1), dtype=torch.float32, device=device)
        self.rank = torch.empty(G, max(ns, 1), **i32)
        self.edge = torch.empty(G, max(ns, 1), **i32)
        self.dst_idx = torch.empty(G, max(r, 1), **i32)
        self.dst_cnt = torch.empty(G, nd, **i32)
        self.dst_cursor = torch.empty(G, nd, **i32)
        self.dst_ptr = torch.empty(G, nd + 1, **i32)
        self.members = torch.empty(G, max(r, 1), **i32)
        self.row_of_token = torch.empty(G, L, **i32)
        self.key_bias = torch.empty(G, L - r, dtype=torch.float32, device=device)
        self.merged_src = torch.empty(G, L - r, **i32)
        self.member_rows = torch.empty(G, max(r, 1), **i32)
        self.struct = _MapsStruct(G, N, text_len, ns, nd, r, L, L - r, *[
            t.data_ptr() for t in (a_idx, b_idx, self.node_idx, self.node_max, self.rank, self.edge, self.dst_idx,
                                   self.dst_cnt, self.dst_cursor, self.dst_ptr, self.members, self.row_of_token,
                                   self.key_bias, self.merged_src, self.member_rows)])

    @property
    def sizes(self) -> torch.Tensor:
        """[G, n_dst] token count of each dst after merging (the reference's `counter`)."""
        return 1 + self.dst_cnt


def match(metric: torch.Tensor, a_idx: torch.Tensor, b_idx: torch.Tensor, r: int, text_len: int) -> TomeMaps:
    """Bipartite matching of a normalised metric [G, N, C] and all merge/unmerge maps."""
    _lib.require_gpu(metric, a_idx, b_idx)
    G, N, C = metric.shape
    r = max(0, min(int(r), a_idx.numel()))
    maps = TomeMaps(G, N, text_len, a_idx, b_idx, r, metric.device)
    lib = _lib.load()
    ws_bytes = ctypes.c_int64(0)
    _lib.check(lib.sa_tome_match_workspace(G, a_idx.numel(), b_idx.numel(), ctypes.byref(ws_bytes)),
               "sa_tome_match_workspace")
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=metric.device)
    metric = metric.contiguous()
    with torch.cuda.device(metric.device):
        rc = lib.sa_tome_match(metric.data_ptr(), C, ctypes.byref(maps.struct), ws.data_ptr(), ws.numel(),
                               _lib.stream_of(metric))
    _lib.check(rc, "sa_tome_match")
    maps._ws = ws  # keep the workspace alive until the stream has used it
    return maps


# Device index -> event recorded on the stream of the last sa_tome_match_noalloc call.
_NOALLOC_LAST = {}


def match_noalloc(metric: torch.Tensor, a_idx: torch.Tensor, b_idx: torch.Tensor, r: int, text_len: int) -> TomeMaps:
    """match() through `sa_tome_match_noalloc`: the library allocates nothing and no workspace
    is passed (its partials live in a fixed 16 MiB device array per GPU; larger problems raise
    ValueError). The maps themselves are caller buffers, allocated here.

    Calls on one GPU share that array, so their kernels must not overlap. Calls from this
    function are ordered: each call's stream waits for an event recorded after the previous
    call on the same GPU (whatever its stream). Under graph capture no event is waited for or
    recorded (the capture's own stream order applies)."""
    _lib.require_gpu(metric, a_idx, b_idx)
    G, N, C = metric.shape
    r = max(0, min(int(r), a_idx.numel()))
    maps = TomeMaps(G, N, text_len, a_idx, b_idx, r, metric.device)
    metric = metric.contiguous()
    dev = metric.device
    stream = torch.cuda.current_stream(dev)
    capturing = torch.cuda.is_current_stream_capturing()
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    prev = _NOALLOC_LAST.get(key)
    if prev is not None and not capturing:
        stream.wait_event(prev)
    with torch.cuda.device(dev):
        rc = _lib.load().sa_tome_match_noalloc(metric.data_ptr(), C, ctypes.byref(maps.struct), stream.cuda_stream)
    _lib.check(rc, "sa_tome_match_noalloc")
    if not capturing:
        ev = torch.cuda.Event()
        ev.record(stream)
        _NOALLOC_LAST[key] = ev
    return maps


def _apply(fn_name, x, maps: TomeMaps, heads_per_group: int, rows_out: int, out: Optional[torch.Tensor]):
    _lib.require_gpu(x)
    x = _bf16(x)
    B, H, _, D = x.shape
    if out is None:
        out = torch.empty(B, H, rows_out, D, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        rc = getattr(_lib.load(), fn_name)(x.data_ptr(), _lib.i64(*x.stride()[:3]), B, H, D, heads_per_group,
                                           ctypes.byref(maps.struct), out.data_ptr(), _lib.i64(*out.stride()[:3]),
                                           _lib.stream_of(x))
    _lib.check(rc, fn_name)
    return out


def merge(x: torch.Tensor, maps: TomeMaps, heads_per_group: int, out=None) -> torch.Tensor:
    """[B, H, L, 64] -> [B, H, Lm, 64]: [text | unm | dst means] (`sa_tome_merge`)."""
    if x.shape[2] != maps.L:
        raise ValueError(f"merge: tensor has {x.shape[2]} tokens, maps expect {maps.L}")
    return _apply("sa_tome_merge", x, maps, heads_per_group, maps.Lm, out)


def merge_many(xs, maps: TomeMaps, heads_per_group: int):
    """merge() of up to three [B, H, L, 64] tensors with one set of maps in one launch
    (`sa_tome_merge_multi`); returns the merged tensors in order."""
    xs = [_bf16(x) for x in xs]
    if not 1 <= len(xs) <= 3:
        raise ValueError("merge_many takes 1 to 3 tensors")
    _lib.require_gpu(*xs)
    B, H, L, D = xs[0].shape
    for x in xs:
        if tuple(x.shape) != (B, H, L, D) or x.device != xs[0].device:
            raise ValueError("merge_many: tensors must share shape and device")
    if L != maps.L:
        raise ValueError(f"merge: tensor has {L} tokens, maps expect {maps.L}")
    outs = [torch.empty(B, H, maps.Lm, D, dtype=x.dtype, device=x.device) for x in xs]
    n = len(xs)
    xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs])
    op = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    xst = _lib.i64(*[s for x in xs for s in x.stride()[:3]])
    ost = _lib.i64(*[s for o in outs for s in o.stride()[:3]])
    with torch.cuda.device(xs[0].device):
        rc = _lib.load().sa_tome_merge_multi(n, xp, xst, B, H, D, heads_per_group, ctypes.byref(maps.struct), op, ost,
                                             _lib.stream_of(xs[0]))
    _lib.check(rc, "sa_tome_merge_multi")
    return outs


def unmerge(xm: torch.Tensor, maps: TomeMaps, heads_per_group: int, out=None) -> torch.Tensor:
    """[B, H, Lm, 64] -> [B, H, L, 64]: every token reads its merged row (`sa_tome_unmerge`)."""
    if xm.shape[2] != maps.Lm:
        raise ValueError(f"unmerge: tensor has {xm.shape[2]} rows, maps expect {maps.Lm}")
    return _apply("sa_tome_unmerge", xm, maps, heads_per_group, maps.L, out)
