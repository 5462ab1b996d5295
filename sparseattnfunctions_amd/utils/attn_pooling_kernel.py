"""`attn_with_pooling` of special_attentions/utils/attn_pooling_kernel.py (:230-289), on MI355X.

Dense (or causal) attention that also returns the 2-D max-pooled attention map
Po [B, H, nd, nd] (nd = ceil(L / block_size), block_size in {32, 64, 128}): Po[i][j] is the
largest softmax probability of query block i against key block j, each row then divided by
its sum. It is a block-score map for the mask builders, e.g.
`SparseGen_Plus.transfer_attn_to_kv_list(Po, ...)` for block_size 64.

One call runs the block-sparse attention kernel over every key block (causal: the blocks up
to the diagonal, the diagonal tile masked to keys <= query) in its pooling mode. Each query
row stores its largest scaled logit R per 32- or 64-key column to a workspace. For block
sizes 32 and 64 each wave's 64 query rows are whole Po rows, and the wave forms them after
its rows: Po = max over the block's rows of exp2(R - lse), normalised. For block size 128 the
rows' log-sum-exps are stored too, and a reduce kernel does this over two waves' rows. The
probability matrix itself is never written.

q, k and v are bf16, fp16 or fp32 (one dtype), head_dim 64 or 128. Po is fp32 for bf16 and
fp32 inputs and fp16 for fp16 inputs, the dtypes the reference returns (it computes bf16 inputs
in fp32 and fp16 inputs in fp16, storing Po in that dtype).

Arithmetic. fp32 inputs run the fp32 kernel (fp32 MFMA, P and row sums in fp32), as the
reference does. bf16 and fp16 inputs run, by default, the 16-bit kernel: bf16 (fp16) products
with fp32 accumulation and P rounded to the input dtype before P.V, where the reference casts
bf16 inputs up to fp32 first (:235-240); `attn_with_pooling(..., precision="fp32")` does what
the reference does (inputs cast to fp32, the fp32 kernel, the output cast back to the input
dtype), at the fp32 MFMA rate (1/16 of bf16's). The rows of a last, partial query block that
lie past L take no part in its maximum; the reference reads them without bounds checks.
"""
from __future__ import annotations

import ctypes
import math

import torch

from .. import _lib
from .block_sparse_attn_kernel import _prep_qkv


class _attention_pooling(torch.autograd.Function):
    """forward(ctx, q, k, v, causal, sm_scale, block_size) -> (o, Po), as the reference
    (:230-287); like the reference it has no backward."""

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale, block_size, precision=None):
        assert block_size in {32, 64, 128}
        if precision not in (None, "fp32"):
            raise ValueError(f"precision must be None or 'fp32', got {precision!r}")
        types = (torch.bfloat16, torch.float16, torch.float32)
        q, k, v = _prep_qkv(q, types), _prep_qkv(k, types), _prep_qkv(v, types)
        if not q.dtype == k.dtype == v.dtype:
            raise TypeError(f"q, k, v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
        orig_dtype = q.dtype
        if precision == "fp32" and q.dtype != torch.float32:
            q, k, v = q.float(), k.float(), v.float()
        fp16 = q.dtype == torch.float16
        fp32 = q.dtype == torch.float32
        _lib.require_gpu(q, k, v)
        B, H, L, D = q.shape
        Hk = k.shape[1]
        assert k.shape[-1] == D and v.shape[-1] == D
        assert k.shape[1] == v.shape[1]
        if k.shape[0] != B or v.shape[0] != B or k.shape[2] != L or v.shape[2] != L:
            raise ValueError(f"k, v must be [B, H_kv, {L}, {D}], got {tuple(k.shape)}, {tuple(v.shape)}")
        nd = math.ceil(L / block_size)
        o = torch.empty_like(q)
        po = torch.empty(B, H, nd, nd, dtype=torch.float32, device=q.device)
        lib = _lib.load()
        ws_bytes = ctypes.c_int64(0)
        _lib.check(lib.sa_attn_pooling_workspace(B, H, L, block_size, ctypes.byref(ws_bytes)),
                   "sa_attn_pooling_workspace")
        ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=q.device)
        fn = "sa_attn_pooling_fwd_f16" if fp16 else ("sa_attn_pooling_fwd_f32" if fp32 else "sa_attn_pooling_fwd")
        with torch.cuda.device(q.device):
            _lib.check(getattr(lib, fn)(
                q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
                v.data_ptr(), _lib.i64(*v.stride()[:3]), o.data_ptr(), _lib.i64(*o.stride()[:3]),
                B, H, Hk, L, D, 1 if causal else 0, float(sm_scale), block_size, po.data_ptr(),
                _lib.i64(*po.stride()[:3]), ws.data_ptr(), ws.numel(), _lib.stream_of(q)), fn)
        return o.to(orig_dtype), (po.to(torch.float16) if fp16 else po)


def attn_with_pooling(q, k, v, causal, sm_scale, block_size, precision=None):
    """(o, Po) as the reference's `attn_with_pooling = _attention_pooling.apply` (:289); the
    optional `precision="fp32"` computes 16-bit inputs in fp32 as the reference does."""
    return _attention_pooling.apply(q, k, v, causal, sm_scale, block_size, precision)


def is_hip() -> bool:
    """The reference's backend probe (Triton's active target is "hip" on ROCm): this build runs
    on HIP only."""
    return True
