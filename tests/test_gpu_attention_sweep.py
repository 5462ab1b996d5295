"""Randomised parity sweep of the block-sparse attention entry points against the fp64 oracle.

Each seed draws a shape (B, H, Lq, Lk with partial tiles, head dim 64 or 128), a dtype (bf16
or fp16), a block density (down to lists with empty rows), an optional key bias, an optional
32-value-column launch and a score amplitude that sometimes pushes rows off the unshifted
exp2 pass. Long key ranges with few query blocks take the key-range split. The bar is the
attention bar of test_gpu_attention.py (max-abs 2e-2, mean-abs 2e-3 and the reference's
allclose(1e-2, 1e-2) against the oracle on the same 16-bit inputs).
"""
import math
import random

import pytest
import torch

from conftest import case
from oracle.attention import masked_attention
from sparseattnfunctions_amd._kv import kv_list_from_mask
from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import block_sparse_attention

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _draw(seed):
    rng = random.Random(seed)
    B, H = rng.choice([1, 2]), rng.choice([1, 2, 3])
    D = rng.choice([64, 64, 128])
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    Lk = rng.randint(4033, 6000) if rng.random() < 0.4 else rng.randint(1, 1500)
    Lq = rng.randint(1, max(1, min(900, 4_000_000 // (B * H * Lk))))
    density = rng.choice([0.05, 0.3, 0.7, 1.0])
    bias = rng.random() < 0.3
    v32 = dtype == torch.bfloat16 and D == 64 and rng.random() < 0.3
    amp = rng.choice([1.0, 1.0, 4.0])
    return B, H, Lq, Lk, D, dtype, density, bias, v32, amp


def _parts(n_items, max_cnt, D):
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import split_parts
    return split_parts(n_items, max_cnt, D)


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_against_oracle(dev, seed):
    B, H, Lq, Lk, D, dtype, density, bias, v32, amp = _draw(seed)
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    split = not bias and not v32 and _parts(B * H * nqb, nkb, D) > 1
    case(f"seed={seed} B={B} H={H} Lq={Lq} Lk={Lk} D={D} {dtype} density={density} bias={bias} v32={v32} "
         f"amp={amp} split={split}")
    g = torch.Generator().manual_seed(1000 + seed)
    q = (torch.randn(B, H, Lq, D, generator=g) * amp).to(dtype)
    k = (torch.randn(B, H, Lk, D, generator=g) * amp).to(dtype)
    v = torch.randn(B, H, Lk, D, generator=g).to(dtype)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < density
    key_bias = torch.log(torch.randint(1, 6, (B, 1, Lk), generator=g).float()) if bias else None
    scale = 1 / math.sqrt(D)
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, scale,
                                 key_bias=None if key_bias is None else key_bias.to(dev),
                                 v_cols=32 if v32 else None)
    torch.cuda.synchronize()
    assert out.shape == (B, H, Lq, 32 if v32 else D)
    want = masked_attention(q, k, v, mask, scale, key_bias=None if key_bias is None else key_bias.double())
    if v32:
        want = want[..., :32]
    got = out.float().cpu().double()
    assert torch.isfinite(got).all()
    err = (got - want).abs()
    assert err.max().item() <= MAX_ABS, err.max().item()
    assert err.mean().item() <= MEAN_ABS, err.mean().item()
    assert torch.allclose(got, want, atol=1e-2, rtol=1e-2)
    empty = ~mask.any(-1)  # query blocks with an empty list write 0
    for b, h, m in empty.nonzero().tolist():
        assert torch.all(got[b, h, 64 * m: 64 * (m + 1)] == 0)
