"""GPU parity of attn_with_pooling (utils/attn_pooling_kernel.py) against the fp64 oracle.

Tolerances: out max-abs <= 2e-2 and mean-abs <= 2e-3 (the attention bar); Po relative 5e-3
(+1e-7 absolute): its entries are exp2 of fp32 logits minus the row's log-sum-exp, whose
row sum accumulates bf16-rounded probabilities.
At the C2 shape, size-independent properties: out is bit-identical to the block-sparse kernel (bf16 scores)
over every block (the pooling mode only adds stores), Po rows sum to one, causal Po is zero
above the diagonal.
"""
import math

import pytest
import torch

from conftest import case
from oracle.pooling import pooled_attention
from sparseattnfunctions_amd.utils.attn_pooling_kernel import attn_with_pooling

pytestmark = pytest.mark.gpu


def _qkv(seed, B, H, Hk, L, scale=1.0, D=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, L, D, generator=g) * scale).to(dtype)
    k = (torch.randn(B, Hk, L, D, generator=g) * scale).to(dtype)
    v = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Hk", [4, 2])
def test_pooled_attention_matches_oracle(dev, bs, causal, Hk):
    case(f"attn_with_pooling bs={bs} causal={causal} Hk={Hk}")
    q, k, v = _qkv(bs + 7 * Hk + causal, 1, 4, Hk, 1000, scale=1.5)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, 0.125, bs)
    want_o, want_po = pooled_attention(q, k, v, causal, 0.125, bs)
    err = (o.cpu().double() - want_o).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (err.max().item(), err.mean().item())
    assert po.shape == want_po.shape and po.dtype == torch.float32
    assert torch.allclose(po.cpu().double(), want_po, rtol=5e-3, atol=1e-7), (po.cpu().double() - want_po).abs().max()
    if causal:
        nd = po.shape[-1]
        assert torch.equal(po.cpu()[..., torch.ones(nd, nd, dtype=torch.bool).triu(1)],
                           torch.zeros_like(po.cpu()[..., torch.ones(nd, nd, dtype=torch.bool).triu(1)]))


@pytest.mark.parametrize("L", [40, 70, 130])
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_pooled_attention_short_sequences(dev, L, bs, causal):
    # fewer tokens than one or two blocks: partial last key and query blocks in every mode
    case(f"attn_with_pooling L={L} bs={bs} causal={causal}")
    q, k, v = _qkv(L + bs + causal, 1, 2, 1, L)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, 0.125, bs)
    want_o, want_po = pooled_attention(q, k, v, causal, 0.125, bs)
    assert (o.cpu().double() - want_o).abs().max().item() <= 2e-2
    assert torch.allclose(po.cpu().double(), want_po, rtol=5e-3, atol=1e-7)


@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_pooled_attention_several_column_chunks(dev, bs, causal):
    # L = 2200: Po rows of 35 (bs 64) or 69 (bs 32) columns, so the attention kernel's Po
    # epilogue runs over two or three 32-column chunks, including a partial last one.
    case(f"attn_with_pooling L=2200 bs={bs} causal={causal}")
    q, k, v = _qkv(2200 + bs + causal, 1, 1, 1, 2200)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, 0.125, bs)
    want_o, want_po = pooled_attention(q, k, v, causal, 0.125, bs)
    assert (o.cpu().double() - want_o).abs().max().item() <= 2e-2
    assert torch.allclose(po.cpu().double(), want_po, rtol=5e-3, atol=1e-7), (po.cpu().double() - want_po).abs().max()


def test_pooled_attention_large_scores(dev):
    # scores of several hundred: the kernel's safe pass; Po must not depend on it
    case("attn_with_pooling large scores")
    q, k, v = _qkv(21, 1, 2, 2, 640, scale=6.0)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), False, 0.125, 64)
    want_o, want_po = pooled_attention(q, k, v, False, 0.125, 64)
    assert (o.cpu().double() - want_o).abs().max().item() <= 2e-2
    assert torch.allclose(po.cpu().double(), want_po, rtol=5e-3, atol=1e-7)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128), (torch.float16, 128)])
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_pooled_attention_fp16_and_head_dim_128(dev, dtype, D, bs, causal):
    # The reference takes fp16 as well as bf16, and any head dim of 16..256 (:252). Po comes
    # back in the dtype the reference returns: fp16 for fp16 inputs, fp32 for bf16 ones. fp16
    # Po adds one fp16 rounding (relative 2^-11; entries under 2^-14 are fp16 subnormals,
    # absolute 2^-25).
    case(f"attn_with_pooling dtype={dtype} D={D} bs={bs} causal={causal}")
    q, k, v = _qkv(D + bs + causal, 1, 4, 2, 300, scale=1.5, D=D, dtype=dtype)
    scale = 1 / math.sqrt(D)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, scale, bs)
    want_o, want_po = pooled_attention(q, k, v, causal, scale, bs)
    assert o.dtype == dtype and o.shape == q.shape
    assert po.dtype == (torch.float16 if dtype == torch.float16 else torch.float32)
    err = (o.cpu().double() - want_o).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (err.max().item(), err.mean().item())
    assert torch.allclose(po.cpu().double(), want_po, rtol=6e-3, atol=1e-7), (po.cpu().double() - want_po).abs().max()


# fp32 arithmetic, as the reference computes attn_with_pooling (bf16 inputs cast to fp32,
# :235-240): fp32 inputs always, 16-bit inputs with precision="fp32". The bar is fp32
# accuracy against the fp64 oracle on the same inputs: out max-abs 2e-5 / mean-abs 2e-6, Po
# relative 2e-5 (+1e-9 absolute).
F32_MAX, F32_MEAN = 2e-5, 2e-6


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D,Hk", [(64, 4), (64, 2), (128, 2)])
def test_pooled_attention_fp32(dev, bs, causal, D, Hk):
    case(f"attn_with_pooling fp32 bs={bs} causal={causal} D={D} Hk={Hk}")
    q, k, v = _qkv(bs + 3 * Hk + causal + D, 1, 4, Hk, 600, scale=1.5, D=D, dtype=torch.float32)
    scale = 1 / math.sqrt(D)
    o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, scale, bs)
    assert o.dtype == torch.float32 and po.dtype == torch.float32
    want_o, want_po = pooled_attention(q, k, v, causal, scale, bs)
    err = (o.cpu().double() - want_o).abs()
    assert err.max().item() <= F32_MAX and err.mean().item() <= F32_MEAN, (err.max().item(), err.mean().item())
    assert po.shape == want_po.shape
    assert torch.allclose(po.cpu().double(), want_po, rtol=2e-5, atol=1e-9), (po.cpu().double() - want_po).abs().max()
    if causal:
        nd = po.shape[-1]
        up = torch.ones(nd, nd, dtype=torch.bool).triu(1)
        assert torch.all(po.cpu()[..., up] == 0)


@pytest.mark.parametrize("L", [40, 130])
def test_pooled_attention_fp32_short(dev, L):
    case(f"attn_with_pooling fp32 L={L}")
    q, k, v = _qkv(L, 2, 2, 2, L, dtype=torch.float32)
    for bs in (32, 64, 128):
        for causal in (False, True):
            o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, 0.125, bs)
            want_o, want_po = pooled_attention(q, k, v, causal, 0.125, bs)
            assert (o.cpu().double() - want_o).abs().max().item() <= F32_MAX
            assert torch.allclose(po.cpu().double(), want_po, rtol=2e-5, atol=1e-9)


def test_pooled_attention_bf16_in_fp32_arithmetic(dev):
    # precision="fp32": bf16 inputs computed as the reference computes them (cast to fp32);
    # Po at the fp32 bar against the oracle on the bf16 values, out rounded once to bf16.
    case("attn_with_pooling bf16 inputs, precision fp32")
    q, k, v = _qkv(77, 1, 4, 2, 900, scale=1.5)
    for bs, causal in ((64, False), (128, True), (32, True)):
        o, po = attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), causal, 0.125, bs, precision="fp32")
        assert o.dtype == torch.bfloat16 and po.dtype == torch.float32
        want_o, want_po = pooled_attention(q, k, v, causal, 0.125, bs)
        assert torch.allclose(po.cpu().double(), want_po, rtol=2e-5, atol=1e-9)
        # the only rounding of out is the final one to bf16: within half a bf16 ulp of the oracle
        # (plus the fp32 bar), and equal to the fp32 result of the same inputs rounded once
        err = (o.cpu().double() - want_o).abs()
        assert torch.all(err <= want_o.abs() * 2.0 ** -8 + 2e-5)
        o32, _ = attn_with_pooling(q.float().to(dev), k.float().to(dev), v.float().to(dev), causal, 0.125, bs)
        assert torch.equal(o, o32.to(torch.bfloat16))
    with pytest.raises(ValueError):
        attn_with_pooling(q.to(dev), k.to(dev), v.to(dev), False, 0.125, 64, precision="fp64")


@pytest.mark.parametrize("causal", [False, True])
def test_pooled_attention_c2_shape_properties(dev, causal):
    case(f"attn_with_pooling C2 shape causal={causal}")
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import block_sparse_attention
    from sparseattnfunctions_amd.block_mask_attn import dense_kv_list
    B, H, L = 2, 30, 17776
    gen = torch.Generator(device=dev).manual_seed(5)
    q, k, v = (torch.randn(B, H, L, 64, device=dev, generator=gen).to(torch.bfloat16) for _ in range(3))
    o, po = attn_with_pooling(q, k, v, causal, 0.125, 64)
    torch.cuda.synchronize()
    nd = math.ceil(L / 64)
    assert po.shape == (B, H, nd, nd)
    assert torch.isfinite(po).all() and (po >= 0).all()
    assert torch.allclose(po.sum(-1), torch.ones(B, H, nd, device=dev), atol=1e-5)
    if causal:
        assert (po[..., torch.ones(nd, nd, dtype=torch.bool, device=dev).triu(1)] == 0).all()
        # a few rows against torch's causal SDPA in fp32
        ref = torch.nn.functional.scaled_dot_product_attention(q[:1, :2].float(), k[:1, :2].float(),
                                                               v[:1, :2].float(), is_causal=True)
        assert (o[:1, :2].float() - ref).abs().max().item() <= 2e-2
    else:
        # the plain kernel with the bf16 scores that the pooling mode computes
        dense = block_sparse_attention(q, k, v, dense_kv_list(B, H, nd, nd, q.device), 0.125, fp16_scores=False)
        assert torch.equal(o, dense)
