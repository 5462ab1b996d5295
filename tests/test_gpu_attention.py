"""GPU parity of the block-sparse attention kernel against the CPU oracle (fp64).

Tolerances: max-abs <= 2e-2 and mean-abs <= 2e-3 against the oracle
computed from the same bf16 inputs; the reference's own check, allclose(atol=1e-2,
rtol=1e-2) (block_sparse_attn_kernel.py:337), is asserted as well.
"""
import math

import pytest
import torch

from conftest import case
from oracle.attention import masked_attention
from sparseattnfunctions_amd._kv import KVList, kv_list_from_mask
from sparseattnfunctions_amd.block_mask_attn import dense_kv_list
from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import (
    block_sparse_attention, block_sparse_triton_fn, sparse_attention_factory)
from sparseattnfunctions_amd.workloads import config1_inputs

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _rand(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _check(got, want, atol_ref=True):
    got = got.float().cpu().double()
    err = (got - want).abs()
    assert torch.isfinite(got).all()
    assert err.max().item() <= MAX_ABS, err.max().item()
    assert err.mean().item() <= MEAN_ABS, err.mean().item()
    if atol_ref:
        assert torch.allclose(got, want, atol=1e-2, rtol=1e-2)


def test_config1_parity(dev):
    case("config1 B=1 H=2 L=2048 random block mask (seed 1)")
    q, k, v, mask, scale = config1_inputs()
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    out = block_sparse_triton_fn(qb.to(dev), kb.to(dev), vb.to(dev), mask.to(dev), scale)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    _check(out, masked_attention(qb, kb, vb, mask, scale))


@pytest.mark.parametrize("seed", [0, 1])
def test_reference_test_topk_partial_block(dev, seed):
    # block_sparse_attn_kernel.py:296-339: B=1, H=3, L=257 (partial last block), all-ones mask.
    case(f"L=257 all-ones seed={seed}")
    q, k, v = (_rand((1, 3, 257, 64), seed * 3 + i) for i in range(3))
    mask = torch.ones(1, 3, 5, 5, dtype=torch.bool)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 1 / 8)
    _check(out, masked_attention(q, k, v, mask, 1 / 8))


def test_reference_test_q_shorter_than_k(dev):
    # block_sparse_attn_kernel.py:343-390: Lq=128 < Lk=256, top-1 mask with column 0 forced.
    case("Lq=128 Lk=256 top-1")
    q, k, v = _rand((2, 4, 128, 64), 10), _rand((2, 4, 256, 64), 11), _rand((2, 4, 256, 64), 12)
    scores = _rand((2, 4, 4, 4), 13, torch.float32)
    scores[..., 0] = 100
    mask = torch.zeros(2, 4, 4, 4, dtype=torch.bool)
    mask.scatter_(-1, scores.topk(1, dim=-1).indices, True)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 1 / 8)
    _check(out, masked_attention(q, k, v, mask, 1 / 8))


@pytest.mark.parametrize("L,density,seed", [(64, 1.0, 0), (130, 0.5, 1), (1000, 0.3, 2), (2048, 0.1, 3)])
def test_random_masks(dev, L, density, seed):
    case(f"random mask L={L} density={density}")
    q, k, v = (_rand((2, 3, L, 64), 100 * seed + i) for i in range(3))
    nb = math.ceil(L / 64)
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand(2, 3, nb, nb, generator=g) < density
    mask[..., 0] = True
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125)
    _check(out, masked_attention(q, k, v, mask, 0.125))


def test_empty_rows_write_zero(dev):
    case("empty rows")
    q, k, v = (_rand((1, 2, 256, 64), 40 + i) for i in range(3))
    mask = torch.ones(1, 2, 4, 4, dtype=torch.bool)
    mask[0, 1, 2] = False
    mask[0, 0] = False
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125).cpu()
    assert torch.all(out[0, 0] == 0) and torch.all(out[0, 1, 128:192] == 0)
    _check(out, masked_attention(q, k, v, mask, 0.125))


@pytest.mark.parametrize("D", [64, 128])
def test_strided_and_broadcast(dev, D):
    # q/k/v as views of a [B, L, H, D] buffer (non-contiguous heads) and a [1,1,n,n] mask.
    case(f"strided BLHD views + broadcast mask D={D}")
    B, L, H = 2, 300, 4
    base = [_rand((B, L, H, D), 50 + i) for i in range(3)]
    q, k, v = (t.to(dev).permute(0, 2, 1, 3) for t in base)
    nb = math.ceil(L / 64)
    g = torch.Generator().manual_seed(5)
    mask = torch.rand(1, 1, nb, nb, generator=g) < 0.5
    mask[..., 0] = True
    out = block_sparse_triton_fn(q, k, v, mask.to(dev), 0.125)
    want = masked_attention(*(t.permute(0, 2, 1, 3) for t in base), mask, 0.125)
    _check(out, want)


@pytest.mark.parametrize("Lk", [20, 33, 57, 100, 300, 1000])
@pytest.mark.parametrize("with_bias,D", [(False, 64), (True, 64), (False, 128)])
def test_contiguous_and_strided_key_rows_agree(dev, Lk, with_bias, D):
    # Contiguous 64-element K/V rows are copied through per-tile buffer descriptors based at
    # the tile's rows 0 and 32 (sized to the head's last row; empty when row 32 is past it);
    # strided rows through per-load offsets. Same values, same arithmetic: bit-identical
    # outputs, including the partial last tile and Lk < 32 (an empty second descriptor).
    # Head dim 128 (wave pairs, each copying one 128-byte half of every row) likewise.
    case(f"contiguous vs strided K/V Lk={Lk} bias={with_bias} D={D}")
    B, H, Lq = 2, 3, 130
    q = _rand((B, H, Lq, D), 160).to(dev)
    kc, vc = _rand((B, H, Lk, D), 161).to(dev), _rand((B, H, Lk, D), 162).to(dev)
    ks = torch.empty(B, Lk, H, D, dtype=torch.bfloat16, device=dev).permute(0, 2, 1, 3)
    vs = torch.empty(B, Lk, H, D, dtype=torch.bfloat16, device=dev).permute(0, 2, 1, 3)
    ks.copy_(kc)
    vs.copy_(vc)
    assert ks.stride(2) == H * D and kc.stride(2) == D
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    g = torch.Generator().manual_seed(Lk)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.7
    mask[..., nkb - 1] = True  # the partial last tile in every row
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    bias = None
    if with_bias:
        bias = torch.log(torch.randint(1, 5, (B, H, Lk), generator=g).float()).to(dev)
    oc = block_sparse_attention(q, kc, vc, kv, 0.125, key_bias=bias)
    os_ = block_sparse_attention(q, ks, vs, kv, 0.125, key_bias=bias)
    assert torch.equal(oc, os_)
    want = masked_attention(q.cpu(), kc.cpu(), vc.cpu(), mask, 0.125,
                            key_bias=None if bias is None else bias.cpu().double())
    _check(oc, want)


def test_key_bias(dev):
    case("key bias")
    B, H, L = 2, 3, 700
    q, k, v = (_rand((B, H, L, 64), 60 + i) for i in range(3))
    g = torch.Generator().manual_seed(7)
    bias = torch.log(torch.randint(1, 6, (B, 1, L), generator=g).float())
    mask = torch.ones(1, 1, 11, 11, dtype=torch.bool)
    kv = kv_list_from_mask(mask.to(dev), B, H, 11, 11)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, key_bias=bias.to(dev))
    _check(out, masked_attention(q, k, v, mask, 0.125, key_bias=bias.double()))


def test_key_bias_short_lists(dev):
    # Lists of 0, 1, 2, 3 and all 11 blocks (random blocks, the last one partial) with a
    # per-head bias: the bias rows are copied two tiles ahead into alternating slots, and past
    # the end of a list into a slot nothing reads.
    case("key bias, lists of 0-3 and 11 blocks")
    B, H, L, nb = 1, 2, 700, 11
    q, k, v = (_rand((B, H, L, 64), 150 + i) for i in range(3))
    g = torch.Generator().manual_seed(17)
    mask = torch.zeros(B, H, nb, nb, dtype=torch.bool)
    for h in range(H):
        for r in range(nb):
            n = (0, 1, 2, 3, nb)[(r + h) % 5]
            mask[0, h, r, torch.randperm(nb, generator=g)[:n]] = True
    bias = 2 * torch.randn(B, H, L, generator=g)
    kv = kv_list_from_mask(mask.to(dev), B, H, nb, nb)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, key_bias=bias.to(dev))
    _check(out, masked_attention(q, k, v, mask, 0.125, key_bias=bias.double()))


@pytest.mark.parametrize("D", [64, 128])
def test_large_scores_redo_with_running_max(dev, D):
    # Head 0 has scores of several hundred (exp2 overflows without the max subtraction),
    # head 1 ordinary ones: the kernel must redo exactly the items whose sums left range.
    case(f"large scores on one head D={D}")
    B, H, L = 1, 2, 300
    q, k, v = (_rand((B, H, L, D), 130 + i) for i in range(3))
    q[:, 0] *= 16
    k[:, 0] *= 16
    nb = math.ceil(L / 64)
    g = torch.Generator().manual_seed(13)
    mask = torch.rand(B, H, nb, nb, generator=g) < 0.6
    mask[..., 0] = True
    scale = 1 / math.sqrt(D)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
    _check(out, masked_attention(q, k, v, mask, scale))


def test_head_dim_128_redo_when_one_half_overflows(dev):
    # At head dim 128 a query block is computed by two waves of 32 rows each. Here only rows
    # 0-31 of each block of head 0 have scores of several hundred: one wave's row sums leave
    # range, the other's do not, and the pair must redo the block together (the two waves'
    # barriers must match) and still give both halves exactly.
    case("head dim 128, large scores in rows 0-31 of each block")
    B, H, L, D = 1, 2, 320, 128
    q, k, v = (_rand((B, H, L, D), 530 + i) for i in range(3))
    rows = (torch.arange(L) % 64) < 32
    q[:, 0, rows] *= 48  # log2-domain scores up to ~330 in rows 0-31; rows 32-63 stay below 10
    nb = math.ceil(L / 64)
    g = torch.Generator().manual_seed(531)
    mask = torch.rand(B, H, nb, nb, generator=g) < 0.6
    mask[..., 0] = True
    scale = 1 / math.sqrt(D)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
    _check(out, masked_attention(q, k, v, mask, scale))


def test_uniform_negative_bias_is_shift_invariant(dev):
    # A bias of -300 on every key underflows exp2 without the max subtraction; softmax is
    # shift invariant, so the result must equal the unbiased one.
    case("uniform -300 key bias")
    B, H, L = 1, 2, 200
    q, k, v = (_rand((B, H, L, 64), 140 + i) for i in range(3))
    mask = torch.ones(1, 1, 4, 4, dtype=torch.bool)
    kv = kv_list_from_mask(mask.to(dev), B, H, 4, 4)
    bias = torch.full((B, 1, L), -300.0)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, key_bias=bias.to(dev))
    _check(out, masked_attention(q, k, v, mask, 0.125))


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 64), (torch.bfloat16, 128),
                                     (torch.float16, 128)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_row_mapped_queries_and_outputs(dev, with_bias, dtype, D):
    # Logical query i reads q row q_rows[i] (-1: zero padding) and is written to out row
    # o_rows[i] (-1: dropped): a permute + pad -> attend -> unpad + unpermute in one launch.
    case(f"row maps bias={with_bias} dtype={dtype} D={D}")
    B, H, Lsrc, Lk = 2, 3, 300, 260
    g = torch.Generator().manual_seed(21)
    q, k, v = _rand((B, H, Lsrc, D), 150, dtype), _rand((B, H, Lk, D), 151, dtype), _rand((B, H, Lk, D), 152, dtype)
    perm = torch.randperm(Lsrc, generator=g)
    q_rows = torch.cat([perm[:150], torch.full((20,), -1), perm[150:], torch.full((10,), 7 * Lsrc)]).int()
    o_rows = q_rows.clone()
    o_rows[5] = -1  # this logical row is computed but not stored
    Lq = q_rows.numel()
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.6
    mask[..., 0] = True
    bias = torch.log(torch.randint(1, 5, (B, 1, Lk), generator=g).float()) if with_bias else None
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    out = torch.full((B, H, Lsrc, D), 3.0, dtype=dtype, device=dev)
    scale = 1 / math.sqrt(D)
    block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, scale, key_bias=None if bias is None else bias.to(dev),
                           out=out, q_rows=q_rows.to(dev), o_rows=o_rows.to(dev))
    out = out.cpu()
    valid = (q_rows >= 0) & (q_rows < Lsrc)
    ql = torch.zeros(B, H, Lq, D, dtype=dtype)
    ql[:, :, valid] = q[:, :, q_rows[valid].long()]
    want = masked_attention(ql, k, v, mask, scale, key_bias=None if bias is None else bias.double())
    stored = valid.clone()
    stored[5] = False
    _check(out[:, :, o_rows[stored].long()], want[:, :, stored])
    untouched = torch.ones(Lsrc, dtype=torch.bool)
    untouched[o_rows[stored].long()] = False
    assert torch.all(out[:, :, untouched] == 3.0)


def test_mask_to_kv_list_matches_nonzero(dev):
    case("mask_to_kv_list")
    g = torch.Generator().manual_seed(8)
    mask = torch.rand(2, 3, 7, 150, generator=g) < 0.3
    kv = kv_list_from_mask(mask.to(dev), 2, 3, 7, 150)
    idx, cnt = kv.idx.cpu(), kv.cnt.cpu()
    flat = mask.reshape(-1, 150)
    for r in range(flat.shape[0]):
        want = torch.nonzero(flat[r]).flatten().int()
        assert cnt[r].item() == want.numel()
        assert torch.equal(idx[r, : cnt[r]], want)
    assert torch.equal(kv.to_mask().cpu(), mask)


def test_invalid_list_entries_are_skipped(dev):
    case("invalid kv entries")
    q, k, v = (_rand((1, 1, 128, 64), 70 + i) for i in range(3))
    idx = torch.tensor([[0, 99, -3], [1, 2, 0]], dtype=torch.int32)
    cnt = torch.tensor([3, 1], dtype=torch.int32)
    kv = KVList(idx.to(dev), cnt.to(dev), 1, 1, 2, 2)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125)
    mask = torch.tensor([[[[True, False], [False, True]]]])
    _check(out, masked_attention(q, k, v, mask, 0.125))


def test_factory_and_backward(dev):
    case("factory + backward")
    fn = sparse_attention_factory(64, 64)
    q, k, v = (_rand((1, 1, 64, 64), 80 + i).to(dev) for i in range(3))
    m = torch.ones(1, 1, 1, 1, dtype=torch.bool, device=dev)
    out = fn(q, k, v, m, 0.125)
    assert out.shape == q.shape
    with pytest.raises(ValueError):  # BLOCK_M must be a power of two from 16 to 1024
        sparse_attention_factory(96, 64)(q, k, v, m, 0.125)
    qg = q.clone().requires_grad_(True)
    o = block_sparse_triton_fn(qg, k, v, m, 0.125)
    with pytest.raises(NotImplementedError):
        o.float().sum().backward()


def test_cogvideox_shape_subset_of_heads(dev):
    # Full CogVideoX-2B shape (B=2, H=30, L=17776) with a random ~20% mask; the oracle checks
    # 3 of the 60 heads in full and 40 sampled rows (text, random, the last) of every head.
    case("CogVideoX shape random 20% mask")
    B, H, L = 2, 30, 17776
    nb = math.ceil(L / 64)
    q, k, v = (_rand((B, H, L, 64), 90 + i) for i in range(3))
    g = torch.Generator().manual_seed(9)
    mask = torch.rand(B, H, nb, nb, generator=g) < 0.2
    mask[:, :, :4, :] = True
    mask[:, :, :, :4] = True
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125).cpu()
    heads = [(0, 0), (1, 17), (1, 29)]
    want = masked_attention(q, k, v, mask, 0.125, heads=heads)
    for b, h in heads:
        _check(out[b, h], want[b, h])
    for b in range(B):
        for h in range(H):
            rows = torch.unique(torch.cat([torch.randint(0, 256, (8,), generator=g),
                                           torch.randint(256, L, (31,), generator=g), torch.tensor([L - 1])]))
            w = masked_attention(q, k, v, mask, 0.125, heads=[(b, h)], rows=rows)[b, h]
            _check(out[b, h, rows], w)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128), (torch.float16, 128)])
def test_fp16_and_head_dim_128(dev, dtype, D):
    # The reference accepts head_dim 64 or 128 (:231) and any 16-bit input type (P is rounded
    # to v's dtype, :107). Partial last block, Lq < Lk, a random mask with an empty row.
    case(f"dtype={dtype} D={D}")
    for (Lq, Lk, seed) in [(257, 257, 1), (200, 385, 2)]:
        q = _rand((2, 3, Lq, D), 100 + seed, dtype)
        k = _rand((2, 3, Lk, D), 110 + seed, dtype)
        v = _rand((2, 3, Lk, D), 120 + seed, dtype)
        nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
        g = torch.Generator().manual_seed(seed)
        mask = torch.rand(2, 3, nqb, nkb, generator=g) < 0.5
        mask[:, :, :, 0] = True
        mask[1, 2, 1] = False  # an empty row writes 0
        scale = 1 / math.sqrt(D)
        out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
        assert out.dtype == dtype and out.shape == q.shape
        _check(out, masked_attention(q, k, v, mask, scale))


@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128)])
def test_fp16_and_head_dim_128_key_bias(dev, dtype, D):
    case(f"key bias dtype={dtype} D={D}")
    q, k, v = (_rand((1, 2, 300, D), 130 + i, dtype) for i in range(3))
    bias = torch.log(torch.randint(1, 5, (1, 2, 300), generator=torch.Generator().manual_seed(3)).float())
    nb = math.ceil(300 / 64)
    kv = kv_list_from_mask(torch.ones(1, 1, nb, nb, dtype=torch.bool, device=dev), 1, 2, nb, nb)
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 1 / 8, key_bias=bias.to(dev))
    _check(out, masked_attention(q, k, v, torch.ones(1, 1, nb, nb, dtype=torch.bool), 1 / 8, key_bias=bias.double()))


def test_fp16_large_scores_use_running_max(dev):
    # fp16 P cannot hold exp2 of raw scores of several hundred: the fp16 fast pass subtracts
    # each row's maximum over the first tile, and rows whose later tiles exceed it by more
    # than 2^16 are redone with the running maximum.
    case("fp16 large scores")
    q = (_rand((1, 1, 128, 64), 140) * 6).half()
    k = (_rand((1, 1, 128, 64), 141) * 6).half()
    v = _rand((1, 1, 128, 64), 142, torch.float16)
    mask = torch.ones(1, 1, 2, 2, dtype=torch.bool)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 1 / 8)
    _check(out, masked_attention(q, k, v, mask, 1 / 8))


@pytest.mark.parametrize("large_first", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_fp16_offset_from_first_tile(dev, large_first, D):
    # Key block 0 small, key block 1 with scores ~35 (log2 units) higher: with the large block
    # first, its row maxima make every exp2 argument <= 0; with the small block first, the
    # second tile's P exceeds fp16's range (P = inf, row sum inf) and the item is redone
    # with the running maximum. Both must match the fp64 oracle.
    case(f"fp16 first-tile offset large_first={large_first} D={D}")
    q = _rand((1, 2, 128, D), 150)
    k = _rand((1, 2, 128, D), 151)
    small, large = slice(0, 64), slice(64, 128)
    if large_first:
        small, large = large, small
    k[:, :, small] *= 0.01
    k[:, :, large] *= 10.0 * math.sqrt(64 / D)
    q, k = q.half(), k.half()
    v = _rand((1, 2, 128, D), 152, torch.float16)
    mask = torch.ones(1, 2, 2, 2, dtype=torch.bool)
    # Lists hold key block 0 then 1, so the small block is the first tile unless large_first.
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), dense_kv_list(1, 2, 2, 2, dev), 1 / 8)
    _check(out, masked_attention(q, k, v, mask, 1 / 8))
    if D == 128:  # plain lists at head dim 128 run the wave-pair kernel; the key-bias variant does not
        zero = torch.zeros(1, 2, 128, dtype=torch.float32, device=dev)
        outb = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), dense_kv_list(1, 2, 2, 2, dev), 1 / 8,
                                      key_bias=zero)
        _check(outb, masked_attention(q, k, v, mask, 1 / 8))


def test_mixed_or_fp64_dtypes_rejected(dev):
    case("dtype errors")
    q = _rand((1, 1, 64, 64), 150).to(dev)
    m = torch.ones(1, 1, 1, 1, dtype=torch.bool, device=dev)
    with pytest.raises(TypeError):
        block_sparse_triton_fn(q, q.half(), q, m, 1 / 8)
    with pytest.raises(TypeError):
        block_sparse_triton_fn(q.float(), q.float(), q, m, 1 / 8)
    with pytest.raises(TypeError):
        block_sparse_triton_fn(q.double(), q.double(), q.double(), m, 1 / 8)
    with pytest.raises(AssertionError):  # head dims the reference asserts: 64 or 128
        qq = torch.randn(1, 1, 64, 96, device=dev)
        block_sparse_triton_fn(qq, qq, qq, m, 1 / 8)


# fp32 inputs: the reference's kernel takes them too (tl.dot on fp32 tiles, P cast to v's
# dtype, so kept in fp32). Without the bf16 rounding of P the bar is fp32 accuracy: max-abs
# 2e-5, mean-abs 2e-6 against the fp64 oracle on the same fp32 inputs.
F32_MAX, F32_MEAN = 2e-5, 2e-6


def _check_f32(got, want, max_abs=F32_MAX, mean_abs=F32_MEAN):
    assert got.dtype == torch.float32
    err = (got.cpu().double() - want).abs()
    assert torch.isfinite(got).all()
    assert err.max().item() <= max_abs, err.max().item()
    assert err.mean().item() <= mean_abs, err.mean().item()


def test_config1_parity_fp32(dev):
    # BASELINE configs[0] in its own dtype: B=1, H=2, L=2048, d=64, fp32, the seed-1 mask.
    case("C1 fp32")
    q, k, v, mask, scale = config1_inputs()
    assert q.dtype == torch.float32
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
    _check_f32(out, masked_attention(q, k, v, mask, scale))


@pytest.mark.parametrize("Lq,Lk,seed", [(257, 257, 1), (130, 385, 2), (64, 20, 3), (1000, 1000, 4)])
def test_fp32_random_masks(dev, Lq, Lk, seed):
    # partial last tiles, Lq != Lk, an empty row, an entry outside the grid in one list
    case(f"fp32 Lq={Lq} Lk={Lk}")
    B, H = 2, 3
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, n, 64, generator=g) for n in (Lq, Lk, Lk))
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.5
    mask[..., nkb - 1] = True
    mask[1, 2, 0] = False  # an empty row writes 0
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    first = kv.idx[0, 0].item()  # row (0, 0, 0): its first entry moved outside the grid is skipped
    kv.idx[0, 0] = nkb + 3
    mask[0, 0, 0, first] = False
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125)
    _check_f32(out, masked_attention(q, k, v, mask, 0.125))
    assert torch.all(out[1, 2, :64] == 0)


@pytest.mark.parametrize("Lq,Lk,seed", [(257, 257, 11), (130, 385, 12), (700, 700, 13)])
def test_fp32_head_dim_128(dev, Lq, Lk, seed):
    # head dim 128 (the reference accepts 64 and 128 for any dtype, :230-231): two 64-wide
    # halves of d in the scores, eight 16-row d blocks of the output
    case(f"fp32 d=128 Lq={Lq} Lk={Lk}")
    B, H = 1, 3
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, n, 128, generator=g) for n in (Lq, Lk, Lk))
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.5
    mask[..., 0] = True
    mask[0, 1, 1] = False  # an empty row writes 0
    scale = 1 / math.sqrt(128)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
    assert out.shape == q.shape
    _check_f32(out, masked_attention(q, k, v, mask, scale))
    assert torch.all(out[0, 1, 64:128].cpu() == 0)


def test_fp32_strided_and_large_scores(dev):
    # BLHD views (strided rows) and scores of several hundred (the running maximum)
    case("fp32 strided, large scores")
    B, L, H = 1, 300, 2
    g = torch.Generator().manual_seed(9)
    base = [torch.randn(B, L, H, 64, generator=g) * (6.0 if i < 2 else 1.0) for i in range(3)]
    q, k, v = (t.to(dev).permute(0, 2, 1, 3) for t in base)
    nb = math.ceil(L / 64)
    mask = torch.rand(1, 1, nb, nb, generator=g) < 0.6
    mask[..., 0] = True
    out = block_sparse_triton_fn(q, k, v, mask.to(dev), 0.125)
    # logits up to ~300: fp32 rounding of a logit alone is 2^-24 * 300 ~ 2e-5, so the bar
    # scales with them (max-abs 1e-4)
    _check_f32(out, masked_attention(*(t.permute(0, 2, 1, 3) for t in base), mask, 0.125), 1e-4, 1e-5)


def _split_parts(n_items, max_cnt, D=64):
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import split_parts
    return split_parts(n_items, max_cnt, D)


@pytest.mark.parametrize("B,H,Lq,Lk,D,dtype,amp", [
    (1, 2, 200, 8192, 64, torch.bfloat16, 1.0),   # partial last query block
    (2, 3, 64, 4500, 64, torch.bfloat16, 1.0),    # partial last key block
    (1, 2, 64, 4096, 128, torch.bfloat16, 1.0),   # head dim 128
    (1, 2, 100, 4096, 64, torch.float16, 1.0),    # fp16 (each part offsets by its first tile's row maxima)
    (1, 2, 128, 6000, 64, torch.bfloat16, 8.0),   # scores of several hundred: parts redo safely
])
def test_key_range_split_dense(dev, B, H, Lq, Lk, D, dtype, amp):
    # Few query blocks over long lists: each block's list is split into key ranges whose fp32
    # partials a second kernel merges (the reference's Triton grid has one program per block).
    case(f"key-range split B={B} H={H} Lq={Lq} Lk={Lk} D={D} {dtype} amp={amp}")
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    assert _split_parts(B * H * nqb, nkb, D) > 1
    q = (_rand((B, H, Lq, D), 500, torch.float32) * amp).to(dtype)
    k = (_rand((B, H, Lk, D), 501, torch.float32) * amp).to(dtype)
    v = _rand((B, H, Lk, D), 502, dtype)
    mask = torch.ones(B, H, nqb, nkb, dtype=torch.bool)
    scale = 1 / math.sqrt(D)
    out = block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), scale)
    # scores of several hundred: fp32 rounding of the logits alone is ~2e-5 of them, and the
    # softmax is near one-hot, so the bar stays the attention bar
    _check(out, masked_attention(q, k, v, mask, scale))


def test_key_range_split_sparse_lists(dev):
    # Lists shorter than the parts (empty key ranges), an empty list (writes 0), entries
    # outside the grid, and a one-block list.
    case("key-range split, sparse lists")
    B, H, Lq, Lk = 1, 3, 192, 6000
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    assert _split_parts(B * H * nqb, nkb) > 1
    q, k, v = (_rand((B, H, n, 64), 510 + i) for i, n in enumerate((Lq, Lk, Lk)))
    g = torch.Generator().manual_seed(51)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.08
    mask[0, 0, 1] = False
    mask[0, 1, 2] = False
    mask[0, 1, 2, 17] = True
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    kv.idx[2, kv.cnt[2].item()] = nkb + 5  # past the count: never read
    assert kv.cnt[4].item() > 0
    first = kv.idx[4, 0].item()
    kv.idx[4, 0] = -3  # an entry outside the grid is skipped
    mask[0, 1, 1, first] = False
    out = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125).cpu()
    assert torch.all(out[0, 0, 64:128] == 0)
    _check(out, masked_attention(q, k, v, mask, 0.125))


def test_key_range_split_matches_unsplit(dev):
    # The same query blocks in a launch with enough blocks to run unsplit: the outputs agree
    # up to the fp32 summation order of the partials (one bf16 rounding step). The unsplit
    # launch takes the bf16 scores of the split one (fp16_scores=False).
    case("key-range split vs unsplit")
    Lk = 8192
    q, k, v = _rand((1, 2, 128, 64), 520), _rand((1, 2, Lk, 64), 521), _rand((1, 2, Lk, 64), 522)
    reps = 300
    assert _split_parts(1 * 2 * 2, Lk // 64) > 1 and _split_parts(1 * 2 * 2 * reps, Lk // 64) == 1
    kd, vd = k.to(dev), v.to(dev)
    small = block_sparse_attention(q.to(dev), kd, vd, dense_kv_list(1, 2, 2, Lk // 64, dev), 0.125)
    big = block_sparse_attention(q.repeat(1, 1, reps, 1).to(dev), kd, vd, dense_kv_list(1, 2, 2 * reps, Lk // 64, dev),
                                 0.125, fp16_scores=False)
    torch.cuda.synchronize()
    d = (small.float() - big[:, :, :128].float()).abs()
    assert d.max().item() <= 2 ** -8, d.max().item()
    assert (d > 0).float().mean().item() < 0.05
    _check(small, masked_attention(q, k, v, torch.ones(1, 2, 2, Lk // 64, dtype=torch.bool), 0.125))


def test_key_range_split_row_maps(dev):
    # Row-mapped queries and outputs with a split launch: the merge kernel writes through o_rows.
    case("key-range split with row maps")
    B, H, Lsrc, Lk = 1, 2, 200, 4096
    g = torch.Generator().manual_seed(53)
    q, k, v = _rand((B, H, Lsrc, 64), 530), _rand((B, H, Lk, 64), 531), _rand((B, H, Lk, 64), 532)
    perm = torch.randperm(Lsrc, generator=g)
    q_rows = torch.cat([perm[:120], torch.full((8,), -1), perm[120:]]).int()
    o_rows = q_rows.clone()
    o_rows[3] = -1
    Lq = q_rows.numel()
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    assert _split_parts(B * H * nqb, nkb) > 1
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.7
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    out = torch.full((B, H, Lsrc, 64), 3.0, dtype=torch.bfloat16, device=dev)
    block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, out=out, q_rows=q_rows.to(dev),
                           o_rows=o_rows.to(dev))
    out = out.cpu()
    valid = q_rows >= 0
    ql = torch.zeros(B, H, Lq, 64, dtype=torch.bfloat16)
    ql[:, :, valid] = q[:, :, q_rows[valid].long()]
    want = masked_attention(ql, k, v, mask, 0.125)
    stored = valid.clone()
    stored[3] = False
    _check(out[:, :, o_rows[stored].long()], want[:, :, stored])
    untouched = torch.ones(Lsrc, dtype=torch.bool)
    untouched[o_rows[stored].long()] = False
    assert torch.all(out[:, :, untouched] == 3.0)


@pytest.mark.parametrize("with_bias", [False, True])
def test_v32_matches_first_columns(dev, with_bias):
    # 32 value columns (segment-indicator v): the output equals the first 32 columns of the
    # full launch bit for bit (same scores, softmax and P.V chains), and the oracle within the
    # attention bar; partial last tiles, an empty list, strided 32-column output.
    case(f"v32 bias={with_bias}")
    B, H, Lq, Lk = 2, 3, 300, 1000
    q, k, v = _rand((B, H, Lq, 64), 540), _rand((B, H, Lk, 64), 541), _rand((B, H, Lk, 64), 542)
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    g = torch.Generator().manual_seed(54)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.5
    mask[..., 0] = True
    mask[1, 0, 2] = False  # an empty list writes 0
    bias = torch.log(torch.randint(1, 5, (B, 1, Lk), generator=g).float()) if with_bias else None
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    bd = None if bias is None else bias.to(dev)
    # the 64-column launch with the bf16 scores that the 32-column one computes
    full = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, key_bias=bd, fp16_scores=False)
    wide = torch.full((B, H, Lq, 48), 5.0, dtype=torch.bfloat16, device=dev)
    got = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), kv, 0.125, key_bias=bd, out=wide[..., 8:40],
                                 v_cols=32)
    torch.cuda.synchronize()
    assert got.shape == (B, H, Lq, 32)
    assert torch.equal(got, full[..., :32])
    assert torch.all(wide[..., :8] == 5.0) and torch.all(wide[..., 40:] == 5.0)
    want = masked_attention(q, k, v, mask, 0.125, key_bias=None if bias is None else bias.double())
    _check(got, want[..., :32])
    assert torch.all(got.cpu()[1, 0, 128:192] == 0)
    with pytest.raises(NotImplementedError):
        block_sparse_attention(q.half().to(dev), k.half().to(dev), v.half().to(dev), kv, 0.125, v_cols=32)


def _split_call(q, k, v, kv, scale, parts, ws, nbytes, out, fp16=False):
    from sparseattnfunctions_amd import _lib
    B, H, Lq, D = q.shape
    fn = "sa_block_sparse_fwd_split_f16" if fp16 else "sa_block_sparse_fwd_split"
    rc = getattr(_lib.load(), fn)(
        q.data_ptr(), _lib.i64(*q.stride()[:3]), k.data_ptr(), _lib.i64(*k.stride()[:3]),
        v.data_ptr(), _lib.i64(*v.stride()[:3]), out.data_ptr(), _lib.i64(*out.stride()[:3]),
        B, H, Lq, k.shape[2], D, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, float(scale),
        None, 0, None, 0, parts, None if ws is None else ws.data_ptr(), nbytes, _lib.stream_of(q))
    _lib.check(rc, fn)
    return out


def test_key_range_split_caller_workspace(dev):
    # The split runs in a workspace the caller owns: two calls with the same arguments give
    # the same bits (also after the workspace held other data), both match the fp64 oracle,
    # and parts = 1 without a workspace is the plain entry point's unsplit launch, bit for bit.
    from sparseattnfunctions_amd import _lib
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import split_workspace_bytes
    case("key-range split with a caller workspace")
    B, H, Lq, Lk, D = 1, 3, 130, 7000, 64
    nqb, nkb = math.ceil(Lq / 64), math.ceil(Lk / 64)
    parts = _split_parts(B * H * nqb, nkb, D)
    assert parts > 1
    q, k, v = _rand((B, H, Lq, D), 540), _rand((B, H, Lk, D), 541), _rand((B, H, Lk, D), 542)
    g = torch.Generator().manual_seed(54)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.6
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    nbytes = split_workspace_bytes(B * H * nqb, D, parts)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=dev)
    o1 = _split_call(qd, kd, vd, kv, 0.125, parts, ws, nbytes, torch.empty_like(qd))
    ws.fill_(0xFF)  # NaN patterns: every partial is rewritten by the next call
    o2 = _split_call(qd, kd, vd, kv, 0.125, parts, ws, nbytes, torch.empty_like(qd))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    want = masked_attention(q, k, v, mask, 0.125)
    _check(o1, want)
    # Other part counts: the same result up to the fp32 summation order of the partials.
    o3 = _split_call(qd, kd, vd, kv, 0.125, 3, ws, nbytes, torch.empty_like(qd))
    _check(o3, want)
    # parts = 1 with no workspace, and the plain entry point (never split): one wave per block.
    o4 = _split_call(qd, kd, vd, kv, 0.125, 1, None, 0, torch.empty_like(qd))
    o5 = torch.empty_like(qd)
    rc = _lib.load().sa_block_sparse_fwd(
        qd.data_ptr(), _lib.i64(*qd.stride()[:3]), kd.data_ptr(), _lib.i64(*kd.stride()[:3]),
        vd.data_ptr(), _lib.i64(*vd.stride()[:3]), o5.data_ptr(), _lib.i64(*o5.stride()[:3]),
        B, H, Lq, Lk, D, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, None, None, 0.125, None, 0,
        _lib.stream_of(qd))
    _lib.check(rc, "sa_block_sparse_fwd")
    torch.cuda.synchronize()
    assert torch.equal(o4, o5)
    _check(o5, want)
    d = (o1.float() - o5.float()).abs()
    assert d.max().item() <= 2 ** -8, d.max().item()
    # A short workspace is refused before any launch.
    rc = _lib.load().sa_block_sparse_fwd_split(
        qd.data_ptr(), _lib.i64(*qd.stride()[:3]), kd.data_ptr(), _lib.i64(*kd.stride()[:3]),
        vd.data_ptr(), _lib.i64(*vd.stride()[:3]), o5.data_ptr(), _lib.i64(*o5.stride()[:3]),
        B, H, Lq, Lk, D, kv.idx.data_ptr(), kv.cnt.data_ptr(), kv.max_cnt, 0.125, None, 0, None, 0, parts,
        ws.data_ptr(), nbytes - 4, _lib.stream_of(qd))
    assert rc == _lib.SA_ERR_INVALID


def _token_mask(mask, Lq, Lk, bm, bn):
    """Token-level [B, H, Lq, Lk] expansion of a block mask of bm x bn blocks."""
    rows = torch.arange(Lq) // bm
    cols = torch.arange(Lk) // bn
    return mask[:, :, rows][:, :, :, cols]


@pytest.mark.parametrize("bm,bn,Lq,Lk", [
    (32, 32, 300, 300), (16, 64, 200, 333), (64, 16, 257, 190), (128, 128, 500, 500),
    (128, 64, 300, 450), (32, 128, 260, 515), (16, 16, 150, 170), (256, 32, 600, 300),
])
def test_factory_block_shapes(dev, bm, bn, Lq, Lk):
    # sparse_attention_factory(BLOCK_M, BLOCK_N) (block_sparse_attn_kernel.py:283-291): mask row
    # m covers query rows m*BLOCK_M.., column n keys n*BLOCK_N.. (:139-155). Against the fp64
    # oracle on the token-level expansion of the mask; rows whose cells are all off write 0.
    case(f"factory BLOCK_M={bm} BLOCK_N={bn} Lq={Lq} Lk={Lk}")
    B, H = 1, 2
    g = torch.Generator().manual_seed(bm * 13 + bn + Lq)
    q, k, v = _rand((B, H, Lq, 64), 600 + bm), _rand((B, H, Lk, 64), 601 + bn), _rand((B, H, Lk, 64), 602)
    nM, nN = math.ceil(Lq / bm), math.ceil(Lk / bn)
    mask = torch.rand(B, H, nM, nN, generator=g) < 0.35
    mask[0, 0, 0] = False  # an empty row of cells
    mask[0, 1, -1] = True  # a full row of cells, last (partial) one included
    fn = sparse_attention_factory(BLOCK_M=bm, BLOCK_N=bn)
    out = fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125)
    tok = _token_mask(mask, Lq, Lk, bm, bn)
    want = masked_attention(q, k, v, tok, 0.125, block=1)
    _check(out, want)
    assert torch.all(out[0, 0, :min(bm, Lq)].cpu() == 0)
    # the same mask at 64 x 64 granularity where it is one: bit-identical to the 64 path
    if bm == 64 and bn == 64:
        assert torch.equal(out, block_sparse_triton_fn(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125))


def test_factory_block_shapes_fp16_and_d128(dev):
    case("factory 32 x 32, fp16 and head dim 128")
    g = torch.Generator().manual_seed(71)
    for dtype, D in ((torch.float16, 64), (torch.bfloat16, 128)):
        q, k, v = (torch.randn(1, 2, 230, D, generator=g).to(dtype) for _ in range(3))
        mask = torch.rand(1, 2, 8, 8, generator=g) < 0.4
        mask[..., 0] = True
        out = sparse_attention_factory(32, 32)(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 1 / math.sqrt(D))
        _check(out, masked_attention(q, k, v, _token_mask(mask, 230, 230, 32, 32), 1 / math.sqrt(D), block=1))


def test_factory_block_shapes_fp32(dev):
    # fp32 inputs: whole-tile shapes (multiples of 64) run the fp32 kernel on the expanded
    # lists; smaller blocks need token masks, which the fp32 kernel does not have.
    case("factory fp32")
    g = torch.Generator().manual_seed(72)
    q, k, v = (torch.randn(1, 2, 300, 64, generator=g) for _ in range(3))
    mask = torch.rand(1, 2, 3, 5, generator=g) < 0.5
    mask[..., 0] = True
    out = sparse_attention_factory(128, 64)(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.125)
    _check_f32(out, masked_attention(q, k, v, _token_mask(mask, 300, 300, 128, 64), 0.125, block=1))
    with pytest.raises(NotImplementedError):
        sparse_attention_factory(32, 64)(q.to(dev), k.to(dev), v.to(dev), torch.ones(1, 2, 10, 5, dtype=torch.bool,
                                                                                    device=dev), 0.125)
