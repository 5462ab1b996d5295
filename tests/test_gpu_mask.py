"""GPU parity of block pooling and top-k kv-list construction: bit-exact against the C oracle."""
import math

import pytest
import torch

from conftest import case
from oracle import native
from sparseattnfunctions_amd.block_masks import meanpool_topk_kv_list, pool_blocks, topk_kv_list
from sparseattnfunctions_amd.workloads import COGVIDEOX_2B, cogvideox_qkv, topk_count

pytestmark = pytest.mark.gpu


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _same_lists(kv, idx, cnt):
    gi, gc = kv.idx.cpu(), kv.cnt.cpu()
    assert torch.equal(gc, cnt)
    for r in range(cnt.numel()):
        assert torch.equal(gi[r, : cnt[r]], idx[r, : cnt[r]]), r


@pytest.mark.parametrize("L,block", [(64, 64), (257, 64), (1000, 64), (300, 128)])
def test_pool_bit_exact(dev, L, block):
    case(f"pool L={L} block={block}")
    q, k = _rand((2, 3, L, 64), 1), _rand((2, 3, L, 64), 2)
    qp, kp = pool_blocks(q.to(dev), k.to(dev), block)
    assert torch.equal(qp.cpu(), native.block_pool(q, block))
    assert torch.equal(kp.cpu(), native.block_pool(k, block))


def test_pool_strided_input(dev):
    case("pool strided")
    base = _rand((2, 500, 4, 64), 3)
    qp, _ = pool_blocks(base.to(dev).permute(0, 2, 1, 3))
    assert torch.equal(qp.cpu(), native.block_pool(base.permute(0, 2, 1, 3)))


@pytest.mark.parametrize("nkb,topk,n_text", [(5, 2, 1), (100, 20, 4), (278, 55, 4), (705, 70, 4), (1024, 1, 0)])
def test_topk_from_pooled_bit_exact(dev, nkb, topk, n_text):
    case(f"topk pooled nkb={nkb} topk={topk}")
    g = torch.Generator().manual_seed(nkb)
    qp = torch.randn(3, nkb, 64, generator=g)
    kp = torch.randn(3, nkb, 64, generator=g)
    kv, mask, scores = topk_kv_list(qp.to(dev), kp.to(dev), 1, 3, topk, n_text, return_mask=True, return_scores=True)
    idx, cnt, omask, oscores = native.block_topk(qp, kp, topk, n_text)
    assert torch.equal(scores.cpu().reshape(-1, nkb), oscores)
    assert torch.equal(mask.cpu().reshape(-1, nkb), omask.bool())
    _same_lists(kv, idx, cnt)


def test_topk_ties_and_specials_from_scores(dev):
    case("topk ties / NaN / signed zero")
    g = torch.Generator().manual_seed(5)
    s = torch.randint(0, 4, (2, 30, 278), generator=g).float()
    s[0, 0, :3] = torch.tensor([float("nan"), -0.0, 0.0])
    s[0, 1, 7] = float("inf")
    s[0, 2, 9] = float("-inf")
    loc = (torch.rand(30, 278, generator=g) < 0.1)
    kv, mask = topk_kv_list(None, None, 1, 2, 27, 4, local_bitmap=loc.to(dev), scores_in=s.to(dev),
                            return_mask=True)
    idx, cnt, omask, _ = native.block_topk(None, None, 27, 4, local=loc, scores_in=s)
    assert torch.equal(mask.cpu().reshape(-1, 278), omask.bool())
    _same_lists(kv, idx, cnt)


def test_config2_mask_bit_exact(dev):
    # Full config-2 rule at the CogVideoX-2B shape: mean-pool, fp32 scores, top-55 + text.
    case("config2 mask full shape")
    geom = COGVIDEOX_2B
    q, k, _ = cogvideox_qkv(0)
    topk = topk_count(0.2, geom.nb)
    assert topk == 55
    kv = meanpool_topk_kv_list(q.to(dev), k.to(dev), topk, geom.n_text_blocks)
    idx, cnt, _, _ = native.block_topk(native.block_pool(q), native.block_pool(k), topk, geom.n_text_blocks)
    _same_lists(kv, idx, cnt)
    # Every video row keeps exactly |top-k U text columns| blocks; text rows keep all.
    c = kv.cnt.cpu().reshape(60, geom.nb)
    assert torch.all(c[:, :4] == geom.nb)
    assert torch.all((c[:, 4:] >= topk) & (c[:, 4:] <= topk + 4))


def _torch_topk_mask(x, topk, dense_last):
    """The reference's own recipe (block_sparse_attn_kernel.py:31-39) with torch CPU ops."""
    bsz, nh, n, _ = x.shape
    idx = torch.topk(x, topk, dim=-1).indices
    m = torch.zeros(bsz, nh, n, n, dtype=torch.bool)
    m.scatter_(-1, idx, True)
    if dense_last:
        m[:, :, -2:, :] = True
    return m


@pytest.mark.parametrize("n,topk,dense_last,dtype", [(32, 8, False, torch.float32), (278, 55, True, torch.float32),
                                                      (100, 100, False, torch.float32), (64, 1, True, torch.bfloat16)])
def test_mask_from_topk_matches_torch(dev, n, topk, dense_last, dtype):
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import get_sparse_attn_mask_from_topk

    case(f"get_sparse_attn_mask_from_topk n={n} topk={topk} dense_last={dense_last} {dtype}")
    g = torch.Generator().manual_seed(n + topk)
    # Tie-free rows: a random permutation of distinct values per row (exact in bf16 up to 256).
    x = torch.argsort(torch.rand(2, 3, n, n, generator=g), dim=-1).to(torch.float32) - n / 2
    x = x.to(dtype)
    got = get_sparse_attn_mask_from_topk(x.to(dev), topk, use_dense_for_last_block=dense_last)
    assert got.dtype == torch.bool and got.shape == (2, 3, n, n)
    assert torch.equal(got.cpu(), _torch_topk_mask(x.float(), topk, dense_last))


def test_mask_from_topk_ties_vs_oracle(dev):
    from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import get_sparse_attn_mask_from_topk

    case("get_sparse_attn_mask_from_topk ties")
    g = torch.Generator().manual_seed(11)
    x = torch.randint(0, 3, (1, 4, 50, 50), generator=g).float()
    x[0, 0, 0, :4] = torch.tensor([float("nan"), float("inf"), -0.0, 0.0])
    got = get_sparse_attn_mask_from_topk(x.to(dev), 7, use_dense_for_last_block=True)
    _, _, omask, _ = native.block_topk(None, None, 7, 0, scores_in=x.reshape(4, 50, 50))
    want = omask.bool().reshape(1, 4, 50, 50).clone()
    want[:, :, -2:, :] = True
    assert torch.equal(got.cpu(), want)
    # Exactly topk entries in every row above the dense tail.
    assert torch.all(got[:, :, :-2].sum(-1).cpu() == 7)
    with pytest.raises(RuntimeError):
        get_sparse_attn_mask_from_topk(x.to(dev), 51)
