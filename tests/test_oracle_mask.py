"""Pins the C oracle of block pooling and top-k selection (oracle/sa_oracle.c)."""
import torch

from oracle import native


def _bf16(vals):
    return torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16)


def test_pool_exact_on_integers():
    # Integer-valued bf16 inputs: fp32 sums are exact, so the mean is one IEEE division.
    g = torch.Generator().manual_seed(0)
    x = torch.randint(-100, 101, (2, 3, 150, 64), generator=g).to(torch.bfloat16)
    got = native.block_pool(x)
    sums = x.double().reshape(6, 150, 64)
    for blk, (t0, t1) in enumerate([(0, 64), (64, 128), (128, 150)]):
        want = sums[:, t0:t1].sum(1).float() / float(t1 - t0)
        assert torch.equal(got[:, blk], want)


def test_pool_sums_tokens_in_ascending_order():
    # [2^24, 1 x 63]: ascending order rounds every +1 away (tie to even) -> 2^24 / 64 = 2^18;
    # any other association of the sum would give a larger value.
    x = torch.ones(1, 1, 64, 64, dtype=torch.bfloat16)
    x[0, 0, 0, :] = 2.0 ** 24
    assert torch.all(native.block_pool(x) == 2.0 ** 18)
    x2 = x.flip(2)  # ones first: 63 + 2^24 -> 16777280
    assert torch.all(native.block_pool(x2) == 16777280.0 / 64)


def test_pool_close_to_fp64_mean():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 2, 300, 64, generator=g).to(torch.bfloat16)
    got = native.block_pool(x).double()
    xd = x.double().reshape(2, 300, 64)
    for blk in range(5):
        want = xd[:, 64 * blk:min(300, 64 * blk + 64)].mean(1)
        assert torch.allclose(got[:, blk], want, atol=1e-5)


def test_score_is_ascending_fused_chain():
    lib = native.lib()
    import ctypes
    a = 1.0 + 2.0 ** -12
    q = (ctypes.c_float * 2)(a, 1.0)
    k = (ctypes.c_float * 2)(a, -(1.0 + 2.0 ** -11))
    # fmaf(a, a, 0) rounds (tie to even) to 1 + 2^-11, then fmaf(1, -(1 + 2^-11), .) = 0.
    assert lib.oracle_block_score(q, k, 2) == 0.0
    q2 = (ctypes.c_float * 2)(1.0, a)
    k2 = (ctypes.c_float * 2)(-(1.0 + 2.0 ** -11), a)
    # Reversed order: fmaf(a, a, -(1 + 2^-11)) keeps the exact 2^-24.
    assert lib.oracle_block_score(q2, k2, 2) == 2.0 ** -24


def _brute(scores, topk, n_text, local=None):
    BH, nqb, nkb = scores.shape
    mask = torch.zeros(BH, nqb, nkb, dtype=torch.uint8)
    for bh in range(BH):
        for r in range(nqb):
            order = sorted(range(nkb), key=lambda c: (-scores[bh, r, c].item(), c))
            for c in order[:topk]:
                mask[bh, r, c] = 1
            mask[bh, r, :n_text] = 1
            if r < n_text:
                mask[bh, r, :] = 1
            if local is not None:
                mask[bh, r] |= local[r]
    return mask


def test_topk_brute_force_with_ties_and_local():
    g = torch.Generator().manual_seed(2)
    scores = torch.randint(0, 6, (3, 9, 13), generator=g).float()  # many ties
    local = (torch.rand(9, 13, generator=g) < 0.2).to(torch.uint8)
    for topk in (0, 1, 4, 13, 20):
        idx, cnt, mask, _ = native.block_topk(None, None, topk, 2, local=local, scores_in=scores)
        want = _brute(scores, topk, 2, local)
        assert torch.equal(mask.reshape(3, 9, 13), want)
        for r in range(27):
            assert torch.equal(idx[r, : cnt[r]], torch.nonzero(want.reshape(27, 13)[r]).flatten().int())


def test_topk_matches_torch_topk_without_ties():
    # The reference rule (torch.topk + scatter, block_sparse_attn_kernel.py:31-39) on
    # tie-free scores, with no text forcing.
    g = torch.Generator().manual_seed(3)
    scores = torch.randn(4, 20, 278, generator=g)
    _, _, mask, _ = native.block_topk(None, None, 55, 0, scores_in=scores)
    ref = torch.zeros(4, 20, 278, dtype=torch.bool)
    ref.scatter_(-1, torch.topk(scores, 55, dim=-1).indices, True)
    assert torch.equal(mask.reshape(4, 20, 278).bool(), ref)


def test_topk_special_cases():
    s = torch.zeros(1, 3, 6)
    idx, cnt, mask, _ = native.block_topk(None, None, 2, 0, scores_in=s)
    assert torch.equal(mask.reshape(3, 6)[:, :2].sum(), torch.tensor(6)) and mask.sum() == 6  # all ties -> lowest
    s = torch.tensor([[[0.0, -0.0, 1.0]]])
    _, _, mask, _ = native.block_topk(None, None, 2, 0, scores_in=s)
    assert mask.flatten().tolist() == [1, 0, 1]  # +0 ranks above -0 (bit-pattern order)
    s = torch.tensor([[[float("nan"), 5.0, float("inf")]]])
    _, _, mask, _ = native.block_topk(None, None, 1, 0, scores_in=s)
    assert mask.flatten().tolist() == [1, 0, 0]  # positive NaN ranks first


def test_pooled_scores_match_fp64():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 2, 640, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 640, 64, generator=g).to(torch.bfloat16)
    qp, kp = native.block_pool(q), native.block_pool(k)
    _, _, _, scores = native.block_topk(qp, kp, 3, 0)
    want = torch.einsum("brd,bcd->brc", qp.double(), kp.double())
    assert torch.allclose(scores.reshape(2, 10, 10).double(), want, atol=1e-5)
