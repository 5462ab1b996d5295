"""Pins the CPU attention oracle (oracle/attention.py) against independent checks."""
import math

import pytest
import torch

from oracle.attention import expand_block_mask, flops_of_mask, masked_attention


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64)


def test_all_ones_mask_equals_library_sdpa():
    # Reference invariant: an all-ones block mask is dense attention (block_sparse_attn_kernel.py:315).
    q, k, v = (_rand((1, 3, 257, 64), s) for s in range(3))
    mask = torch.ones(1, 3, 5, 5, dtype=torch.bool)
    got = masked_attention(q, k, v, mask, 0.125)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.125)
    assert torch.allclose(got, want, atol=1e-12, rtol=1e-10)


def test_brute_force_tiny():
    # Pure-Python softmax over explicitly enumerated allowed keys (block = 2 tokens).
    q, k, v = _rand((1, 1, 5, 3), 3), _rand((1, 1, 7, 3), 4), _rand((1, 1, 7, 3), 5)
    mask = torch.tensor([[1, 0, 1, 0], [0, 1, 0, 1], [1, 1, 0, 0]], dtype=torch.bool)[None, None]
    got = masked_attention(q, k, v, mask, 0.7, block=2)
    for i in range(5):
        keys = [j for j in range(7) if mask[0, 0, i // 2, j // 2]]
        s = [0.7 * sum(q[0, 0, i, d].item() * k[0, 0, j, d].item() for d in range(3)) for j in keys]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        z = sum(w)
        for d in range(3):
            o = sum(w[t] * v[0, 0, keys[t], d].item() for t in range(len(keys))) / z
            assert abs(got[0, 0, i, d].item() - o) < 1e-12


def test_single_allowed_key_returns_its_value():
    # Closed form: if only the last (partial) block with a single valid key is allowed,
    # every row returns that key's value regardless of the scores.
    q, k, v = _rand((1, 2, 64, 64), 6), _rand((1, 2, 129, 64), 7), _rand((1, 2, 129, 64), 8)
    mask = torch.zeros(1, 2, 1, 3, dtype=torch.bool)
    mask[..., 2] = True
    got = masked_attention(q, k, v, mask, 0.125)
    assert torch.allclose(got, v[:, :, 128:129, :].expand_as(got), atol=1e-14)


def test_identical_keys_give_block_mean_of_values():
    q = _rand((1, 1, 64, 64), 9)
    k = _rand((1, 1, 1, 64), 10).expand(1, 1, 128, 64).clone()
    v = _rand((1, 1, 128, 64), 11)
    mask = torch.tensor([[[[True, False]]]])
    got = masked_attention(q, k, v, mask, 0.3)
    assert torch.allclose(got, v[:, :, :64].mean(dim=2, keepdim=True).expand_as(got), atol=1e-13)


def test_key_block_order_and_empty_rows():
    q, k, v = _rand((2, 2, 200, 64), 12), _rand((2, 2, 300, 64), 13), _rand((2, 2, 300, 64), 14)
    g = torch.Generator().manual_seed(15)
    mask = torch.rand(2, 2, 4, 5, generator=g) < 0.5
    mask[0, 1, 2] = False  # an empty row
    base = masked_attention(q, k, v, mask, 0.125)
    assert torch.all(base[0, 1, 128:192] == 0)
    # Permuting key blocks (full blocks only) together with the mask columns changes nothing.
    perm = torch.tensor([3, 1, 0, 2])
    kp = torch.cat([k[:, :, 64 * p:64 * p + 64] for p in perm] + [k[:, :, 256:]], dim=2)
    vp = torch.cat([v[:, :, 64 * p:64 * p + 64] for p in perm] + [v[:, :, 256:]], dim=2)
    mp = torch.cat([mask[..., perm], mask[..., 4:]], dim=-1)
    assert torch.allclose(masked_attention(q, kp, vp, mp, 0.125), base, atol=1e-12)


def test_key_bias_matches_sdpa_attn_mask():
    q, k, v = (_rand((1, 2, 100, 64), s) for s in (16, 17, 18))
    bias = torch.log(torch.arange(1, 101, dtype=torch.float64)).reshape(1, 1, 100).expand(1, 2, 100)
    got = masked_attention(q, k, v, torch.ones(1, 1, 2, 2, dtype=torch.bool), 0.125, key_bias=bias)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=bias[:, :, None, :], scale=0.125)
    assert torch.allclose(got, want, atol=1e-12)


def test_expand_and_flops():
    m = torch.tensor([[[[1, 0], [1, 1]]]], dtype=torch.bool)
    e = expand_block_mask(m, 70, 100)
    assert e.shape == (1, 1, 70, 100)
    assert e[0, 0, :64, :64].all() and not e[0, 0, :64, 64:].any() and e[0, 0, 64:, :].all()
    # 64x64 + 6x64 + 6x36 valid pairs
    assert flops_of_mask(m, 70, 100) == 4 * 64 * (64 * 64 + 6 * 64 + 6 * 36)


@pytest.mark.parametrize("L", [257])
def test_partial_last_block_masks_tail(L):
    # Keys past L in the last block must not contribute (kernel :87-89).
    q, k, v = (_rand((1, 1, L, 64), s) for s in (19, 20, 21))
    m = torch.ones(1, 1, 5, 5, dtype=torch.bool)
    got = masked_attention(q, k, v, m, 0.125)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.125)
    assert torch.allclose(got, want, atol=1e-12)


def test_row_subset_equals_full_rows():
    # `rows=` computes the selected query rows as the full call does (to fp64 rounding: the
    # matmul's summation order depends on the chunk shape), including rows of different
    # blocks, an empty block row, a key bias and a token mask.
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 2, 300, 64, generator=g) for _ in range(3))
    bm = torch.rand(1, 2, 5, 5, generator=g) < 0.5
    bm[0, 1, 2] = False
    bias = torch.randn(1, 2, 300, generator=g)
    tm = lambda r: (r[:, None] + torch.arange(300)[None, :]) % 3 != 0
    rows = torch.tensor([0, 1, 63, 64, 130, 150, 255, 299])
    full = masked_attention(q, k, v, bm, 0.125, key_bias=bias, token_mask=tm)
    part = masked_attention(q, k, v, bm, 0.125, key_bias=bias, token_mask=tm, rows=rows, row_chunk=3)
    assert part.shape == (1, 2, rows.numel(), 64)
    assert torch.allclose(part, full[:, :, rows], rtol=0, atol=1e-12)
    assert torch.all(part[0, 1, 4:6] == 0)  # rows 130 and 150 sit in the empty block row
