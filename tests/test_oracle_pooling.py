"""Pins the pooled-attention oracle (oracle/pooling.py) with closed forms, a brute force and SDPA."""
import math

import pytest
import torch

from oracle.pooling import pooled_attention


@pytest.mark.parametrize("L,bs", [(200, 64), (96, 32), (300, 128)])
def test_uniform_attention_closed_form(L, bs):
    # q = 0: P = 1/L everywhere, every block's maximum is 1/L, so every Po row is 1/nd.
    g = torch.Generator().manual_seed(1)
    q = torch.zeros(1, 2, L, 16, dtype=torch.float64)
    k, v = torch.randn(1, 2, L, 16, generator=g), torch.randn(1, 2, L, 16, generator=g)
    out, po = pooled_attention(q, k, v, False, 0.25, bs)
    nd = math.ceil(L / bs)
    assert torch.allclose(po, torch.full_like(po, 1 / nd), atol=1e-14)
    assert torch.allclose(out, v.double().mean(dim=2, keepdim=True).expand_as(out), atol=1e-12)


@pytest.mark.parametrize("L,bs", [(200, 64), (96, 32), (300, 128)])
def test_uniform_causal_closed_form(L, bs):
    # q = 0, causal: P[r][c] = 1/(r+1) for c <= r. The largest entry of block (i, j <= i) is
    # 1/(i*bs + 1) (first row of block i), so row i of Po is 1/(i+1) on j <= i and 0 beyond.
    g = torch.Generator().manual_seed(2)
    q = torch.zeros(1, 1, L, 16, dtype=torch.float64)
    k, v = torch.randn(1, 1, L, 16, generator=g), torch.randn(1, 1, L, 16, generator=g)
    _, po = pooled_attention(q, k, v, True, 0.25, bs)
    nd = math.ceil(L / bs)
    want = torch.zeros(nd, nd, dtype=torch.float64)
    for i in range(nd):
        want[i, : i + 1] = 1 / (i + 1)
    assert torch.allclose(po[0, 0], want, atol=1e-14)


@pytest.mark.parametrize("causal", [False, True])
def test_brute_force_tiny(causal):
    # Explicit loops: per row, exp of the scaled scores (max-subtracted), block maxima of the
    # probabilities, then row normalisation. Two query heads share one key head.
    B, H, Hk, L, D, bs = 1, 2, 1, 70, 4, 32
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, n, L, D, generator=g, dtype=torch.float64) for n in (H, Hk, Hk))
    scale = 0.7
    out, po = pooled_attention(q, k, v, causal, scale, bs)
    nd = math.ceil(L / bs)
    for h in range(H):
        P = [[0.0] * L for _ in range(L)]
        for r in range(L):
            keys = range(r + 1) if causal else range(L)
            sc = {c: sum(q[0, h, r, d].item() * k[0, 0, c, d].item() for d in range(D)) * scale for c in keys}
            mx = max(sc.values())
            z = sum(math.exp(x - mx) for x in sc.values())
            for c, x in sc.items():
                P[r][c] = math.exp(x - mx) / z
            o = [sum(P[r][c] * v[0, 0, c, d].item() for c in range(L)) for d in range(D)]
            assert max(abs(o[d] - out[0, h, r, d].item()) for d in range(D)) < 1e-12
        for i in range(nd):
            row = []
            for j in range(nd):
                row.append(max(P[r][c] for r in range(i * bs, min(L, i * bs + bs))
                               for c in range(j * bs, min(L, j * bs + bs))))
            s = sum(row)
            for j in range(nd):
                assert abs(po[0, h, i, j].item() - row[j] / s) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_out_matches_sdpa(causal):
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 3, 150, 32, generator=g, dtype=torch.float64) for _ in range(3))
    out, _ = pooled_attention(q, k, v, causal, 1 / math.sqrt(32), 64)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)
    assert torch.allclose(out, want, atol=1e-12)
