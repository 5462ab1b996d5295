"""Pins of oracle/backup.py (the frame-factored block mask of the backup path): pure-Python
brute force on tiny geometries, uniform-attention closed forms, and the row-sum invariant."""
import math

import torch

from oracle import backup


def test_kron_mask_brute_force():
    g = torch.Generator().manual_seed(0)
    frame = torch.rand(2, 3, 4, 4, generator=g) < 0.5
    inner = torch.rand(2, 3, 3, 2, generator=g) < 0.6
    got = backup.kron_mask(inner, frame, pad=2)
    assert got.shape == (2, 3, 4 * 3 + 2, 4 * 2 + 2) and got.dtype == torch.float32
    for b in range(2):
        for h in range(3):
            for i in range(14):
                for j in range(10):
                    if i >= 12 or j >= 8:
                        want = 1.0
                    else:
                        want = float(bool(frame[b, h, i // 3, j // 2]) and bool(inner[b, h, i % 3, j % 2]))
                    assert got[b, h, i, j].item() == want, (b, h, i, j)


def _brute_softmax_rows(qr, kr, scale, bias_cols=0, bias=0.0):
    out = []
    for qv in qr:
        s = [sum(float(a) * float(c) for a, c in zip(qv, kv)) * scale + (bias if j < bias_cols else 0.0)
             for j, kv in enumerate(kr)]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        out.append([x / z for x in e])
    return out


def test_frame_scope_map_brute_force_tiny():
    T, f, S, ns, d = 3, 3, 5, 2, 4
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 1, T + f * S, d, generator=g)
    k = torch.randn(1, 1, T + f * S, d, generator=g)
    draws = torch.tensor([4, 1])
    got = backup.frame_scope_map(q, k, draws, T, f, S, ns, scale=0.5)
    idx = [0, 1, 2] + [T + fr * S + int(x) for fr in range(f) for x in draws]
    P = _brute_softmax_rows([q[0, 0, i].tolist() for i in idx], [k[0, 0, i].tolist() for i in idx], 0.5,
                            bias_cols=T, bias=backup.composition(ns, S))
    for f1 in range(f):
        for f2 in range(f):
            want = sum(P[T + f1 * ns + s1][T + f2 * ns + s2] for s1 in range(ns) for s2 in range(ns)) / ns
            assert abs(got[0, 0, f1, f2].item() - want) < 1e-12


def test_frame_scope_map_uniform_closed_form():
    # q = 0: every sampled row spreads its mass over the text keys (weight ns/S each, the bias
    # is log(ns/S) up to bf16 rounding) and the f*ns sampled keys (weight 1 each), so every
    # entry of the map is ns / (T * e^c + f * ns).
    T, f, S, ns = 226, 13, 1350, 60
    q = torch.zeros(1, 2, T + f * S, 64)
    k = torch.randn(1, 2, T + f * S, 64, generator=torch.Generator().manual_seed(2))
    got = backup.frame_scope_map(q, k, torch.arange(ns) * 7, T, f, S, ns)
    c = backup.composition(ns, S)
    want = ns / (T * math.exp(c) + f * ns)
    assert torch.allclose(got, torch.full_like(got, want), rtol=0, atol=1e-12)
    assert abs(c - math.log(ns / S)) <= 2 ** -7  # bf16 rounding of log(60/1350): half an ulp at 3.1


def test_inner_cell_sums_brute_force_and_invariants():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 14, 4, generator=g)
    k = torch.randn(1, 2, 14, 4, generator=g)
    got = backup.inner_cell_sums(q, k, original_length=10, stride=4)  # q_len 12, k_len 8
    assert got.shape == (1, 2, 3, 2)
    for h in range(2):
        P = _brute_softmax_rows(q[0, h, :12].tolist(), k[0, h, :8].tolist(), 1 / 8)
        for i in range(3):
            for j in range(2):
                want = sum(P[4 * i + a][4 * j + c] for a in range(4) for c in range(4))
                assert abs(got[0, h, i, j].item() - want) < 1e-12
    # every query row sums to one: each block row of cells sums to the rows in the block
    assert torch.allclose(got.sum(-1), torch.full((1, 2, 3), 4.0, dtype=torch.float64), atol=1e-12)
    # uniform attention (q = 0): every full cell holds stride * stride / k_len
    z = backup.inner_cell_sums(torch.zeros(1, 1, 1408, 64), k.new_zeros(1, 1, 1350, 64).normal_(generator=g))
    assert z.shape == (1, 1, 22, 21)
    assert torch.allclose(z, torch.full_like(z, 64 * 64 / 1344), atol=1e-10)
