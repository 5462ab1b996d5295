"""Matching metrics built to separate summation orders of the ToMe src . dst scores (shared by
the CPU check that they do and the GPU test that the matching kernels agree on them)."""
import torch


def adversarial_metric(kind, a, b, G, N, C=64, seed=0):
    """fp32 [G, N, C] metrics that separate summation orders of the src . dst scores: each
    score is an fmaf chain over the C channels, which match_mfma_kernel issues as 16 chained
    v_mfma_f32_16x16x4_f32 (four channels per step) and match_kernel as scalar fmaf."""
    g = torch.Generator().manual_seed(seed)
    shape = (G, N, C)
    sign = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0)
    mant = 1 + torch.rand(shape, generator=g)
    if kind == "exponents":  # operand exponents over [-56, 56]: partial sums absorb each other
        return sign * mant * torch.exp2(torch.randint(-56, 57, shape, generator=g).float())
    if kind == "subnormal":
        # operands in [2^-78, 2^-66): products, partial sums and most best scores in fp32's
        # subnormal range (< 2^-126); a quarter of the src rows carry one channel of 2^-40,
        # whose scores are normal
        x = sign * mant * torch.exp2(torch.randint(-78, -67, shape, generator=g).float())
        src = a.cpu().long()
        big = torch.zeros(G, N, dtype=torch.bool)
        big[:, src] = torch.rand(G, src.numel(), generator=g) < 0.25
        x[..., 5] = torch.where(big, sign[..., 5] * 2.0 ** -40, x[..., 5])
        return x
    if kind == "cancel":
        # src rows (u, u(1+e)) and dst rows (w, -w(1+d)) on interleaved channel pairs: each
        # pair of products nearly cancels, so every step of the chain rounds a large partial
        u = torch.randn(G, N, C // 2, generator=g) * 4
        e = torch.randn(G, N, C // 2, generator=g) * 2.0 ** -12
        x = torch.empty(shape)
        x[..., 0::2] = u
        x[..., 1::2] = u * (1 + e)
        dst = b.cpu().long()
        x[:, dst, 1::2] = -x[:, dst, 1::2]
        return x
    if kind == "ties":
        # duplicated dst rows (argmax ties: the lower dst wins), duplicated src rows (equal
        # node_max: the edge order keeps the lower src), zero rows (every score 0)
        x = torch.randn(shape, generator=g).round()  # small integers: many exactly equal scores
        src, dst = a.cpu().long(), b.cpu().long()
        x[:, dst[1::2]] = x[:, dst[0:-1:2]]
        x[:, src[1::3]] = x[:, src[0:-1:3]]
        x[:, src[::7]] = 0
        return x
    raise ValueError(kind)
