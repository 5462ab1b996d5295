"""Pins the token-merging oracle (oracle/sa_oracle.c) on the CPU."""
import numpy as np
import pytest
import torch

from oracle import native


def _reference_partition(T, Hp, Wp, sx, sy, st, choice=None):
    """numpy restatement of merge_unmerge.py:62-92 (stable argsort of the {-1, 0} buffer)."""
    t = T - 1
    hsy, wsx, tst = Hp // sy, Wp // sx, t // st
    rand_idx = np.zeros((tst, hsy, wsx, 1), dtype=np.int64) if choice is None else choice.numpy().reshape(tst, hsy, wsx, 1)
    view = np.zeros((tst, hsy, wsx, st * sy * sx), dtype=np.int64)
    np.put_along_axis(view, rand_idx, -1, axis=3)
    view = view.reshape(tst, hsy, wsx, st, sy, sx).transpose(0, 3, 1, 4, 2, 5).reshape(tst * st, hsy * sy, wsx * sx)
    buf = np.zeros((t, Hp, Wp), dtype=np.int64)
    buf[: tst * st, : hsy * sy, : wsx * sx] = view
    order = np.argsort(buf.reshape(-1), kind="stable") + Wp * Hp
    num_dst = tst * hsy * wsx
    a = order[num_dst:]
    b = np.concatenate([np.arange(Hp * Wp), order[:num_dst]])
    return a, b


@pytest.mark.parametrize("geo", [(13, 30, 45, 2, 2, 1), (13, 30, 45, 3, 3, 4), (4, 5, 7, 2, 3, 2), (1, 3, 3, 1, 1, 1)])
def test_partition_matches_reference_restatement(geo):
    a, b = native.tome_partition(*geo)
    ra, rb = _reference_partition(*geo)
    assert np.array_equal(a.numpy(), ra) and np.array_equal(b.numpy(), rb)
    N = geo[0] * geo[1] * geo[2]
    assert sorted(a.tolist() + b.tolist()) == list(range(N))


def test_partition_counts_of_the_configs():
    a, b = native.tome_partition(13, 30, 45, 2, 2, 1)
    assert (a.numel(), b.numel()) == (12240, 5310)      # config 4
    a, b = native.tome_partition(13, 30, 45, 3, 3, 4)
    assert b.numel() == 1800                              # reference default (MergeAttention.py:16)


def test_partition_random_choice():
    g = torch.Generator().manual_seed(0)
    choice = torch.randint(0, 2 * 3 * 2, (2, 2, 3), generator=g, dtype=torch.int32)
    a, b = native.tome_partition(5, 6, 7, 2, 3, 2, choice)
    ra, rb = _reference_partition(5, 6, 7, 2, 3, 2, choice)
    assert np.array_equal(a.numpy(), ra) and np.array_equal(b.numpy(), rb)


def _qkv(B, H, L, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, H, L, 64, generator=g).to(torch.bfloat16) for _ in range(3))


def test_metric_against_fp64():
    k, v, _ = _qkv(2, 3, 40, 1)
    m0 = native.tome_metric(k, None, 10, 0)
    ref = k.double()[:, :, 10:].sum(1)
    ref = ref / ref.norm(dim=-1, keepdim=True)
    assert torch.allclose(m0.double(), ref, atol=1e-6)
    m1 = native.tome_metric(k, v, 10, 1)
    kk, vv = k.double()[:, :, 10:], v.double()[:, :, 10:]
    cat = torch.cat([kk, kk.norm(dim=-1, keepdim=True), vv, vv.norm(dim=-1, keepdim=True)], -1)
    cat = cat / cat.norm(dim=-1, keepdim=True)
    assert torch.allclose(m1.double(), cat.reshape(6, 30, 130), atol=1e-6)


def test_match_brute_force_and_ties():
    g = torch.Generator().manual_seed(2)
    G, N, C = 2, 60, 8
    metric = torch.randn(G, N, C, generator=g)
    metric = metric / metric.norm(dim=-1, keepdim=True)
    a_idx = torch.arange(0, N, 2, dtype=torch.int32)
    b_idx = torch.arange(1, N, 2, dtype=torch.int32)
    b_list = b_idx.tolist()
    # duplicate dst vectors: the argmax tie must go to the lower dst position
    metric[:, b_list[7]] = metric[:, b_list[3]]
    r = 12
    maps = native.tome_match(metric, a_idx, b_idx, r, 5)
    for gi in range(G):
        s = metric[gi, a_idx.long()].double() @ metric[gi, b_idx.long()].double().T
        best = s.max(-1)
        for i in range(a_idx.numel()):
            top = s[i].topk(2).values
            if top[0] - top[1] > 1e-5:  # decision margin well above fp32 rounding
                assert maps["node_idx"][gi, i].item() == best.indices[i].item()
        assert not (maps["node_idx"][gi] == 7).any()  # dst 7 duplicates dst 3 -> never wins
        # edge order: stable sort of node_max descending
        nm = maps["node_max"][gi].numpy()
        assert np.array_equal(maps["edge"][gi].numpy(), np.argsort(-nm, kind="stable"))
        assert torch.equal(maps["dst_idx"][gi], maps["node_idx"][gi][maps["edge"][gi][:r].long()])
        assert maps["dst_cnt"][gi].sum().item() == r


def test_maps_and_merge_invariants():
    T, Hp, Wp, text = 4, 6, 8, 10
    a_idx, b_idx = native.tome_partition(T, Hp, Wp, 2, 2, 1)
    B, H = 2, 3
    N = T * Hp * Wp
    L = text + N
    k, v, q = _qkv(B, H, L, 3)
    metric = native.tome_metric(k, None, text, 0)
    for r in (0, 20, a_idx.numel()):
        maps = native.tome_match(metric, a_idx, b_idx, r, text)
        U = a_idx.numel() - r
        for g in range(B):
            sizes = 1 + maps["dst_cnt"][g]
            assert U + sizes.sum().item() == N
            rot = maps["row_of_token"][g]
            assert torch.equal(rot[:text], torch.arange(text, dtype=torch.int32))
            assert rot.max().item() == L - r - 1 and rot.min().item() == 0
        # a constant tensor merges to the same constant; unmerge(merge(x)) restores it
        c = torch.full((B, H, L, 64), 0.375, dtype=torch.bfloat16)
        mc = native.tome_merge(c, maps, a_idx, b_idx, r, text, H)
        assert torch.equal(mc, torch.full_like(mc, 0.375))
        assert torch.equal(native.tome_unmerge(mc, maps, H), c)
        # merged rows are fp32 means of their members (checked in fp64 within bf16 rounding)
        mq = native.tome_merge(q, maps, a_idx, b_idx, r, text, H)
        back = native.tome_unmerge(mq, maps, H)
        for g in range(B):
            rot = maps["row_of_token"][g].long()
            for row in range(L - r):
                toks = (rot == row).nonzero().flatten()
                mean = q[g, :, toks].double().mean(1)
                assert torch.allclose(mq[g, :, row].double(), mean, atol=1e-2, rtol=8e-3)
                if toks.numel() == 1:
                    assert torch.equal(mq[g, :, row], q[g, :, toks[0]])
            assert torch.equal(back[g], mq[g][:, rot])
    # r = 0 is a pure permutation (merge_unmerge.py:56-57 returns identity closures)
    maps = native.tome_match(metric, a_idx, b_idx, 0, text)
    assert torch.equal(native.tome_unmerge(native.tome_merge(q, maps, a_idx, b_idx, 0, text, H), maps, H), q)


def test_key_bias_is_bf16_log_of_sizes():
    a_idx, b_idx = native.tome_partition(3, 4, 4, 2, 2, 1)
    k, _, _ = _qkv(1, 2, 5 + 48, 4)
    maps = native.tome_match(native.tome_metric(k, None, 5, 0), a_idx, b_idx, 10, 5)
    U = a_idx.numel() - 10
    kb = maps["key_bias"][0]
    assert torch.all(kb[: 5 + U] == 0)
    want = torch.log((1 + maps["dst_cnt"][0]).float().to(torch.bfloat16)).to(torch.bfloat16).float()
    assert torch.equal(kb[5 + U:], want)


def test_library_partition_matches_oracle():
    from sparseattnfunctions_amd import _tome
    for geo in [(13, 30, 45, 2, 2, 1), (13, 30, 45, 3, 3, 4), (4, 5, 7, 2, 3, 2)]:
        a, b = _tome.partition(*geo, device="cpu")
        oa, ob = native.tome_partition(*geo)
        assert torch.equal(a, oa) and torch.equal(b, ob)


def _chain_node_max(metric, a_idx, b_idx, order, ftz=False):
    """Best score per src with the C channels added in `order` (fp64 product and sum, rounded
    to fp32 after each step: an fmaf chain up to rare double roundings). `ftz` flushes
    subnormal fp32 results to zero after each step."""
    out = []
    for gi in range(metric.shape[0]):
        A = metric[gi, a_idx.long()].numpy().astype(np.float64)
        B = metric[gi, b_idx.long()].numpy().astype(np.float64)
        acc = np.zeros((A.shape[0], B.shape[0]), dtype=np.float32)
        for c in order:
            acc = (acc.astype(np.float64) + A[:, c:c + 1] * B[None, :, c]).astype(np.float32)
            if ftz:
                acc[np.abs(acc) < np.float32(2.0 ** -126)] = 0
        out.append(acc.max(-1))
    return np.stack(out)


@pytest.mark.parametrize("kind", ["exponents", "cancel"])
def test_adversarial_metrics_separate_summation_orders(kind):
    # The metrics of the GPU test of the matching kernels can tell an in-order fmaf chain over
    # the channels from the reverse order and from a four-wide interleaved order: the best
    # score of some src differs between them.
    from tome_adversarial import adversarial_metric
    T, Hp, Wp = 6, 12, 20
    a, b = native.tome_partition(T, Hp, Wp, 2, 2, 1)
    x = adversarial_metric(kind, a, b, 2, T * Hp * Wp)
    assert torch.isfinite(x).all()
    maps = native.tome_match(x, a, b, a.numel(), 226)
    fwd = _chain_node_max(x, a, b, range(64))
    # the emulation follows the oracle's in-order chain
    assert (fwd == maps["node_max"].numpy()).mean() > 0.99
    rev = _chain_node_max(x, a, b, range(63, -1, -1))
    assert (rev != maps["node_max"].numpy()).mean() > 0.01
    # four interleaved chains over channels c = 4j + i, then added in i order
    g4 = _chain_node_max(x, a, b, [c for i in range(4) for c in range(i, 64, 4)])
    assert (g4 != maps["node_max"].numpy()).mean() > 0.01


def test_adversarial_subnormal_metric_needs_subnormals():
    # In the subnormal metric most best scores are subnormal fp32 values (sums on the uniform
    # 2^-149 grid, where the order of additions does not matter), and flushing subnormal
    # results to zero at each step changes them: it tells a chain that keeps subnormals from
    # one that flushes them.
    from tome_adversarial import adversarial_metric
    T, Hp, Wp = 6, 12, 20
    a, b = native.tome_partition(T, Hp, Wp, 2, 2, 1)
    x = adversarial_metric("subnormal", a, b, 2, T * Hp * Wp)
    maps = native.tome_match(x, a, b, a.numel(), 226)
    nm = maps["node_max"].abs()
    assert ((nm > 0) & (nm < 2.0 ** -126)).float().mean() > 0.5
    assert (_chain_node_max(x, a, b, range(64)) == maps["node_max"].numpy()).mean() > 0.99
    ftz = _chain_node_max(x, a, b, range(64), ftz=True)
    assert (ftz != maps["node_max"].numpy()).mean() > 0.5


def test_adversarial_ties_are_ties():
    # The ties metric has exactly equal best scores (small integers: exact sums) on several dst
    # per src, and equal node_max across srcs; the oracle keeps the lower dst and src.
    from tome_adversarial import adversarial_metric
    T, Hp, Wp = 6, 12, 20
    a, b = native.tome_partition(T, Hp, Wp, 2, 2, 1)
    x = adversarial_metric("ties", a, b, 2, T * Hp * Wp)
    maps = native.tome_match(x, a, b, a.numel(), 226)
    for gi in range(2):
        s = x[gi, a.long()].double() @ x[gi, b.long()].double().T
        best = s.max(-1).values
        n_best = (s == best[:, None]).sum(-1)
        assert (n_best > 1).sum() > 50
        first = (s == best[:, None]).float().argmax(-1)
        assert torch.equal(maps["node_idx"][gi].long(), first)
        assert torch.equal(maps["node_max"][gi].double(), best)
        nm = maps["node_max"][gi].numpy()
        assert len(np.unique(nm)) < nm.size // 2
        assert np.array_equal(maps["edge"][gi].numpy(), np.argsort(-nm, kind="stable"))
