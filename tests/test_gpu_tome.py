"""GPU parity of token merging: metric, matching maps, merge and unmerge bit-exact against
the C oracle; MergeAttention outputs within the bf16 tolerances of the fp64 oracle."""
import math

import numpy as np
import pytest
import torch

from conftest import case
from tome_adversarial import adversarial_metric
from oracle import native
from oracle.attention import masked_attention
from sparseattnfunctions_amd import _tome
from sparseattnfunctions_amd.MergeAttention import REFERENCE_MERGE_CONFIG, MergeAttention
from sparseattnfunctions_amd.utils import merge_unmerge
from sparseattnfunctions_amd.workloads import Geometry, cogvideox_qkv

pytestmark = pytest.mark.gpu


def _check(got, want):
    err = (got.float().cpu().double() - want).abs()
    assert torch.isfinite(got.float()).all()
    assert err.max().item() <= 2e-2, err.max().item()
    assert err.mean().item() <= 2e-3, err.mean().item()


def _maps_equal(maps, want, fields=("node_idx", "node_max", "edge", "dst_idx", "dst_cnt", "row_of_token", "key_bias")):
    for f in fields:
        got = getattr(maps, f).cpu()
        if f in ("node_idx", "node_max", "edge"):
            got = got[:, : maps.n_src]
        if f == "dst_idx":
            got = got[:, : maps.r]
        assert torch.equal(got, want[f]), f


def _check_members(maps):
    # CSR members: for each dst, its merged srcs in ascending edge order.
    ptr, mem, dst = maps.dst_ptr.cpu(), maps.members.cpu(), maps.dst_idx.cpu()
    for g in range(maps.G):
        assert torch.equal(ptr[g, 1:] - ptr[g, :-1], maps.dst_cnt.cpu()[g])
        for d in range(0, maps.n_dst, max(1, maps.n_dst // 50)):
            seg = mem[g, ptr[g, d]:ptr[g, d + 1]]
            want = (dst[g, : maps.r] == d).nonzero().flatten().int()
            assert torch.equal(seg, want)


@pytest.mark.parametrize("mode", [0, 1])
def test_small_pipeline_bit_exact(dev, mode):
    case(f"tome small mode={mode}")
    geom = Geometry(text_len=226, T=4, Hp=6, Wp=10)
    q, k, v = cogvideox_qkv(5, B=2, H=3, geom=geom)
    metric = _tome.metric_from_qkv(k.to(dev), v.to(dev), geom.text_len, mode)
    om = native.tome_metric(k, v, geom.text_len, mode)
    assert torch.equal(metric.cpu(), om)
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    oa, ob = native.tome_partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1)
    for r in (0, 37, oa.numel()):
        maps = _tome.match(metric, a, b, r, geom.text_len)
        want = native.tome_match(om, oa, ob, r, geom.text_len)
        _maps_equal(maps, want)
        _check_members(maps)
        hpg = 3 if mode == 0 else 1
        for x in (q, k, v):
            xm = _tome.merge(x.to(dev), maps, hpg)
            assert torch.equal(xm.cpu(), native.tome_merge(x, want, oa, ob, r, geom.text_len, hpg))
            assert torch.equal(_tome.unmerge(xm, maps, hpg).cpu(), native.tome_unmerge(xm.cpu(), want, hpg))


def test_crowded_dsts_bit_exact(dev):
    # Every src row equals one of two unit vectors u, w and every dst row is u except one
    # that is w: all u-srcs pick the first dst (ties go to the lowest index), all w-srcs the
    # w dst. With every src merged, one dst holds 7 860 members (more than 1 024: the member
    # sort's serial path) and the other 300 (several 64-member chunks).
    case("tome crowded dsts")
    geom = Geometry(text_len=226, T=9, Hp=30, Wp=45)
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    oa, ob = native.tome_partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1)
    n_video = geom.T * geom.Hp * geom.Wp
    g = torch.Generator().manual_seed(11)
    u, w = torch.randn(2, 64, generator=g)
    u, w = u / u.norm(), w / w.norm()
    metric = u.repeat(1, n_video, 1)  # [1, N, 64]
    w_src = oa[torch.randperm(oa.numel(), generator=g)[:300]].long()
    metric[0, w_src] = w
    metric[0, ob[5].long()] = w
    r = oa.numel()
    maps = _tome.match(metric.to(dev), a, b, r, geom.text_len)
    want = native.tome_match(metric, oa, ob, r, geom.text_len)
    _maps_equal(maps, want)
    cnt = maps.dst_cnt.cpu()[0]
    assert cnt[0].item() == oa.numel() - 300 and cnt[5].item() == 300
    ptr, mem, dst = maps.dst_ptr.cpu(), maps.members.cpu(), maps.dst_idx.cpu()
    for d in (0, 5):
        seg = mem[0, ptr[0, d]:ptr[0, d + 1]]
        assert torch.equal(seg, (dst[0, :r] == d).nonzero().flatten().int()), d
    q = cogvideox_qkv(6, B=1, H=1, geom=geom)[0]
    xm = _tome.merge(q.to(dev), maps, 1)
    assert torch.equal(xm.cpu(), native.tome_merge(q, want, oa, ob, r, geom.text_len, 1))


def _misaligned(x):
    """A copy of x whose base is 4 bytes past a 16-byte boundary (contiguous)."""
    buf = torch.empty(x.numel() + 4, dtype=x.dtype, device=x.device)
    y = buf[1: 1 + x.numel()].view(x.shape)
    y.copy_(x)
    assert y.is_contiguous() and y.data_ptr() % 16 == 4
    return y


@pytest.mark.parametrize("kind", ["exponents", "subnormal", "cancel", "ties"])
def test_match_kernels_adversarial_bit_exact(dev, kind):
    # The 64-channel matching runs on the matrix cores on the assumption that
    # v_mfma_f32_16x16x4_f32 adds its four products to the accumulator as an in-order fmaf
    # chain. On metrics built to separate summation orders, the MFMA path (aligned metric), the
    # VALU match_kernel (the same metric at a base that is not 16-byte aligned) and the C
    # oracle's fmaf chain must give the same maps bit for bit, scores included.
    geom = Geometry(text_len=226, T=6, Hp=12, Wp=20)
    G, N = 2, geom.n_video
    case(f"tome match adversarial metric: {kind}")
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    oa, ob = native.tome_partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1)
    x = adversarial_metric(kind, a, b, G, N)
    assert torch.isfinite(x).all()
    r = oa.numel()
    want = native.tome_match(x, oa, ob, r, geom.text_len)
    md = x.to(dev)
    assert md.data_ptr() % 16 == 0
    mfma = _tome.match(md, a, b, r, geom.text_len)
    valu = _tome.match(_misaligned(md), a, b, r, geom.text_len)
    torch.cuda.synchronize()
    _maps_equal(valu, want)
    _maps_equal(mfma, want)
    if kind == "subnormal":
        nm = want["node_max"].abs()
        assert ((nm > 0) & (nm < 2.0 ** -126)).any()  # subnormal scores were compared


def test_match_misaligned_metric(dev):
    # A metric whose base is not 16-byte aligned gives the same maps (C4-sized head-sum metric).
    case("tome match misaligned metric")
    geom = Geometry()
    _, k, _ = cogvideox_qkv(8, B=2, H=4, geom=geom)
    metric = _tome.metric_from_qkv(k.to(dev), None, geom.text_len, 0)
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    want = _tome.match(metric, a, b, 4000, geom.text_len)
    got = _tome.match(_misaligned(metric), a, b, 4000, geom.text_len)
    torch.cuda.synchronize()
    for f in ("node_idx", "node_max", "edge", "dst_idx", "dst_cnt", "row_of_token", "key_bias"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f


@pytest.fixture(scope="module")
def c4_oracle():
    """Config 4 inputs (seed 3) and every matching map computed by the C oracle alone: the
    metric, the partition, the argmax of all 12 240 srcs of both groups (no GPU output is
    involved), then the edge order and the merge/unmerge maps from that argmax."""
    q, k, v = cogvideox_qkv(3)
    om = native.tome_metric(k, None, 226, 0)
    oa, ob = native.tome_partition(13, 30, 45, 2, 2, 1)
    idx, mx = native.tome_argmax_all(om, oa, ob)
    want = native.tome_maps(mx, idx, 17550, oa, ob, 4000, 226)
    return dict(q=q, k=k, v=v, metric=om, a=oa, b=ob, maps=want)


def test_config4_maps_bit_exact(dev, c4_oracle):
    case("tome config 4 full shape maps")
    o = c4_oracle
    metric = _tome.metric_from_qkv(o["k"].to(dev), None, 226, 0)
    assert torch.equal(metric.cpu(), o["metric"])
    a, b = _tome.partition(13, 30, 45, 2, 2, 1, dev)
    assert (a.numel(), b.numel()) == (12240, 5310)
    assert torch.equal(a.cpu(), o["a"]) and torch.equal(b.cpu(), o["b"])
    maps = _tome.match(metric, a, b, 4000, 226)
    _maps_equal(maps, o["maps"])
    _check_members(maps)
    assert maps.Lm == 13776 and int(maps.sizes.sum(1)[0]) == 5310 + 4000
    # Merged q, k, v of every head bit-exact against the oracle's merge from its own maps.
    merged = _tome.merge_many([o[n].to(dev) for n in "qkv"], maps, 30)
    for n, xm in zip("qkv", merged):
        want = native.tome_merge(o[n], o["maps"], o["a"], o["b"], 4000, 226, 30)
        assert torch.equal(xm.cpu(), want), n
        assert torch.equal(_tome.merge(o[n].to(dev), maps, 30).cpu(), want), n
    back = _tome.unmerge(merged[2], maps, 30).cpu()
    assert torch.equal(back, native.tome_unmerge(merged[2].cpu(), o["maps"], 30))


def test_merge_attention_config4(dev, c4_oracle):
    case("MergeAttention config 4 end to end")
    o = c4_oracle
    q, k, v = o["q"], o["k"], o["v"]
    proc = MergeAttention()
    out = proc(q.to(dev), k.to(dev), v.to(dev)).cpu()
    want_maps = o["maps"]
    _maps_equal(proc.maps, want_maps)
    a, b = o["a"], o["b"]
    heads = [(0, 0), (0, 17), (1, 8), (1, 29)]
    for bb, hh in heads:
        sel = lambda x: x[bb:bb + 1, hh:hh + 1]
        sub = {f: t[bb:bb + 1] for f, t in want_maps.items()}
        qm, km, vm = (native.tome_merge(sel(x), sub, a, b, 4000, 226, 1) for x in (q, k, v))
        bias = sub["key_bias"].reshape(1, 1, -1).double()
        om = masked_attention(qm, km, vm, torch.ones(1, 1, 1, 1, dtype=torch.bool).expand(1, 1, 216, 216),
                              1 / 8, key_bias=bias)
        want = native.tome_unmerge(om, sub, 1)[0, 0]
        _check(out[bb, hh], want)
    # Every (b, h): its text rows, 32 random video rows and the last row, each through the
    # merged row it is unmerged from, against the fp64 oracle on the oracle's merged tensors.
    g = torch.Generator().manual_seed(4)
    L = q.shape[2]
    for bb in range(q.shape[0]):
        sub = {f: t[bb:bb + 1] for f, t in want_maps.items()}
        bias = sub["key_bias"].reshape(1, 1, -1).double()
        rot = sub["row_of_token"][0].long()
        for hh in range(q.shape[1]):
            sel = lambda x: x[bb:bb + 1, hh:hh + 1]
            qm, km, vm = (native.tome_merge(sel(x), sub, a, b, 4000, 226, 1) for x in (q, k, v))
            rows = torch.unique(torch.cat([torch.arange(226), torch.randint(226, L, (32,), generator=g),
                                           torch.tensor([L - 1])]))
            mrows, inv = torch.unique(rot[rows], return_inverse=True)
            om = masked_attention(qm, km, vm, torch.ones(1, 1, 1, 1, dtype=torch.bool).expand(1, 1, 216, 216),
                                  1 / 8, key_bias=bias, rows=mrows)[0, 0]
            _check(out[bb, hh, rows], om[inv])


def test_merge_attention_reference_setting(dev):
    # The reference's own configuration: per-head (k,|k|,v,|v|) metric, 3x3x4 cells,
    # k/v-only merge (MergeAttention.py:16-48), on a smaller grid.
    case("MergeAttention per-head, k/v merge")
    geom = Geometry(text_len=226, T=5, Hp=6, Wp=9)
    q, k, v = cogvideox_qkv(6, B=2, H=2, geom=geom)
    cfg = dict(REFERENCE_MERGE_CONFIG, w=9, h=6, t=5, r=60)
    proc = MergeAttention(cfg, full_merge=False, metric="kv_norm")
    out = proc(q.to(dev), k.to(dev), v.to(dev)).cpu()
    assert out.shape == q.shape
    maps = proc.maps
    a, b = maps.a_idx.cpu(), maps.b_idx.cpu()
    want = native.tome_match(native.tome_metric(k, v, 226, 1), a, b, 60, 226)
    _maps_equal(maps, want)
    km = native.tome_merge(k, want, a, b, 60, 226, 1)
    vm = native.tome_merge(v, want, a, b, 60, 226, 1)
    Lm = km.shape[2]
    bias = want["key_bias"].reshape(2, 2, Lm).double()
    nb_q, nb_k = math.ceil(q.shape[2] / 64), math.ceil(Lm / 64)
    ref = masked_attention(q, km, vm, torch.ones(1, 1, nb_q, nb_k, dtype=torch.bool), 1 / 8, key_bias=bias)
    _check(out, ref)
    # gap > 1 reuses the maps between re-matches
    proc.gap = 2
    proc(q.to(dev), k.to(dev), v.to(dev))
    assert proc.maps is not maps or proc.calls % 2 == 0


def test_merge_attention_random_dst_choice(dev):
    # The reference draws one dst per (st, sy, sx) cell from the processor's generator at every
    # re-match (MergeAttention.py:20, :30; merge_unmerge.py:66-70). The partition follows the
    # reference's steps (test_oracle_tome's numpy restatement) on the same draws, the maps
    # match the C oracle on that partition, and the next re-match draws again.
    from test_oracle_tome import _reference_partition
    case("MergeAttention reference setting, generator-driven dst choice")
    geom = Geometry(text_len=226, T=5, Hp=6, Wp=9)
    q, k, v = cogvideox_qkv(9, B=2, H=2, geom=geom)
    cfg = dict(REFERENCE_MERGE_CONFIG, w=9, h=6, t=5, r=60)
    proc = MergeAttention.reference(merge_config=cfg, generator=torch.Generator(device=dev).manual_seed(7))
    assert (proc.full_merge, proc.metric, proc.no_rand) == (False, "kv_norm", False)
    twin = torch.Generator(device=dev).manual_seed(7)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    seen = []
    for call in range(3):
        proc(qd, kd, vd)
        draws = torch.randint(3 * 3 * 4, size=((5 - 1) // 4, 6 // 3, 9 // 3, 1), device=dev, generator=twin)
        choice = draws.cpu().reshape(-1)
        assert torch.equal(proc.cell_choice.reshape(-1).long(), choice)
        ra, rb = _reference_partition(5, 6, 9, 3, 3, 4, choice)
        maps = proc.maps
        assert np.array_equal(maps.a_idx.cpu().numpy(), ra) and np.array_equal(maps.b_idx.cpu().numpy(), rb)
        want = native.tome_match(native.tome_metric(k, v, 226, 1), maps.a_idx.cpu(), maps.b_idx.cpu(), 60, 226)
        _maps_equal(maps, want)
        seen.append(tuple(choice.tolist()))
    assert len(set(seen)) > 1  # each re-match draws anew
    # no_rand keeps the top-left token of every cell
    top = MergeAttention(cfg, full_merge=False, metric="kv_norm")
    top(qd, kd, vd)
    ra, rb = _reference_partition(5, 6, 9, 3, 3, 4)
    assert top.cell_choice is None and np.array_equal(top.maps.b_idx.cpu().numpy(), rb)


def test_reference_api_closures(dev):
    case("bipartite_soft_matching_video API")
    geom = Geometry(text_len=226, T=4, Hp=6, Wp=10)
    q, k, v = cogvideox_qkv(7, B=1, H=2, geom=geom)
    kd = k.to(dev)
    metric = kd[:, :, 226:].reshape(2, geom.n_video, 64).float()
    merge, unmerge = merge_unmerge.bipartite_soft_matching_video(metric, 10, 6, 4, 2, 2, 1, r=30, no_rand=True)
    assert merge_unmerge.counter.shape == (2, merge.maps.n_dst, 1)
    assert merge_unmerge.counter.dtype == torch.int64
    xm = merge(kd)
    assert xm.shape == (1, 2, geom.L - 30, 64)
    back = unmerge(xm)
    assert back.shape == kd.shape
    assert torch.equal(merge(kd.reshape(2, geom.L, 64)), xm.reshape(2, geom.L - 30, 64))
    ident = merge_unmerge.bipartite_soft_matching_video(metric, 10, 6, 4, 2, 2, 1, r=0)
    assert ident[0] is merge_unmerge.do_nothing
    g = torch.Generator(device="cpu").manual_seed(0)
    m2, _ = merge_unmerge.bipartite_soft_matching_video(metric, 10, 6, 4, 2, 2, 1, r=30, generator=g)
    assert m2.maps.n_dst == merge.maps.n_dst
