"""The allocation-free matching entry point (sa_tome_match_noalloc) gives the same maps as
sa_tome_match with a workspace, bit for bit, on two calls in a row (the second smaller, so it
reuses the scratch the first one left behind), and rejects problems above its scratch size
before launching anything."""
import ctypes

import pytest
import torch

from conftest import case
from sparseattnfunctions_amd import _lib, _tome
from sparseattnfunctions_amd.workloads import Geometry, cogvideox_qkv

pytestmark = pytest.mark.gpu

FIELDS = ("node_idx", "node_max", "rank", "edge", "dst_idx", "dst_cnt", "dst_ptr", "members", "row_of_token",
          "key_bias", "merged_src", "member_rows")


def _noalloc(metric, a, b, r, text_len):
    G, N, C = metric.shape
    maps = _tome.TomeMaps(G, N, text_len, a, b, max(0, min(r, a.numel())), metric.device)
    with torch.cuda.device(metric.device):
        rc = _lib.load().sa_tome_match_noalloc(metric.data_ptr(), C, ctypes.byref(maps.struct),
                                               _lib.stream_of(metric))
    return rc, maps


def _same(got, want):
    for f in FIELDS:
        g, w = getattr(got, f), getattr(want, f)
        if f in ("dst_idx", "members", "member_rows"):
            g, w = g[:, : want.r], w[:, : want.r]
        assert torch.equal(g.cpu(), w.cpu()), f


@pytest.mark.parametrize("mode", [0, 1])
def test_match_noalloc_equals_workspace_entry(dev, mode):
    # Call 1: config 4 (B=2, H=30, 13x30x45, r=4000) with the head-summed metric, or a per-head
    # metric on fewer heads; call 2: a smaller grid and r.
    cases = [(Geometry(), 2, 30 if mode == 0 else 2, 4000, 3), (Geometry(T=4, Hp=6, Wp=10), 2, 3, 37, 5)]
    for geom, B, H, r, seed in cases:
        case(f"tome match noalloc mode={mode} T={geom.T} r={r}")
        _, k, v = cogvideox_qkv(seed, B=B, H=H, geom=geom)
        metric = _tome.metric_from_qkv(k.to(dev), v.to(dev) if mode == 1 else None, geom.text_len, mode)
        a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
        want = _tome.match(metric, a, b, r, geom.text_len)
        rc, got = _noalloc(metric, a, b, r, geom.text_len)
        assert rc == _lib.SA_OK, _lib.load().sa_last_error()
        torch.cuda.synchronize()
        _same(got, want)
        assert torch.equal(_tome.match_noalloc(metric, a, b, r, geom.text_len).edge.cpu(), want.edge.cpu())


def test_match_noalloc_rejects_oversized(dev):
    # 60 per-head groups of the config-4 grid need 60 * 16 * 12240 * 8 bytes of partials
    # (94 MB), above the 16 MiB scratch: refused on the host, nothing is launched.
    case("tome match noalloc oversized")
    geom = Geometry()
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    metric = torch.zeros(60, geom.n_video, 64, device=dev)
    rc, _ = _noalloc(metric, a, b, 4000, geom.text_len)
    assert rc == _lib.SA_ERR_INVALID
    assert b"scratch" in _lib.load().sa_last_error()
    with pytest.raises(ValueError):
        _tome.match_noalloc(metric, a, b, 4000, geom.text_len)


def test_match_noalloc_calls_on_two_streams(dev):
    # Calls on one GPU share its scratch array; match_noalloc orders its calls across streams
    # (each waits for an event after the previous call), so two calls issued back to back on
    # two streams, with no synchronisation between them, both give the workspace entry's maps.
    case("tome match noalloc on two streams")
    geom = Geometry(T=6, Hp=12, Wp=20)
    a, b = _tome.partition(geom.T, geom.Hp, geom.Wp, 2, 2, 1, dev)
    metrics, wants = [], []
    for seed in (11, 12):
        _, k, _ = cogvideox_qkv(seed, B=2, H=4, geom=geom)
        m = _tome.metric_from_qkv(k.to(dev), None, geom.text_len, 0)
        metrics.append(m)
        wants.append(_tome.match(m, a, b, 300, geom.text_len))
    main = torch.cuda.current_stream(dev)
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    got = []
    for s, m in zip(streams, metrics):
        s.wait_stream(main)
        with torch.cuda.stream(s):
            got.append(_tome.match_noalloc(m, a, b, 300, geom.text_len))
    torch.cuda.synchronize()
    for g, w in zip(got, wants):
        _same(g, w)
