"""GPU tests: the C2 step and the key-bias fp16-score launch captured in a HIP graph.

Every entry point on these paths takes caller buffers and launches kernels only (no device
allocation, no memset nodes), so `torch.cuda.graph` can capture them. Each test warms the path
up eagerly (the work-order cache fills there), captures one call, then replays the graph
several times with new inputs copied into the captured tensors, eager work and
synchronisations between the replays, and checks every replay bit for bit against an eager
call on the same inputs (the kernels are deterministic).
"""
import pytest
import torch

from conftest import case
from sparseattnfunctions_amd._kv import kv_list_from_mask
from sparseattnfunctions_amd.block_mask_attn import BlockSparseAttention
from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import block_sparse_attention
from sparseattnfunctions_amd.workloads import Geometry

pytestmark = pytest.mark.gpu


def _rand(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).bfloat16().to(dev)


def _capture(fn, n_warm=2):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(n_warm):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_graph_c2_step(dev):
    # BlockSparseAttention.forward: pooling pass with the fp16 keys, top-k lists, fp16-score
    # attention.
    case("HIP graph: mean-pool top-k step")
    geom = Geometry(text_len=100, T=3, Hp=12, Wp=16)
    shape = (1, 4, geom.L, 64)
    proc = BlockSparseAttention(64, keep_ratio=0.3, geometry=geom)
    q, k, v = (_rand(shape, 1100 + i, dev) for i in range(3))
    g, out = _capture(lambda: proc(q, k, v))
    for rep in range(3):
        new = [_rand(shape, 1200 + 3 * rep + i, dev) for i in range(3)]
        want = proc(*new)  # eager call on the same inputs
        torch.cuda.synchronize()
        for dst, src in zip((q, k, v), new):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        assert torch.isfinite(out.float()).all()


def test_graph_k16_key_bias(dev):
    # sa_block_sparse_fwd_k16 with prepared = 0 and a key bias: the fp16 copy of k, the bias
    # times log2(e) and the attention, three launches in one entry point.
    case("HIP graph: fp16 scores with a key bias")
    B, H, L = 1, 3, 900
    nb = (L + 63) // 64
    q, k, v = (_rand((B, H, L, 64), 1300 + i, dev) for i in range(3))
    gen = torch.Generator().manual_seed(1303)
    bias = torch.log(torch.randint(1, 9, (B, 1, L), generator=gen).float()).to(dev)
    mask = torch.rand(B, H, nb, nb, generator=gen) < 0.6
    mask[..., 0] = True
    kv = kv_list_from_mask(mask.to(dev), B, H, nb, nb)

    def call(q, k, v, bias):
        return block_sparse_attention(q, k, v, kv, 0.125, key_bias=bias, fp16_scores=True)

    g, out = _capture(lambda: call(q, k, v, bias))
    for rep in range(3):
        new = [_rand((B, H, L, 64), 1400 + 3 * rep + i, dev) for i in range(3)]
        nbias = torch.log(torch.randint(1, 9, (B, 1, L), generator=gen).float()).to(dev)
        want = call(*new, nbias)
        torch.cuda.synchronize()
        for dst, src in zip((q, k, v, bias), (*new, nbias)):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        assert not torch.equal(out, block_sparse_attention(q, k, v, kv, 0.125, key_bias=bias, fp16_scores=False))
