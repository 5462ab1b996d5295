"""GPU parity of the frame-factored backup path (block_mask_attn.forward_backup and the
utils/mask_related.py functions behind it): the Kronecker mask bit-exact against the oracle;
the frame-scope map and the inner-frame cell sums against the fp64 oracle; the energy cuts
bit-exact against the C oracle on the GPU's own maps; the whole call against the fp64
attention oracle on sampled rows of every head."""
import pytest
import torch

from conftest import case
from oracle import backup, native
from oracle.attention import masked_attention
from sparseattnfunctions_amd.block_mask_attn import BlockSparseAttention
from sparseattnfunctions_amd.utils import mask_related as mr
from sparseattnfunctions_amd.workloads import cogvideox_qkv

pytestmark = pytest.mark.gpu

T, F, S, NS = 226, 13, 1350, 60


@pytest.fixture(scope="module")
def c2_inputs():
    return cogvideox_qkv(0)


def _check(got, want):
    err = (got.float().cpu().double() - want).abs()
    assert torch.isfinite(got.float()).all()
    assert err.max().item() <= 2e-2, err.max().item()
    assert err.mean().item() <= 2e-3, err.mean().item()


def test_get_block_mask_matches_oracle(dev):
    case("get_block_mask")
    g = torch.Generator().manual_seed(0)
    frame = torch.rand(2, 3, F, F, generator=g) < 0.4
    inner = torch.rand(2, 3, 22, 21, generator=g) < 0.7
    got = mr.get_block_mask(inner.to(dev), frame.to(dev))
    assert got.shape == (2, 3, 13 * 22 + 4, 13 * 21 + 4) and got.dtype == torch.float32
    assert torch.equal(got.cpu(), backup.kron_mask(inner, frame))


def test_frame_scope_mask(dev, c2_inputs):
    case("generate_attention_mask_frame_scope")
    q, k, _ = c2_inputs
    draws = torch.randint(0, S, (NS,), generator=torch.Generator().manual_seed(4))
    qd, kd = q.to(dev), k.to(dev)
    got_map = mr.frame_scope_map(qd, kd, draws=draws).cpu()
    want_map = backup.frame_scope_map(q, k, draws)
    # per-row masses are bf16 (relative 2^-9), summed over 60 rows in fp32
    assert torch.allclose(got_map.double(), want_map, rtol=4e-3, atol=1e-6), (got_map.double() - want_map).abs().max()
    mask = mr.generate_attention_mask_frame_scope(qd, kd, draws=draws).cpu()
    assert mask.shape == (2, 30, F, F) and mask.dtype == torch.bool
    _, _, om = native.energy_list(got_map.reshape(60, 1, F * F), 2, 0.9, 0, F * F, 1, 0)
    assert torch.equal(mask.reshape(60, F * F), om.bool().reshape(60, F * F))
    # against the cut of the fp64 map: only boundary entries may differ
    _, _, o64 = native.energy_list(want_map.float().reshape(60, 1, F * F), 2, 0.9, 0, F * F, 1, 0)
    assert (mask.reshape(60, -1) != o64.bool().reshape(60, -1)).float().mean().item() <= 0.01


@pytest.mark.parametrize("scope,thr", [("row", 1.0), ("row", 0.9), ("head", 0.9)])
def test_inner_frame_mask(dev, c2_inputs, scope, thr):
    case(f"get_inner_frame_mask scope={scope} threshold={thr}")
    q, k, v = c2_inputs
    starts = torch.randint(0, 7, (2, 13), generator=torch.Generator().manual_seed(5))
    qp, kp, _ = mr.preprocess_qkv(q.to(dev), k.to(dev), v.to(dev), starts=starts)
    cells = mr.inner_frame_cell_sums(qp, kp).cpu()
    want = backup.inner_cell_sums(qp.cpu(), kp.cpu())
    assert cells.shape == (2, 30, 22, 21)
    assert torch.allclose(cells.double(), want, rtol=4e-3, atol=1e-4), (cells.double() - want).abs().max()
    mask = mr.get_inner_frame_mask(qp, kp, scope=scope, threshold=thr).cpu()
    if scope == "row":
        _, _, om = native.energy_list(cells.reshape(60, 22, 21), 2, thr, 0, 21, 1, 0)
        om = om.reshape(2, 30, 22, 21)
    else:
        _, _, om = native.energy_list(cells.reshape(60, 1, 22 * 21), 3, thr, 0, 22 * 21, 1, 0)
        om = om.reshape(2, 30, 22, 21)
    assert torch.equal(mask, om.bool())
    if thr == 1.0:
        # threshold 1: every cell keeps mass far above fp32 resolution, so all are kept
        assert mask.all()


def test_calc_attn_probabilities(dev):
    case("calc_attn")
    g = torch.Generator().manual_seed(6)
    q = torch.randn(1, 2, 100, 64, generator=g).bfloat16()
    k = torch.randn(1, 2, 70, 64, generator=g).bfloat16()
    got = mr.calc_attn(q.to(dev), k.to(dev)).cpu()
    assert got.dtype == torch.bfloat16 and got.shape == (1, 2, 100, 70)
    want = torch.softmax(q.double() @ k.double().transpose(-1, -2) / 8, dim=-1)
    assert (got.double() - want).abs().max().item() <= 2 ** -8 * want.max().item()


def test_forward_backup(dev, c2_inputs):
    case("BlockSparseAttention.forward_backup")
    q, k, v = c2_inputs
    draws = torch.randint(0, S, (NS,), generator=torch.Generator().manual_seed(7))
    starts = torch.randint(0, 7, (2, 13), generator=torch.Generator().manual_seed(8))
    proc = BlockSparseAttention()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = proc.forward_backup(qd, kd, vd, frame_draws=draws, starts=starts).cpu()
    assert out.shape == q.shape
    # The oracle mask from the GPU's two factor masks (each checked above), the processed
    # layout from preprocess_qkv (checked against the reference's ops in test_gpu_layout).
    outer = mr.generate_attention_mask_frame_scope(qd, kd, draws=draws).cpu()
    qp, kp, vp = mr.preprocess_qkv(qd, kd, vd, starts=starts)
    inner = mr.get_inner_frame_mask(qp, kp).cpu()
    mask = backup.kron_mask(inner, outer).bool()
    assert torch.equal(proc.last_kv.to_mask().cpu(), mask)
    qp, kp, vp = qp.cpu(), kp.cpu(), vp.cpu()
    fp = 1408
    gen = torch.Generator().manual_seed(9)
    for b in range(2):
        for h in range(30):
            tok = torch.unique(torch.cat([torch.randint(0, T, (8,), generator=gen),
                                          torch.randint(T, T + F * S, (32,), generator=gen)]))
            t = tok - T
            prow = torch.where(tok < T, F * fp + tok, (t // S) * fp + t % S)
            order = torch.argsort(prow)
            want = masked_attention(qp, kp, vp, mask, 1 / 8, heads=[(b, h)], rows=prow[order])[b, h]
            _check(out[b, h, tok[order]], want)
