"""GPU parity of the adaptive estimator (SparseGen_Plus): sampled tokens and block scores
against oracle/estimator.py, the energy / adaptive top-k lists bit-exact against the C oracle
on the GPU's own scores, and the BlockSparseAttention processor end to end.

Tolerances: sampled block scores (fp32 on the GPU, fp64 in the oracle) rtol 1e-4,
atol 1e-6; token ids, kv lists and masks bit-exact; attention as in test_gpu_attention
(max-abs 2e-2, mean-abs 2e-3 against the fp64 masked-attention oracle).
"""
import json
import math

import pytest
import torch

from conftest import case
from oracle import estimator as oest
from oracle import native
from oracle.attention import masked_attention
from sparseattnfunctions_amd import SparseGen_Plus as sgp
from sparseattnfunctions_amd.estimator import energy_kv_list, sample_block_tokens, sampled_block_scores
from sparseattnfunctions_amd.utils import mask_related as mr
from sparseattnfunctions_amd.workloads import cogvideox_qkv

pytestmark = pytest.mark.gpu


def _bf16(shape, seed, scale=1.0):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * scale).to(torch.bfloat16)


def _rand(shape, seed):
    return torch.rand(shape, generator=torch.Generator().manual_seed(seed))


@pytest.mark.parametrize("L,S", [(64, 8), (700, 8), (257, 16), (1000, 16)])
def test_sampled_tokens_and_rows(dev, L, S):
    case(f"sample_block_tokens L={L} num_keep={S}")
    B, H = 2, 3
    q, k = _bf16((B, H, L, 64), 1), _bf16((B, H, L, 64), 2)
    nb = math.ceil(L / 64)
    rq, rk = _rand((B, H, nb, 64), 3), _rand((B, H, nb, 64), 4)
    qs, ks, tq, tk = sample_block_tokens(q.to(dev), k.to(dev), S, rq.to(dev), rk.to(dev))
    torch.cuda.synchronize()
    want_q, want_k = oest.sample_tokens(rq, L, S), oest.sample_tokens(rk, L, S)
    assert torch.equal(tq.cpu().long(), want_q.reshape(B * H, -1))
    assert torch.equal(tk.cpu().long(), want_k.reshape(B * H, -1))
    ns = nb * S
    for bh in range(B * H):
        b, h = divmod(bh, H)
        assert torch.equal(qs[bh, :ns].cpu(), q[b, h][want_q[b, h]])
        assert torch.equal(ks[bh, :ns].cpu(), k[b, h][want_k[b, h]])


def test_random_sample_tokens_and_padding(dev):
    case("random_sample_tokens / pad_to_multiple")
    x = _bf16((1, 2, 256, 64), 5)
    g = torch.Generator(device=dev).manual_seed(7)
    got = mr.random_sample_tokens(x.to(dev), 64, 8, generator=g).cpu()
    rand = torch.rand(1, 2, 4, 64, device=dev, generator=torch.Generator(device=dev).manual_seed(7)).cpu()
    tok = oest.sample_tokens(rand, 256, 8)
    assert torch.equal(got, torch.stack([x[0, h][tok[0, h]] for h in range(2)])[None])
    y = _bf16((1, 2, 100, 64), 6)
    p = mr.pad_to_multiple(y.to(dev), 64).cpu()
    assert p.shape == (1, 2, 128, 64) and torch.equal(p[:, :, :100], y)
    assert torch.equal(p[:, :, 100:], y[:, :, 99:100].expand(1, 2, 28, 64))


@pytest.mark.parametrize("L,S", [(200, 8), (700, 8), (1000, 16), (300, 16)])
def test_sampled_block_scores(dev, L, S):
    case(f"sampled_block_scores L={L} num_keep={S}")
    B, H = 1, 3
    q, k = _bf16((B, H, L, 64), 10, 2.0), _bf16((B, H, L, 64), 11, 2.0)
    nb = math.ceil(L / 64)
    rq, rk = _rand((B, H, nb, 64), 12), _rand((B, H, nb, 64), 13)
    got = sampled_block_scores(q.to(dev), k.to(dev), S, rq.to(dev), rk.to(dev)).cpu().double()
    want = oest.sampled_block_scores(q, k, rq, rk, S)
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-6), (got - want).abs().max().item()


def test_sampled_block_scores_cogvideox_shape(dev):
    # Config-2 geometry (B=2, H=30, L=17776, 278 blocks), num_keep = 8 as SparseGen_Plus uses.
    case("sampled_block_scores CogVideoX shape")
    q, k, _ = cogvideox_qkv(0)
    B, H, L, _ = q.shape
    nb = 278
    rq, rk = _rand((B, H, nb, 64), 20), _rand((B, H, nb, 64), 21)
    got = sampled_block_scores(q.to(dev), k.to(dev), 8, rq.to(dev), rk.to(dev)).cpu().double()
    assert torch.allclose(got.sum(-1), torch.full((B, H, nb), 8.0, dtype=torch.float64), rtol=1e-4)
    heads = [(0, 0), (1, 29)]
    want = oest.sampled_block_scores(q, k, rq, rk, 8, heads=heads)
    for b, h in heads:
        assert torch.allclose(got[b, h], want[b, h], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("mode", ["energy", "topk"])
@pytest.mark.parametrize("nkb", [5, 64, 65, 278, 400, 700, 1024])
def test_energy_lists_bit_exact(dev, mode, nkb):
    case(f"energy_kv_list mode={mode} nkb={nkb}")
    B, H, nqb = 2, 3, 9
    g = torch.Generator().manual_seed(nkb)
    scores = torch.rand(B, H, nqb, nkb, generator=g) ** 4
    scores[0, 0, 1] = 0.5  # ties
    scores[1, 2, 3, : nkb // 2] = 0.125
    kv, mask = energy_kv_list(scores.to(dev), mode, init_k=0.2, max_retain_ratio=0.85, min_retain_ratio=0.1,
                              energy_threshold=0.95, return_mask=True)
    torch.cuda.synchronize()
    min_keep, max_keep = max(1, int(nkb * 0.1)), max(1, int(nkb * 0.85))
    k0 = max(1, int(nkb * 0.2))
    idx, cnt, omask = native.energy_list(scores.reshape(B * H, nqb, nkb), 0 if mode == "energy" else 1, 0.95,
                                         min_keep, max_keep, k0, 4)
    assert torch.equal(mask.cpu(), omask.bool().reshape(B, H, nqb, nkb))
    assert torch.equal(kv.cnt.cpu(), cnt)
    for r in range(B * H * nqb):
        assert torch.equal(kv.idx[r, : cnt[r]].cpu(), idx[r, : cnt[r]])


def test_energy_lists_on_sampled_scores_cogvideox(dev):
    # The full SparseGen_Plus mask source at config-2 size: GPU scores -> GPU lists, checked
    # bit-exact by the C oracle on the same scores; mask is what transfer_attn_to_mask returns.
    case("estimator + energy lists CogVideoX shape")
    q, k, _ = cogvideox_qkv(0)
    B, H = q.shape[:2]
    g = torch.Generator(device=dev).manual_seed(3)
    pooled = mr.calc_attn_block_sum_efficient(q.to(dev), k.to(dev), num_keep=8, generator=g)
    thr = float(sgp.concentrated_interpolation(0.9, 0.98, 50, concentration=0.5)[10])
    mask = sgp.transfer_attn_to_mask(pooled, "energy", max_retain_ratio=0.85, min_retain_ratio=0.1,
                                     energy_threshold=thr)
    _, _, omask = native.energy_list(pooled.cpu().reshape(B * H, 278, 278), 0, thr, 27, int(278 * 0.85), 1, 4)
    assert torch.equal(mask.cpu(), omask.bool().reshape(B, H, 278, 278))
    assert 0.05 < mask.float().mean().item() < 0.9


def test_sparsegen_processor_end_to_end(dev, tmp_path):
    case("SparseGen_Plus.BlockSparseAttention warmup + sparse steps")
    B, H, L = 1, 2, 700
    q, k, v = (_bf16((B, H, L, 64), 30 + i) for i in range(3))
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    proc = sgp.BlockSparseAttention(layernum=2, timestep=3, warmup_epoch=1, verbose=False, record_dir=str(tmp_path))
    nb = math.ceil(L / 64)
    full = torch.ones(1, 1, nb, nb, dtype=torch.bool)
    for call in range(6):
        state = torch.cuda.get_rng_state(dev.index or 0)
        out = proc(qd, kd, vd)
        torch.cuda.synchronize()
        assert torch.equal(torch.cuda.get_rng_state(dev.index or 0), state)  # draws are restored
        if call < 2:  # timestep 0 < warmup_epoch: dense
            want = masked_attention(q, k, v, full, 1 / 8)
        else:
            kv = proc.mask.kv(call % 2)
            m = proc.mask[call % 2].cpu()  # the reference's bool [B, H, nb, nb] view
            assert m.dtype == torch.bool and m.shape == (1, 2, nb, nb)
            assert torch.equal(m, kv.to_mask().cpu())
            want = masked_attention(q, k, v, m, 1 / 8)
            assert m[:, :, :4].all() and m[:, :, :, :4].all()
        err = (out.float().cpu().double() - want).abs()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    rec = json.loads((tmp_path / "sparsity_record_sample_0.json").read_text())["records"]
    assert [(r["timestep"], r["layer"]) for r in rec] == [(1, 0), (1, 1), (2, 0), (2, 1)]
    assert all(0.0 <= r["sparsity"] < 1.0 for r in rec)
