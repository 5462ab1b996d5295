"""GPU checks of the layout transforms: preprocess_qkv / reverse_process_out (per-frame pad and
random truncation, utils/mask_related.py:87-187) against the reference's own formulation with
torch CPU ops, their round trip, and the row-mapped attention that reads and writes through
the padded layout without copies (bit-identical to copy -> attend -> copy back)."""
import math

import pytest
import torch
import torch.nn.functional as F

from conftest import case
from sparseattnfunctions_amd._kv import kv_list_from_mask
from sparseattnfunctions_amd.utils.block_sparse_attn_kernel import block_sparse_attention
from sparseattnfunctions_amd.utils.mask_related import padded_layout_maps, preprocess_qkv, reverse_process_out

pytestmark = pytest.mark.gpu

TEXT, FRAME, NF = 226, 1350, 13
L = TEXT + FRAME * NF


def _rand(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _reference_layout(q, k, v, starts):
    """preprocess_qkv with the reference's ops: rearrange to frames, F.pad the queries,
    gather the kept key/value window per (batch, frame), text last."""
    B, H, _, D = q.shape
    qv = q[:, :, TEXT:].reshape(B, H, NF, FRAME, D)
    qv = F.pad(qv.float(), (0, 0, 0, 64 - FRAME % 64)).to(q.dtype)
    keep = FRAME - FRAME % 64
    idx = (torch.arange(keep).view(1, 1, -1) + starts.view(B, NF, 1)).view(B, 1, NF, keep, 1).expand(B, H, NF, keep, D)
    kv_ = [x[:, :, TEXT:].reshape(B, H, NF, FRAME, D).gather(3, idx) for x in (k, v)]
    out = [torch.cat([qv.reshape(B, H, -1, D), q[:, :, :TEXT]], dim=2)]
    out += [torch.cat([x.reshape(B, H, -1, D), y[:, :, :TEXT]], dim=2) for x, y in zip(kv_, (k, v))]
    return out


def test_preprocess_matches_reference_ops_and_round_trips(dev):
    case("preprocess_qkv / reverse_process_out")
    B, H = 2, 2
    q, k, v = (_rand((B, H, L, 64), 10 + i) for i in range(3))
    starts = torch.randint(0, 7, (B, NF), generator=torch.Generator().manual_seed(3))
    qp, kp, vp = preprocess_qkv(q.to(dev), k.to(dev), v.to(dev), starts=starts)
    want = _reference_layout(q, k, v, starts)
    for got, w in zip((qp, kp, vp), want):
        assert torch.equal(got.cpu(), w)
    assert torch.equal(reverse_process_out(qp).cpu(), q)


def test_row_mapped_attention_equals_copies(dev):
    case("padded-layout attention through row maps")
    B, H = 1, 3
    q, k, v = (_rand((B, H, L, 64), 20 + i).to(dev) for i in range(3))
    starts = torch.randint(0, 7, (B, NF), generator=torch.Generator().manual_seed(4))
    qp, kp, vp = preprocess_qkv(q, k, v, starts=starts)
    nqb, nkb = math.ceil(qp.shape[2] / 64), math.ceil(kp.shape[2] / 64)
    g = torch.Generator().manual_seed(5)
    mask = torch.rand(B, H, nqb, nkb, generator=g) < 0.25
    mask[..., -4:] = True  # the text blocks, last in this layout
    kv = kv_list_from_mask(mask.to(dev), B, H, nqb, nkb)
    copies = reverse_process_out(block_sparse_attention(qp, kp, vp, kv, 0.125))
    q_rows, o_rows = padded_layout_maps(L, device=dev)
    fused = block_sparse_attention(q, kp, vp, kv, 0.125, q_rows=q_rows, o_rows=o_rows)
    torch.cuda.synchronize()
    assert fused.shape == q.shape
    assert torch.equal(fused, copies)
