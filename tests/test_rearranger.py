"""The 1.5-5B rearranger permutation of CombinedAttn (combined_attn.py:17-41), pinned on the
CPU against einops applying the reference's rearrange patterns to an index tensor; the GPU
gathers are checked against index_select and for rearranger/recover being inverse."""
import pytest
import torch
from einops import rearrange

from conftest import case
from sparseattnfunctions_amd.combined_attn import CombinedAttn, rearranger_permutation

L = 224 + 11 * 48 * 85


def _einops_perm():
    x = torch.arange(L)[None, None, :, None]
    vid = x[:, :, 224:]
    c1 = rearrange(vid[:, :, : 9 * 48 * 85], "b h (pfn pf phn ph pwn pw) d -> b h (pfn phn pwn pf ph pw) d",
                   pfn=3, pf=3, phn=12, ph=4, pwn=17, pw=5)
    c2 = rearrange(vid[:, :, 9 * 48 * 85:], "b h (pfn pf phn ph pwn pw) d -> b h (pfn phn pwn pf ph pw) d",
                   pfn=1, pf=2, phn=8, ph=6, pwn=17, pw=5)
    return torch.cat([c1, c2, x[:, :, :224]], dim=2).flatten()


def _einops_recover(y):
    text = y[:, :, -224:]
    c1 = rearrange(y[:, :, : 9 * 48 * 85], "b h (pfn phn pwn pf ph pw) d -> b h (pfn pf phn ph pwn pw) d",
                   pfn=3, pf=3, phn=12, ph=4, pwn=17, pw=5)
    c2 = rearrange(y[:, :, 9 * 48 * 85: 11 * 48 * 85], "b h (pfn phn pwn pf ph pw) d -> b h (pfn pf phn ph pwn pw) d",
                   pfn=1, pf=2, phn=8, ph=6, pwn=17, pw=5)
    return torch.cat([text, c1, c2], dim=2)


def test_permutation_matches_einops():
    perm = rearranger_permutation()
    assert perm.dtype == torch.int32 and perm.numel() == L
    assert torch.equal(perm.long(), _einops_perm())
    # recover (as the reference writes it) undoes the permutation
    assert torch.equal(_einops_recover(perm.long()[None, None, :, None]).flatten(), torch.arange(L))


@pytest.mark.gpu
def test_gpu_rearranger_and_recover(dev):
    case("CombinedAttn rearranger/recover, B=1 H=2 L=45104")
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(1, 2, L, 64, generator=g).bfloat16().to(dev) for _ in range(3))
    perm = rearranger_permutation().long().to(dev)
    rq, rk, rv = CombinedAttn.rearranger(q, k, v)
    for x, r in ((q, rq), (k, rk), (v, rv)):
        assert torch.equal(r, x.index_select(2, perm))
    assert torch.equal(CombinedAttn.recover(rq), q)
    with pytest.raises(ValueError):
        CombinedAttn.rearranger(q[:, :, :100], k, v)
