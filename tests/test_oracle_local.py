"""Pins the local-window oracle and checks the library's host bitmap against it (CPU)."""
import torch

from oracle import native
from sparseattnfunctions_amd.block_masks import local_window_bitmap
from sparseattnfunctions_amd.workloads import COGVIDEOX_2B, COGVIDEOX_15_5B, Geometry


def _brute(geom, dt, dh, dw):
    # Independent formulation: coordinates from explicit enumeration of the token grid.
    coords = {}
    tok = geom.text_len
    for t in range(geom.T):
        for h in range(geom.Hp):
            for w in range(geom.Wp):
                coords[tok] = (t, h, w)
                tok += 1
    nb = -(-geom.L // geom.block)
    centre = [min(b * geom.block + geom.block // 2, geom.L - 1) for b in range(nb)]
    out = torch.zeros(nb, nb, dtype=torch.uint8)
    for i, ci in enumerate(centre):
        for j, cj in enumerate(centre):
            if ci in coords and cj in coords:
                a, b = coords[ci], coords[cj]
                out[i, j] = abs(a[0] - b[0]) <= dt and abs(a[1] - b[1]) <= dh and abs(a[2] - b[2]) <= dw
    return out


def test_oracle_matches_brute_force_small():
    for geom, win in [(Geometry(text_len=10, T=3, Hp=4, Wp=5, block=8), (1, 1, 1)),
                      (Geometry(text_len=226, T=2, Hp=10, Wp=15), (1, 2, 3)),
                      (Geometry(text_len=0, T=4, Hp=6, Wp=6, block=16), (0, 1, 1))]:
        assert torch.equal(native.local_window(geom, *win), _brute(geom, *win))


def test_library_host_bitmap_matches_oracle():
    for geom in (COGVIDEOX_2B, COGVIDEOX_15_5B, Geometry(text_len=226, T=2, Hp=10, Wp=15)):
        for win in ((1, 8, 8), (0, 2, 2)):
            assert torch.equal(local_window_bitmap(geom, win), native.local_window(geom, *win))


def test_cogvideox_density_and_invariants():
    geom = COGVIDEOX_2B
    bm = native.local_window(geom, 1, 8, 8).bool()
    nb = bm.shape[0]
    assert nb == 278
    assert torch.equal(bm, bm.T)                          # the window is symmetric
    assert bm[4:, 4:].diagonal().all()                    # every video block sees itself
    assert not bm[:4].any() and not bm[:, :4].any()       # text handled by the text rule
    text = torch.zeros(nb, nb, dtype=torch.bool)
    text[:4] = True
    text[:, :4] = True
    # Density of local U text with the centre-token rule (independently computed as 0.0680).
    assert abs((bm | text).float().mean().item() - 0.0680) < 5e-4


def test_cogvideox_bitmap_matches_fixture():
    # tests/golden/local_window_cogvideox2b.npy (packbits of the 278 x 278 bitmap) pins the
    # config-3 local window of both the oracle and the library's host builder.
    import os
    import numpy as np
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "local_window_cogvideox2b.npy")
    nb = COGVIDEOX_2B.nb
    want = torch.from_numpy(np.unpackbits(np.load(path, allow_pickle=False))[: nb * nb].reshape(nb, nb))
    assert torch.equal(native.local_window(COGVIDEOX_2B, 1, 8, 8), want)
    assert torch.equal(local_window_bitmap(COGVIDEOX_2B, (1, 8, 8)), want)


def test_local_window_perm_identity_and_brute_force():
    from oracle import layout
    from oracle import native
    from sparseattnfunctions_amd.workloads import COGVIDEOX_2B, Geometry

    # identity permutation: the pinned C oracle's window plus the text rows and columns
    g = COGVIDEOX_2B
    got = layout.local_window_perm(torch.arange(g.L), g.L, 64, g.text_len, g.T, g.Hp, g.Wp, 1, 8, 8)
    want = native.local_window(g, 1, 8, 8).clone()
    want[:4, :] = 1
    want[:, :4] = 1
    assert torch.equal(got, want)
    # random permutation of a tiny grid, against explicit loops
    small = Geometry(text_len=5, T=3, Hp=4, Wp=6, block=8)
    perm = torch.randperm(small.L, generator=torch.Generator().manual_seed(3))
    got = layout.local_window_perm(perm, small.L, 8, 5, 3, 4, 6, 1, 1, 2)
    nb = -(-small.L // 8)
    for i in range(nb):
        for j in range(nb):
            ci, cj = int(perm[min(8 * i + 4, small.L - 1)]), int(perm[min(8 * j + 4, small.L - 1)])
            texti = any(int(perm[x]) < 5 for x in range(8 * i, min(8 * i + 8, small.L)))
            textj = any(int(perm[x]) < 5 for x in range(8 * j, min(8 * j + 8, small.L)))
            on = texti or textj
            if ci >= 5 and cj >= 5:
                a, b = ci - 5, cj - 5
                ta, ha, wa = a // 24, (a // 6) % 4, a % 6
                tb, hb, wb = b // 24, (b // 6) % 4, b % 6
                on = on or (abs(ta - tb) <= 1 and abs(ha - hb) <= 1 and abs(wa - wb) <= 2)
            assert got[i, j].item() == int(on), (i, j)


def test_library_perm_bitmap_matches_oracle():
    # The host bitmap of the library (sa_local_window_bitmap_perm) against the oracle, on the
    # 1.5-5B rearranger permutation (CPU only: a host entry point).
    from oracle import layout
    from sparseattnfunctions_amd.block_masks import local_window_bitmap_perm
    from sparseattnfunctions_amd.combined_attn import rearranger_permutation
    from sparseattnfunctions_amd.workloads import COGVIDEOX_15_5B as g

    perm = rearranger_permutation()
    got = local_window_bitmap_perm(g, perm, (1, 8, 8))
    want = layout.local_window_perm(perm, g.L, 64, g.text_len, g.T, g.Hp, g.Wp, 1, 8, 8)
    assert torch.equal(got, want)
    assert got[701:].all() and got[:, 701:].all() and not got[:700, :700].all()  # text blocks 701-704
