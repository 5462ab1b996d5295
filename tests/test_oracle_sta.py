"""Pins the sliding-tile oracle (oracle/sta.py) and checks the library's host tables (CPU)."""
import math

import torch

from oracle import sta
from sparseattnfunctions_amd.SildingTileAttention import StaLayout, config, generate_sta_mask


def _brute_mask(text, img, tile, kern):
    T, Hp, Wp = img
    nt, nh, nw = T // tile[0], Hp // tile[1], Wp // tile[2]
    L = text + T * Hp * Wp
    coords = {}
    pos = text
    for a in range(nt):
        for b in range(nh):
            for c in range(nw):
                for _ in range(tile[0] * tile[1] * tile[2]):
                    coords[pos] = (a, b, c)
                    pos += 1
    m = torch.zeros(L, L, dtype=torch.bool)
    for qi in range(L):
        for ki in range(L):
            if qi < text or ki < text:
                m[qi, ki] = qi < text or ki < text
                continue
            (qt, qh, qw), (kt, kh, kw) = coords[qi], coords[ki]
            ct = min(max(qt, kern[0] // 2), nt - 1 - kern[0] // 2)
            ch = min(max(qh, kern[1] // 2), nh - 1 - kern[1] // 2)
            cw = min(max(qw, kern[2] // 2), nw - 1 - kern[2] // 2)
            m[qi, ki] = abs(ct - kt) <= kern[0] // 2 and abs(ch - kh) <= kern[1] // 2 and abs(cw - kw) <= kern[2] // 2
    return m


def test_token_mask_brute_force_small():
    for text, img, tile, kern in [(5, (2, 6, 6), (2, 2, 2), (1, 3, 3)), (3, (4, 4, 6), (2, 2, 3), (3, 1, 1))]:
        L = text + img[0] * img[1] * img[2]
        want = _brute_mask(text, img, tile, kern)
        got = sta.token_mask(torch.arange(L), L, text, img, tile, kern)
        assert torch.equal(got, want)
        ref = generate_sta_mask(img, kern, tile, text)(None, None, torch.arange(L)[:, None], torch.arange(L)[None, :])
        assert torch.equal(ref, want)


def test_permutation_is_the_einops_rearrange():
    text, img, tile = 3, (2, 4, 6), (2, 2, 3)
    perm = sta.permutation(text, img, tile)
    T, Hp, Wp = img
    # tile-major position of natural token (t, h, w)
    for t in range(T):
        for h in range(Hp):
            for w in range(Wp):
                nat = text + (t * Hp + h) * Wp + w
                a, x = divmod(t, tile[0]); b, y = divmod(h, tile[1]); c, z = divmod(w, tile[2])
                nh, nw = Hp // tile[1], Wp // tile[2]
                j = text + ((((a * nh + b) * nw + c) * tile[0] + x) * tile[1] + y) * tile[2] + z
                assert perm[j].item() == nat


def test_library_tables_expand_to_the_oracle_mask():
    for text, img, tile, kern in [(226, (13, 30, 45), (13, 3, 3), (1, 9, 9)), (30, (4, 12, 12), (2, 3, 3), (1, 3, 3))]:
        lay = StaLayout(kern, tile, img, text, "cpu")
        L, nb = lay.L, lay.nb
        assert torch.equal(lay.perm.long(), sta.permutation(text, img, tile))
        assert torch.equal(lay.perm.long()[lay.inv.long()], torch.arange(L))
        masks = lay.masks
        step = 5 if nb > 100 else 1  # sample the full-size geometry
        shifts = torch.arange(64)
        for qb in list(range(0, nb, step)) + [nb - 1]:
            rows = torch.arange(qb * 64, min(L, qb * 64 + 64))
            want = sta.token_mask(rows, L, text, img, tile, kern)
            n = lay.kv_cnt[qb].item()
            kbs, slots = lay.kv_idx[qb, :n].long(), lay.kv_slot[qb, :n].long()
            got = torch.zeros(rows.numel(), nb, 64, dtype=torch.bool)
            got[:, kbs[slots < 0]] = True
            part = slots >= 0
            words = masks[slots[part]][:, : rows.numel()]                 # [n_part, rows]
            bits = ((words[:, :, None] >> shifts) & 1).bool()            # [n_part, rows, 64]
            got[:, kbs[part]] = bits.permute(1, 0, 2)
            assert torch.equal(got.reshape(rows.numel(), nb * 64)[:, :L], want), qb
        if img == (13, 30, 45):
            assert lay.n_partial == 8857
            allowed = sum(int(sta.token_mask(torch.arange(r, min(L, r + 2048)), L, text, img, tile, kern).sum())
                          for r in range(0, L, 2048))
            assert abs(allowed / (L * L) - 0.5516) < 1e-4


def test_default_config_matches_reference():
    assert config == {"kernel_size": (1, 9, 9), "tile_size": (13, 3, 3), "img_size": (13, 30, 45), "text_length": 226}
