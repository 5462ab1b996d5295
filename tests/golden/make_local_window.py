"""Writes tests/golden/local_window_cogvideox2b.npy: the static config-3 local-window bitmap
(centre-token rule, +-1 latent frame, +-8 patch rows and columns) of the CogVideoX-2B
geometry (226 text + 13 x 30 x 45 video tokens, 278 blocks of 64), bit-packed row-major with
numpy.packbits. Computed with the CPU oracle (oracle/sa_oracle.c, oracle_local_window),
which tests/test_oracle_local.py pins against brute-force token enumeration.
Run from the repo root after `make -C oracle`: python tests/golden/make_local_window.py"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from oracle import native  # noqa: E402
from sparseattnfunctions_amd.workloads import COGVIDEOX_2B  # noqa: E402

WINDOW = (1, 8, 8)

if __name__ == "__main__":
    bm = native.local_window(COGVIDEOX_2B, *WINDOW).numpy().astype(np.uint8)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "local_window_cogvideox2b.npy")
    np.save(path, np.packbits(bm.reshape(-1)))
    print("wrote", path, bm.shape, int(bm.sum()))
