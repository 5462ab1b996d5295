"""Writes tests/golden/input_hashes.json: sha256 of the bf16 (fp32 for config 1) bytes of the
synthetic benchmark inputs, so that the inputs the benchmark and the parity tests use are
pinned. Run from the repo root: python tests/golden/make_input_hashes.py"""
import hashlib
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from sparseattnfunctions_amd.workloads import cogvideox_qkv, config1_inputs  # noqa: E402


def sha(t: torch.Tensor) -> str:
    t = t.contiguous()
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.bfloat16
                          else t.view(torch.int16).numpy().tobytes()).hexdigest()


def hashes() -> dict:
    out = {}
    q, k, v, mask, _ = config1_inputs()
    out["config1"] = {"q": sha(q), "k": sha(k), "v": sha(v), "mask": sha(mask.to(torch.uint8))}
    for name, seed in (("config2_3_5", 0), ("config4", 3)):
        q, k, v = cogvideox_qkv(seed)
        out[name] = {"seed": seed, "shape": list(q.shape), "q": sha(q), "k": sha(k), "v": sha(v)}
    return out


if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "input_hashes.json")
    with open(path, "w") as f:
        json.dump(hashes(), f, indent=1)
    print("wrote", path)
