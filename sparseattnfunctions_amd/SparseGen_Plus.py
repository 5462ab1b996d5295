"""Adaptive block-sparse attention of special_attentions/SparseGen_Plus.py (:12-212), on MI355X.

  * `transfer_attn_to_mask(attn, mode, init_k, max_retain_ratio, min_retain_ratio,
    energy_threshold)` (:12-84): per block-score row, the energy-threshold prefix ("energy")
    or the adaptive top-k ("topk"), text rows/columns forced dense (:81-82). Returns the
    bool mask [B, H, S, S] like the reference; `transfer_attn_to_kv_list` returns the kv
    lists the attention kernel consumes.
  * `concentrated_interpolation` (:85-104): the per-step schedule tables.
  * `BlockSparseAttention(block_size, layernum, timestep, num_samples, warmup_epoch)`
    (:105-212): dense warm-up steps, then per call the sampled estimator
    (calc_attn_block_sum_efficient, num_keep=8), the energy mask with the step's schedule and
    the block-sparse kernel; sparsity records per call, saved as JSON after each sample.

Every tensor operation runs in HIP kernels of libsa_hip.so. Differences from the reference,
by design:
  * the warm-up steps run dense attention through the same kernel (every block kept) instead
    of SageAttention's quantized kernel, which this build does not ship;
  * block scores are fp32 (see utils/mask_related.py of this package);
  * `mask[layer]` gives the bool block mask built from the cached kv lists (`mask.kv(layer)`).
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

from ._kv import KVList, kv_list_from_mask
from .block_mask_attn import dense_kv_list
from .estimator import energy_kv_list
from .utils.block_sparse_attn_kernel import block_sparse_attention
from .utils.mask_related import calc_attn_block_sum_efficient
from .utils.tools import rng_state_preserved

N_TEXT_BLOCKS = 4  # the reference forces rows and columns 0..3 (:81-82)


def transfer_attn_to_kv_list(attn, mode="energy", init_k=None, max_retain_ratio=0.7, min_retain_ratio=0.1,
                             energy_threshold=0.95) -> KVList:
    return energy_kv_list(attn, mode, init_k, max_retain_ratio, min_retain_ratio, energy_threshold,
                          n_text_blocks=N_TEXT_BLOCKS)


def transfer_attn_to_mask(attn, mode="energy", init_k=None, max_retain_ratio=0.7, min_retain_ratio=0.1,
                          energy_threshold=0.95) -> torch.Tensor:
    """Block scores [B, H, S, S] -> bool mask of the same shape."""
    _, mask = energy_kv_list(attn, mode, init_k, max_retain_ratio, min_retain_ratio, energy_threshold,
                             n_text_blocks=N_TEXT_BLOCKS, return_mask=True)
    return mask


def concentrated_interpolation(min_val, max_val, n_points, concentration=0.2):
    """n_points values from max_val down to min_val along a logistic curve, denser near both
    ends the higher `concentration` (clipped to [0.05, 0.95])."""
    c = float(np.clip(concentration, 0.05, 0.95))
    x = np.linspace(-6, 6, n_points)
    cdf = 1 / (1 + np.exp(-x / (2 * (1 - c))))
    return np.clip(max_val - cdf * (max_val - min_val), min_val, max_val)


class LayerMasks:
    """Per-layer cache of the last sparse step's block masks (the reference's `self.mask`
    list, SparseGen_Plus.py:117, 165-172). Item access returns the reference's bool
    [B, H, nqb, nkb] block mask (None before the layer's first sparse step), formed from the
    kv lists the kernel uses; `kv(layer)` returns those lists. A bool/0-1 mask assigned to
    an item is converted to kv lists."""

    def __init__(self, n: int):
        self._kv = [None] * n

    def __len__(self):
        return len(self._kv)

    def __getitem__(self, layer):
        kv = self._kv[layer]
        return None if kv is None else kv.to_mask()

    def __setitem__(self, layer, value):
        if value is None or isinstance(value, KVList):
            self._kv[layer] = value
            return
        B, H, nqb, nkb = value.shape
        self._kv[layer] = kv_list_from_mask(value, B, H, nqb, nkb)

    def __iter__(self):
        return (self[i] for i in range(len(self)))

    def kv(self, layer):
        return self._kv[layer]


class BlockSparseAttention:
    def __init__(self, block_size=64, layernum=42, timestep=50, num_samples=1, warmup_epoch=5,
                 verbose=True, record_dir="."):
        if block_size != 64:
            raise NotImplementedError("the MI355X kernel uses 64-token blocks")
        self.block_size = block_size
        self.sm_scale = 1 / 8
        self.layernum = layernum
        self.timestep = timestep
        self.num_samples = num_samples
        self.counter = 0
        self.sparsity_records = [self._init_sparsity_dict() for _ in range(num_samples)]
        self.update_list = []
        self.warmup_epoch = warmup_epoch
        self.mask = LayerMasks(layernum)
        self.k_list = [0.3, 0.2, 0.15, 0.1]
        self.max_retain_ratio_list = concentrated_interpolation(0.8, 1, 50, concentration=0.5)
        self.min_retain_ratio_list = concentrated_interpolation(0.1, 0.12, 50, concentration=0.5)
        self.energy_threshold_list = concentrated_interpolation(0.9, 0.98, 50, concentration=0.5)
        self.verbose = verbose
        self.record_dir = record_dir

    def _init_sparsity_dict(self):
        return {"records": []}

    def _calculate_sparsity(self, kv: KVList):
        """Fraction of skipped blocks; with B == 1 the reference scores the layer as if the
        other 96 - H heads were 90 % sparse (:126-132)."""
        kept = kv.cnt.sum().item() / (kv.rows * kv.nkb)
        if kv.B == 1:
            return ((1 - kept) * kv.H + 0.9 * (96 - kv.H)) / 96
        return 1 - kept

    def _record_sparsity(self, sample_idx, timestep, layeridx, sparsity):
        self.sparsity_records[sample_idx]["records"].append(
            {"timestep": timestep, "layer": layeridx, "sparsity": sparsity})
        if self.verbose:
            print(f"Sample {sample_idx}, Timestep {timestep}, Layer {layeridx}: Sparsity = {sparsity:.4f}")

    def _save_sparsity_records(self, sample_idx):
        filename = os.path.join(self.record_dir, f"sparsity_record_sample_{sample_idx}.json")
        with open(filename, "w") as f:
            json.dump(self.sparsity_records[sample_idx], f, indent=4)

    def _schedule(self):
        counter = self.counter % (self.layernum * self.timestep)
        step = counter // self.layernum
        return (counter % self.layernum, self.max_retain_ratio_list[step], self.min_retain_ratio_list[step],
                self.energy_threshold_list[step], self.k_list[step] if step < 4 else 0.1)

    def forward(self, q, k, v):
        """Sparse step: sampled block scores -> energy mask -> block-sparse attention."""
        self.sm_scale = 1 / q.size(-1) ** 0.5
        layer, max_r, min_r, thr, cur_k = self._schedule()
        with rng_state_preserved():
            pool = calc_attn_block_sum_efficient(q, k, num_keep=8)
        kv = transfer_attn_to_kv_list(pool, mode="energy", init_k=cur_k, max_retain_ratio=max_r,
                                      min_retain_ratio=min_r, energy_threshold=thr)
        self.mask[layer] = kv
        out = block_sparse_attention(q, k, v, kv, self.sm_scale, n_text_blocks=N_TEXT_BLOCKS)
        sparsity = self._calculate_sparsity(kv)
        self._record_sparsity(self.counter // (self.layernum * self.timestep), self.counter // self.layernum,
                              self.counter % self.layernum, sparsity)
        return out

    def forward_dense(self, q, k, v):
        B, H, L, _ = q.shape
        kv = dense_kv_list(B, H, math.ceil(L / 64), math.ceil(k.shape[2] / 64), q.device)
        return block_sparse_attention(q, k, v, kv, 1 / q.size(-1) ** 0.5)

    def need_update(self, counter):
        return (counter // self.layernum) in self.update_list

    def __call__(self, q, k, v):
        counter = self.counter % (self.layernum * self.timestep)
        if counter // self.layernum < self.warmup_epoch:
            out = self.forward_dense(q, k, v)
        else:
            out = self.forward(q, k, v)
        self.counter += 1
        if self.need_update(self.counter):
            self.mask = LayerMasks(self.layernum)
        if self.counter % (self.layernum * self.timestep) == 0:
            sample_idx = self.counter // (self.layernum * self.timestep) - 1
            self._save_sparsity_records(sample_idx)
            if self.verbose:
                print(f"save_sparsity_records to sparsity_record_sample_{sample_idx}.json")
        return out
