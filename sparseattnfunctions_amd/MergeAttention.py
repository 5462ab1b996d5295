"""`MergeAttention` processor of special_attentions/MergeAttention.py (:14-51), on MI355X.

Called as `proc(q, k, v) -> out` ([B, H, L, 64] bf16, 226 text tokens first). The forward
re-matches every `gap` calls (:25) -- the step count comes from a module `global_vars`
with a `count` attribute when one is importable, as in the reference (:3, :25), else from
this object's own call counter -- then:
  full_merge=True : q, k, v merged -> attention with the proportional bias log(size) on
                    keys (:33-38) -> unmerge (:41-43);
  full_merge=False: k, v merged, attention of all queries over the merged keys (:45-48).
Matching, merge/unmerge and the biased attention are HIP kernels (`sa_tome_*`,
`sa_block_sparse_fwd` with every key block and a key bias).

Default `merge_config` is BASELINE config 4: head-averaged k metric (metric="head_mean_k"),
2x2 spatial stride, no temporal stride, r = 4000, full merge, the top-left token of each
cell as its dst (no_rand=True). The reference's own setting (metric cat(k, |k|, v, |v|) per
head, 3x3x4 stride, r = 9000, k/v-only merge, a random dst per cell drawn at every re-match
from a generator made at construction, :16-20, :30) is `MergeAttention.reference()`, i.e.
`MergeAttention(REFERENCE_MERGE_CONFIG, full_merge=False, metric="kv_norm", no_rand=False)`.
"""
from __future__ import annotations

import math

import torch

from . import _tome
from .block_mask_attn import dense_kv_list
from .utils.block_sparse_attn_kernel import block_sparse_attention
from .utils.merge_unmerge import draw_cell_choice, init_generator

CONFIG4_MERGE_CONFIG = {"w": 45, "h": 30, "t": 13, "sx": 2, "sy": 2, "st": 1, "r": 4000}
REFERENCE_MERGE_CONFIG = {"w": 45, "h": 30, "t": 13, "sx": 3, "sy": 3, "st": 4, "r": 9000}


def _global_count():
    try:
        import global_vars  # the host pipeline's step counter, as the reference reads it
    except ImportError:
        return None
    return getattr(global_vars, "count", None)


class MergeAttention:
    def __init__(self, merge_config=None, full_merge: bool = True, gap: int = 1, metric: str = "head_mean_k",
                 text_len: int = 226, sm_scale: float = None, no_rand: bool = True,
                 generator: torch.Generator = None):
        if metric not in ("head_mean_k", "kv_norm"):
            raise ValueError("metric must be 'head_mean_k' or 'kv_norm'")
        self.merge_config = dict(merge_config or CONFIG4_MERGE_CONFIG)
        self.full_merge = full_merge
        self.gap = gap
        self.metric = metric
        self.text_len = text_len
        self.sm_scale = sm_scale
        self.no_rand = no_rand
        # The reference seeds its generator from the global RNG of the GPU (the CPU without
        # one) when the processor is built (:19, merge_unmerge.py:8-22).
        if generator is None and not no_rand:
            generator = init_generator(torch.device("cuda" if torch.cuda.is_available() else "cpu"))
        self.generator = generator
        self.cell_choice = None  # dst offsets of the last re-match (None: top-left)
        self.maps = None
        self.calls = 0
        self._kv_cache = {}

    @classmethod
    def reference(cls, **kwargs):
        """The reference's configuration (MergeAttention.py:16-48)."""
        args = dict(merge_config=REFERENCE_MERGE_CONFIG, full_merge=False, metric="kv_norm", no_rand=False)
        args.update(kwargs)
        return cls(**args)

    def _count(self):
        c = _global_count()
        return self.calls if c is None else c

    def build_maps(self, k, v):
        cfg = self.merge_config
        mode = 0 if self.metric == "head_mean_k" else 1
        metric = _tome.metric_from_qkv(k, v if mode == 1 else None, self.text_len, mode)
        # One dst per cell: the top-left token, or a draw from the generator at every re-match
        # (merge_unmerge.py:66-70).
        self.cell_choice = None if self.no_rand else draw_cell_choice(
            cfg["t"], cfg["h"], cfg["w"], cfg["sx"], cfg["sy"], cfg["st"], self.generator)
        a_idx, b_idx = _tome.partition(cfg["t"], cfg["h"], cfg["w"], cfg["sx"], cfg["sy"], cfg["st"], k.device,
                                       cell_choice=self.cell_choice)
        return _tome.match(metric, a_idx, b_idx, cfg["r"], self.text_len)

    def _heads_per_group(self, H):
        return H if self.metric == "head_mean_k" else 1

    def _dense(self, B, H, Lq, Lk, device):
        key = (B, H, Lq, Lk, str(device))
        kv = self._kv_cache.get(key)
        if kv is None:
            kv = dense_kv_list(B, H, math.ceil(Lq / 64), math.ceil(Lk / 64), device)
            self._kv_cache[key] = kv
        return kv

    def forward(self, q, k, v):
        B, H, L, D = q.shape
        if self._count() % self.gap == 0 or self.maps is None:
            self.maps = self.build_maps(k, v)
        self.calls += 1
        maps = self.maps
        hpg = self._heads_per_group(H)
        bias = maps.key_bias.reshape(B, H // hpg, maps.Lm).expand(B, H, maps.Lm) if hpg == H else \
            maps.key_bias.reshape(B, H, maps.Lm)
        scale = self.sm_scale if self.sm_scale is not None else 1.0 / math.sqrt(D)
        if self.full_merge:
            qm, km, vm = _tome.merge_many((q, k, v), maps, hpg)
            om = block_sparse_attention(qm, km, vm, self._dense(B, H, maps.Lm, maps.Lm, q.device), scale,
                                        key_bias=bias)
            return _tome.unmerge(om, maps, hpg)
        km, vm = _tome.merge_many((k, v), maps, hpg)
        return block_sparse_attention(q, km, vm, self._dense(B, H, L, maps.Lm, q.device), scale, key_bias=bias)

    def __call__(self, *args, **kwds):
        return self.forward(*args, **kwds)
