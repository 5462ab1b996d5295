"""ctypes binding of libsa_hip.so (the C ABI declared in include/sa_api.h).

PyTorch only provides device memory and the current HIP stream; every computation on the
hot path is a HIP kernel of libsa_hip.so. There is no CPU or PyTorch fallback: if the
library is missing, or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsa_hip.so")

ABI_VERSION = 3  # SA_ABI_VERSION of include/sa_api.h these prototypes describe

SA_OK = 0
SA_ERR_INVALID = -1
SA_ERR_UNSUPPORTED = -2
SA_ERR_HIP = -3

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64P = ctypes.POINTER(ctypes.c_int64)
_F = ctypes.c_float

# name -> (restype, argtypes); must match include/sa_api.h.
_PROTOTYPES = {
    "sa_abi_version": (_I, []),
    "sa_last_error": (ctypes.c_char_p, []),
    "sa_mask_to_kv_list": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _I, _P, _P]),
    "sa_mask_cells_to_kv_list": (_I, [_P, _I64P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P]),
    "sa_cell_tile_masks": (_I, [_I, _I, _P, _I64P]),
    "sa_block_pool": (_I, [_P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "sa_block_pool_k16": (_I, [_P, _I64P, _P, _I64P, _I, _I, _I, _I, _P, _P, _P, ctypes.c_int64, _P]),
    "sa_block_topk_kv_list": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P]),
    "sa_block_sparse_fwd": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I64P, _F, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_f16": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I64P, _F, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_v32": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _P, _P, _I, _P, _I64P, _F, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_f32": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I64P, _F, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_tilemask": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P, _F, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_mapped": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P, _P, _I64P, _F,
         _P, _I, _P, _I, _P, ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_mapped_f16": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P, _P, _I64P, _F,
         _P, _I, _P, _I, _P, ctypes.c_int64, _P],
    ),
    "sa_attn_work_order": (_I, [_I, _I, _I, _I, _I, _P, _I64P]),
    "sa_attn_split_parts": (_I, [ctypes.c_int64, _I, _I, _I, ctypes.POINTER(_I)]),
    "sa_attn_split_workspace": (_I, [ctypes.c_int64, _I, _I, _I64P]),
    "sa_block_sparse_fwd_k16_workspace": (_I, [_I, _I, _I, _I, _I, _I64P]),
    "sa_block_sparse_fwd_k16_prepare": (_I, [_P, _I64P, _I, _I, _I, _I, _P, ctypes.c_int64, _P]),
    "sa_block_sparse_fwd_k16": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _I64P, _F, _P,
         ctypes.c_int64, _I, _P, ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_split": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _F, _P, _I, _P, _I, _I, _P,
         ctypes.c_int64, _P],
    ),
    "sa_block_sparse_fwd_split_f16": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _I, _F, _P, _I, _P, _I, _I, _P,
         ctypes.c_int64, _P],
    ),
    "sa_attn_pooling_workspace": (_I, [_I, _I, _I, _I, _I64P]),
    "sa_attn_pooling_fwd": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _I64P, _P,
         ctypes.c_int64, _P],
    ),
    "sa_attn_pooling_fwd_f32": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _I64P, _P,
         ctypes.c_int64, _P],
    ),
    "sa_attn_pooling_fwd_f16": (
        _I,
        [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _I64P, _P,
         ctypes.c_int64, _P],
    ),
    "sa_gather_tokens_heads": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _I, _P, _I64P, _P]),
    "sa_pattern_maps": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _P, _P]),
    "sa_constrained_mod_factor": (_I, [_P, _I, ctypes.c_int64, _F, _F, _P, _P, _P]),
    "sa_sampled_probs": (_I, [_P, _P, _I, _I, _I, _I, _I, _F, _I, _F, _I, _I, _P, ctypes.c_int64, ctypes.c_int64,
                              _P]),
    "sa_topk_share": (_I, [_P, ctypes.c_int64, ctypes.c_int64, _I, _I, _I, _I, _P, _P]),
    "sa_pattern_gram": (_I, [_P, ctypes.c_int64, ctypes.c_int64, _I, _I, _I, _P, _P]),
    "sa_pattern_sim_gram": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _P, _P]),
    "sa_pattern_judge_finish": (_I, [_P, _P, _P, _I, _I, _I, _I, _F, _F, _P, _P, _P, _P, _P]),
    "sa_pattern_plan": (_I, [_P, _I64P, _P, _I, _I, _I, _I, _I, _F, _F, _F, _F, _F, _P, _P, _P, _P, _P, _P]),
    "sa_pattern_combine": (_I, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                _F, _F, _F, _F, _P, _I64P, _P]),
    "sa_row_group_sums": (_I, [_P, _I64P, _I, _I, _I, _I, _I, _I, _P, _P]),
    "sa_kron_block_mask": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "sa_sta_permutation": (_I, [_I, _I, _I, _I, _P, _P]),
    "sa_sta_block_masks": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "sa_gather_tokens": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _I, _P, _I64P, _P]),
    "sa_local_window_bitmap": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "sa_local_window_bitmap_perm": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "sa_sample_block_tokens": (_I, [_P, _P, _I64P, _P, _P, _I64P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "sa_sampled_block_scores": (_I, [_P, _P, _I, _I, _I, _I, _P, _P]),
    "sa_energy_kv_list": (_I, [_P, _I, _I, _I, _I, _F, _I, _I, _I, _I, _P, _I, _P, _P, _P]),
    "sa_tome_partition": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "sa_tome_metric": (_I, [_P, _I64P, _P, _I64P, _I, _I, _I, _I, _I, _I, _P, _P]),
    "sa_tome_normalize": (_I, [_P, ctypes.c_int64, _I, _P, _P]),
    "sa_tome_match_workspace": (_I, [_I, _I, _I, _I64P]),
    "sa_tome_match": (_I, [_P, _I, _P, _P, ctypes.c_int64, _P]),
    "sa_tome_match_noalloc": (_I, [_P, _I, _P, _P]),
    "sa_tome_merge": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _P, _I64P, _P]),
    "sa_tome_merge_multi": (_I, [_I, _P, _I64P, _I, _I, _I, _I, _P, _P, _I64P, _P]),
    "sa_tome_unmerge": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _P, _I64P, _P]),
}

_lib: Optional[ctypes.CDLL] = None


class SAError(RuntimeError):
    """A HIP runtime failure reported by libsa_hip.so."""


def load() -> ctypes.CDLL:
    """Loads libsa_hip.so once and declares the prototypes of every exported entry point."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `make -C sparseattnfunctions_amd/csrc` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(LIB_PATH)
        lib.sa_abi_version.restype = _I
        version = lib.sa_abi_version()
        if version != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI version {version}, the bindings expect {ABI_VERSION}; rebuild it "
                              "with `make -C sparseattnfunctions_amd/csrc`")
        for name, (res, args) in _PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_names() -> Sequence[str]:
    return tuple(_PROTOTYPES)


def check(rc: int, what: str) -> None:
    """Maps a C status to the exception the reference raises for the same condition."""
    if rc == SA_OK:
        return
    msg = load().sa_last_error().decode(errors="replace") or what
    if rc == SA_ERR_INVALID:
        raise ValueError(msg)
    if rc == SA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise SAError(msg)


def i64(*vals: int):
    return (ctypes.c_int64 * len(vals))(*[int(x) for x in vals])


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_SIDE = {}


def side_stream(device) -> "torch.cuda.Stream":
    """The package's second stream on `device` (default priority), created once: work that
    runs beside the current stream's, ordered with it by wait_stream / events."""
    key = str(torch.device(device))
    s = _SIDE.get(key)
    if s is None:
        s = _SIDE[key] = torch.cuda.Stream(device=device)
    return s


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of the tensor's device (hipStream_t as an integer)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                "special_attentions (MI355X build) runs on the GPU only; got a tensor on "
                f"{t.device}. There is no CPU path."
            )
