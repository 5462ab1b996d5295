"""MI355X-native (gfx950) sparse-attention hot path of special_attentions.

Module layout mirrors the reference package `special_attentions`
(xiaolong-li1/SparseAttnFunctions): the processor classes and utils keep their module and
class names, and their forward passes run the HIP kernels of libsa_hip.so through the C ABI
in include/sa_api.h. `install_alias()` registers this package under the name
`special_attentions` so that code written against the reference imports it unchanged.
"""
from __future__ import annotations

import importlib
import sys

__all__ = ["install_alias"]

_SUBMODULES = (
    "utils",
    "utils.block_sparse_attn_kernel",
    "utils.merge_unmerge",
    "utils.mask_related",
    "utils.attn_pooling_kernel",
    "utils.tools",
    "block_mask_attn",
    "SparseGen_Plus",
    "combined_attn",
    "MergeAttention",
    "SildingTileAttention",
    "partern_attention",
)


def install_alias(name: str = "special_attentions") -> None:
    """Make `import special_attentions.<module>` resolve to this package's modules."""
    pkg = sys.modules[__name__]
    sys.modules.setdefault(name, pkg)
    for sub in _SUBMODULES:
        mod = importlib.import_module(f"{__name__}.{sub}")
        sys.modules.setdefault(f"{name}.{sub}", mod)
