"""After install_alias(), code written against the reference imports the names it uses from
`special_attentions.*` (the module, class and function names of the reference's modules on the
hot path). No GPU calls."""
import importlib

import pytest
import torch

import sparseattnfunctions_amd

# Public names of the reference modules (special_attentions/...), as defined there.
NAMES = {
    "utils.block_sparse_attn_kernel": ["is_hip", "get_sparse_attn_mask_from_topk",
                                       "get_sparse_attn_mask_from_threshold", "_forward", "_sparse_attention",
                                       "sparse_attention_factory", "block_sparse_triton_fn"],
    "utils.merge_unmerge": ["do_nothing", "init_generator", "bipartite_soft_matching_video"],
    "utils.mask_related": ["pad_to_multiple", "random_sample_tokens", "calc_attn_block_sum_efficient",
                           "preprocess_qkv", "reverse_process_out", "generate_attention_mask_frame_scope",
                           "calc_attn", "get_inner_frame_mask", "get_block_mask"],
    "utils.attn_pooling_kernel": ["is_hip", "_attention_pooling", "attn_with_pooling"],
    "utils.tools": ["timeit", "preserve_rng_state"],
    "block_mask_attn": ["BlockSparseAttention"],
    "SparseGen_Plus": ["transfer_attn_to_mask", "concentrated_interpolation", "BlockSparseAttention"],
    "combined_attn": ["CombinedAttn"],
    "MergeAttention": ["MergeAttention"],
    "SildingTileAttention": ["generate_sta_mask", "get_sliding_tile_attention_mask", "SildingTileAttention"],
    "partern_attention": ["get_indexs", "sample_rate", "composition", "scale_factor", "constrained_mod_factor",
                          "ParternAttentionColVersion_V2", "get_softmax", "judge_sparsity", "judge_similarity",
                          "unified_judge"],
}


@pytest.mark.parametrize("module", sorted(NAMES))
def test_reference_names_import_through_alias(module):
    sparseattnfunctions_amd.install_alias()
    mod = importlib.import_module(f"special_attentions.{module}")
    missing = [n for n in NAMES[module] if not hasattr(mod, n)]
    assert not missing, missing
    exec(f"from special_attentions.{module} import {', '.join(NAMES[module])}", {})


def test_preserve_rng_state_restores_generator_and_timeit_prints(capsys):
    from sparseattnfunctions_amd.utils.tools import preserve_rng_state, timeit

    @preserve_rng_state
    def draw():
        return torch.rand(3)

    torch.manual_seed(11)
    inside = draw()
    after = torch.rand(3)
    torch.manual_seed(11)
    assert torch.equal(inside, torch.rand(3)) and torch.equal(after, inside)

    @preserve_rng_state
    def fails():
        torch.rand(5)
        raise ValueError("x")

    torch.manual_seed(12)
    with pytest.raises(ValueError):
        fails()
    got = torch.rand(2)
    torch.manual_seed(12)
    assert torch.equal(got, torch.rand(2))

    @timeit
    def twice(x):
        return 2 * x

    assert twice(21) == 42
    out = capsys.readouterr().out
    assert out.startswith("twice execution took ") and out.rstrip().endswith("ms")
