"""MI355X-native tree-verification path for CAST-style speculative decoding.

    import cast_amd
    nodes = cast_amd.build_tree(top_idx, top_lp, 127)          # host, numpy
    out = cast_amd.varlen_tree_attention(q, k, v, cu_q, cu_kv,  # HIP, gfx950
                                         prefix_len, pack_len, ancestor_mask)
    path, bonus = cast_amd.walk_tree(nodes, logits)            # HIP, gfx950

Mirrors the package facade of cast_trees/__init__.py:17-36: the tree layout
names import with numpy only; the device names load the HIP library on first
use (PEP 562) and raise if it is missing.
"""
from __future__ import annotations

__version__ = "0.1.0"

from .tree import (MAX_PACK, PackedTrees, TreeNode, ancestor_matrix, block_topk, build_chain,
                   build_tree, expected_accepted_length, pack_trees, select_global_topk)

_LAZY = {
    "varlen_tree_attention": "tree_attn",
    "TreeAttnPlan": "tree_attn",
    "tree_bitmask": "verify",
    "greedy_accept": "verify",
    "walk_tree": "verify",
    "walk_trees": "verify",
    "tree_attention_mask": "verify",
    "cache_layers": "verify",
    "gather_cache": "verify",
    "topk_marginals": "draft",
    "build_trees": "draft",
    "build_tree_device": "draft",
}

__all__ = ["__version__", "MAX_PACK", "PackedTrees", "TreeNode", "ancestor_matrix", "block_topk",
           "build_chain", "build_tree", "expected_accepted_length", "pack_trees",
           "select_global_topk", *_LAZY]


def __getattr__(name):
    """Device-side names: import their module on first use and keep the
    result in this module's namespace, so the hook runs once per name."""
    home = _LAZY.get(name)
    if home is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    import importlib
    value = getattr(importlib.import_module(f"{__name__}.{home}"), name)
    globals()[name] = value
    return value


def __dir__():
    return list(__all__)    # dir() sorts
