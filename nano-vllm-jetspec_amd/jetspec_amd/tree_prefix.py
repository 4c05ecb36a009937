"""Entries of speculative/jetspec/tree_prefix.py (prefix-address specialisations).

The reference's prefix variants specialise how a prefix key's page is looked up and keep
FP32 probabilities; this kernel always addresses whole prefix tiles from page bases, so
every variant is the same launch in the exact-probability mode.  Page sizes that are not multiples of 64 go to the reference entry,
as tree_prefix.py:134-137 does.
"""
from __future__ import annotations

from .paged_backend import _launch, _launch_new, _validate
from .tree_attention import packed_tree_attention_reference


def _num_warps(num_warps) -> None:
    if isinstance(num_warps, bool) or num_warps not in (4, 8, 16):
        raise ValueError("num_warps must be 4, 8 or 16")


def packed_tree_attention_prefix(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *, output_dtype=None,
                                 num_warps=4):
    """tree_prefix.py:123-157."""
    _num_warps(num_warps)
    if metadata.block_size % 64:
        return packed_tree_attention_reference(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                               output_dtype=output_dtype)
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    return _launch_new(q, k_pool, v_pool, metadata, scale, dtype, exact=True)


def packed_tree_attention_prefix_single_loop(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *,
                                             output_dtype=None, num_warps=4):
    """tree_prefix.py:266-300."""
    return packed_tree_attention_prefix(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                        output_dtype=output_dtype, num_warps=num_warps)


def packed_tree_attention_prefix_split_exact(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *,
                                             output_dtype=None, num_warps=4):
    """tree_prefix.py:444-463."""
    return packed_tree_attention_prefix(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                        output_dtype=output_dtype, num_warps=num_warps)


def packed_tree_attention_prefix_prevalidated(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, out, *,
                                              num_warps=4):
    """Launch-only entry (tree_prefix.py:466-492): the caller validated and allocated `out`.
    Like the reference's split-exact kernel it keeps FP32 probabilities."""
    return _launch(q, k_pool, v_pool, metadata, scale, out, exact=True)
