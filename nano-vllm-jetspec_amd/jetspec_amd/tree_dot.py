"""Entry of speculative/jetspec/tree_dot.py (the reference's matrix-core precision experiment,
TF32x3 products with FP32 probabilities): the kernel's exact-probability mode."""
from __future__ import annotations

from .paged_backend import _launch_new, _validate
from .tree_attention import packed_tree_attention_reference


def packed_tree_attention_dot(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *, output_dtype=None,
                              query_tile=4, num_warps=4):
    """tree_dot.py:105-144; a non-power-of-two grouping goes to the reference entry, as there."""
    if isinstance(query_tile, bool) or query_tile not in (1, 2, 4, 8):
        raise ValueError("query_tile must be 1, 2, 4 or 8")
    if isinstance(num_warps, bool) or num_warps not in (4, 8, 16):
        raise ValueError("num_warps must be 4, 8 or 16")
    if (isinstance(num_queries_per_kv, int) and not isinstance(num_queries_per_kv, bool)
            and num_queries_per_kv > 0 and num_queries_per_kv & (num_queries_per_kv - 1)):
        return packed_tree_attention_reference(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                               output_dtype=output_dtype)
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    return _launch_new(q, k_pool, v_pool, metadata, scale, dtype, exact=True)
