"""Explicit operator entries of speculative/jetspec/tree_attention.py, on the one HIP kernel.

The qualification harness resolves candidates as ``module:function`` and requires an
``output_dtype`` keyword (benchmarks/jetspec_tree_kernel_qualification.py:33-55); these
entries keep the reference's names, keywords and ValueError messages, and its numerics
contract: FP32 probabilities (the kernel's exact-probability mode), never bf16 ones
(tree_attention.py:1-10).  Their tiling knobs (query tile, warps, register cap) are
CUDA/Triton launch parameters that do not exist on this kernel: they are validated as
the reference validates them and then fixed by the kernel.
"""
from __future__ import annotations

from .paged_backend import _launch_new, _validate


def packed_tree_attention_reference(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *,
                                    output_dtype=None):
    """tree_attention.py:40-62 (explicit FP32 output supported)."""
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    return _launch_new(q, k_pool, v_pool, metadata, scale, dtype, exact=True)


def packed_tree_attention_gqa(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *, output_dtype=None,
                              query_tile=1, num_warps=4):
    """tree_attention.py:138-167: grouped-head reuse of the paged K/V (every entry here groups heads)."""
    if isinstance(query_tile, bool) or query_tile not in (1, 2, 4):
        raise ValueError("query_tile must be 1, 2 or 4")
    if isinstance(num_warps, bool) or num_warps not in (4, 8, 16):
        raise ValueError("num_warps must be 4, 8 or 16")
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    return _launch_new(q, k_pool, v_pool, metadata, scale, dtype, exact=True)


def packed_tree_attention_register_tuned(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *,
                                         output_dtype=None, maxnreg=96):
    """tree_attention.py:170-203; the register cap is a CUDA knob with no meaning here."""
    if isinstance(maxnreg, bool) or maxnreg not in (64, 80, 96, 112, 128):
        raise ValueError("maxnreg must be 64, 80, 96, 112 or 128")
    return packed_tree_attention_reference(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                           output_dtype=output_dtype)
