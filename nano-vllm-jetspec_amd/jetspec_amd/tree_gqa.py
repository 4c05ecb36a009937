"""Entry of speculative/jetspec/tree_gqa.py (the reference's grouped bf16-P serving kernel).

``packed_tree_attention(..., backend="gqa")`` dispatches here, as paged_backend.py:273-276
does.  The kernel's own design already is KV-head-centric with bf16 probabilities in the
P.V product (tree_gqa.py:102-105); ``fp32_probability=True`` selects the kernel's exact
probability mode (the reference's FP32_P switch), and the tiling switches are validated
and fixed.
"""
from __future__ import annotations

import torch

from .paged_backend import _launch_new, _validate


def packed_tree_attention_gqa(q, k_pool, v_pool, metadata, scale, num_queries_per_kv, *, output_dtype=None,
                              query_tile=4, prefix_scalar=True, prune=True, fp32_probability=False):
    """tree_gqa.py:114-140."""
    if query_tile not in (1, 4) or isinstance(query_tile, bool):
        raise ValueError("GQA query tile must be 1 or 4")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("grouped Tensor Core tree attention requires BF16 or FP16")
    if num_queries_per_kv not in (1, 2, 4, 8, 16):
        raise ValueError("grouped tree attention requires power-of-two GQA <=16")
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    return _launch_new(q, k_pool, v_pool, metadata, scale, dtype, exact=bool(fp32_probability))
