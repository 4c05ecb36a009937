"""Incremental prefill chunks on the tree-verify path (speculative/jetspec/prefill.py:14-26).

A prefill chunk of C rows whose first query sits at logical position P lets query j see every
key at position <= P + j.  That is the visibility of a chain tree of C nodes (node j's parent is
j - 1) over a P-key prefix: all prefix keys, then tree nodes 0..j.  So the reference's dense
chunk attention (models/qwen3.py:566-618: a per-layer gather of the context, then SDPA under
``offset_causal_mask``) is the packed tree attention of a chain tree, one launch over the paged
pool, with the chunk's K/V rows in their slots (``chain_tree_masks`` builds the masks for
``PackedTreeMetadata.build``).
"""
from __future__ import annotations

from typing import Sequence

import torch


def offset_causal_mask(prefix_length: int, chunk_length: int, device) -> torch.Tensor | None:
    """prefill.py:14-26: SDPA bool visibility of shape [C, P + C] (True = visible) for a chunk of
    C queries starting at position P; None when P is 0 (the reference then keeps the plain
    causal full-prefill call).  Query j sees key k iff k - j <= P."""
    if prefix_length < 0 or chunk_length < 1:
        raise ValueError("invalid incremental attention lengths")
    if prefix_length == 0:
        return None
    offsets = (torch.arange(prefix_length + chunk_length, device=device).unsqueeze(0)
               - torch.arange(chunk_length, device=device).unsqueeze(1))
    return offsets <= prefix_length


def chain_tree_masks(chunk_lengths: Sequence[int], device) -> list[torch.Tensor]:
    """Self-inclusive ancestor masks of chain trees (node j sees nodes 0..j), one per chunk: the
    tree part of a chunk's visibility, for ``PackedTreeMetadata.build``."""
    masks = []
    for n in chunk_lengths:
        if n < 1:
            raise ValueError("invalid incremental attention lengths")
        masks.append(torch.ones((n, n), dtype=torch.bool, device=device).tril())
    return masks
