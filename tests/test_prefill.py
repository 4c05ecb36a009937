"""Prefill chunks as chain trees (speculative/jetspec/prefill.py:14-26) on the CPU.

offset_causal_mask is pinned by its closed form, query j of a chunk at position P sees key
k iff k <= P + j, computed here by brute force, and by the reference's contract (None at
P = 0, ValueError on invalid lengths).  The chain-tree visibility the packed kernel applies
(every prefix key, then the chain's self-inclusive ancestors from workloads.ancestor_mask of a
parent array, independent of chain_tree_masks) must equal it for every (P, C).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from jetspec_amd import chain_tree_masks, offset_causal_mask, workloads


@pytest.mark.parametrize("prefix,chunk", [(1, 1), (5, 3), (255, 16), (256, 64), (300, 512), (4097, 7)])
def test_offset_causal_mask_matches_brute_force_and_chain_visibility(prefix, chunk):
    mask = offset_causal_mask(prefix, chunk, "cpu")
    assert mask.dtype == torch.bool and tuple(mask.shape) == (chunk, prefix + chunk)
    brute = np.array([[k <= prefix + j for k in range(prefix + chunk)] for j in range(chunk)])
    assert np.array_equal(mask.numpy(), brute)
    chain = workloads.ancestor_mask(workloads.chain_parents(chunk))
    visibility = np.concatenate((np.ones((chunk, prefix), dtype=bool), chain), axis=1)
    assert np.array_equal(mask.numpy(), visibility)
    assert np.array_equal(chain_tree_masks([chunk], "cpu")[0].numpy(), chain)


def test_offset_causal_mask_contract():
    assert offset_causal_mask(0, 9, "cpu") is None
    for prefix, chunk in ((-1, 4), (3, 0), (0, 0)):
        with pytest.raises(ValueError, match="invalid incremental attention lengths"):
            offset_causal_mask(prefix, chunk, "cpu")
    with pytest.raises(ValueError, match="invalid incremental attention lengths"):
        chain_tree_masks([4, 0], "cpu")
