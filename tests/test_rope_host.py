"""Host-side contract of rope_scatter (CPU): the reference's rejection cases
(tests/test_jetspec_tree_fusion.py:75-106) raise before anything is launched."""
from __future__ import annotations

import pytest
import torch

from jetspec_amd import rope_scatter


def fixture(dim=128):
    g = torch.Generator().manual_seed(740319)
    q = torch.randn(7, 8, dim, generator=g).to(torch.bfloat16)
    k = torch.randn(7, 2, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(7, 2, dim, generator=g).to(torch.bfloat16)
    positions = torch.tensor([0, 1, 127, 255, 513, 1023, 2047])
    slots = torch.tensor([257, 1, 767, 256, 0, 513, 511])
    cache = torch.randn(2048, 1, dim)
    pools = torch.randn(2, 4, 256, 2, dim, generator=g).to(torch.bfloat16)
    return [q, k, v, positions, cache, pools[0], pools[1], slots]


def test_cpu_invocation_cannot_launch():
    with pytest.raises(ValueError, match="CUDA tensors"):
        rope_scatter(*fixture())


@pytest.mark.parametrize("dim", [1, 127, 258])
def test_odd_or_too_large_head_dimension_is_rejected(dim):
    args = fixture()
    args[:3] = [torch.empty(7, heads, dim, dtype=torch.bfloat16) for heads in (8, 2, 2)]
    with pytest.raises(ValueError, match="even head geometry"):
        rope_scatter(*args)


def test_qkv_dtype_and_grouping_mismatch_is_rejected():
    args = fixture()
    args[1] = args[1].float()
    with pytest.raises(ValueError, match="matching BF16 or FP32"):
        rope_scatter(*args)
    args = fixture()
    args[0] = args[0][:, :3]
    with pytest.raises(ValueError, match="GQA"):
        rope_scatter(*args)


@pytest.mark.parametrize("index", [3, 7])
def test_bad_integer_vector_is_rejected(index):
    args = fixture()
    args[index] = args[index].float()
    with pytest.raises(ValueError, match="integer"):
        rope_scatter(*args)


def test_bad_cache_layout_is_rejected():
    args = fixture()
    args[4] = args[4].expand(-1, 2, -1)
    with pytest.raises(ValueError, match="cos/sin cache"):
        rope_scatter(*args)
