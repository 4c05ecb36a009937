"""Every operator entry of the reference's module layout, resolved by name (CPU).

The qualification harness picks candidates as ``module:function`` and requires an
``output_dtype`` keyword (benchmarks/jetspec_tree_kernel_qualification.py:33-55).  Here
every entry of tree_attention / tree_gqa / tree_dot / tree_prefix resolves that way
inside ``jetspec_amd``, and each one's own knob validation raises the reference's
ValueError before anything touches a device.
"""
from __future__ import annotations

import importlib
import inspect

import pytest
import torch

ENTRIES = [
    "tree_attention:packed_tree_attention_reference",
    "tree_attention:packed_tree_attention_gqa",
    "tree_attention:packed_tree_attention_register_tuned",
    "tree_gqa:packed_tree_attention_gqa",
    "tree_dot:packed_tree_attention_dot",
    "tree_prefix:packed_tree_attention_prefix",
    "tree_prefix:packed_tree_attention_prefix_single_loop",
    "tree_prefix:packed_tree_attention_prefix_split_exact",
    "paged_backend:packed_tree_attention",
]


def candidate_entry(candidate):
    """The harness's resolver (jetspec_tree_kernel_qualification.py:33-44), rooted at jetspec_amd."""
    module_name, function_name = candidate.split(":", 1)
    module = importlib.import_module("jetspec_amd." + module_name)
    function = getattr(module, function_name)
    if not callable(function) or "output_dtype" not in inspect.signature(function).parameters:
        raise ValueError("candidate must expose explicit output_dtype for pre-BF16 qualification")
    return function


@pytest.mark.parametrize("candidate", ENTRIES)
def test_entry_resolves_with_output_dtype(candidate):
    candidate_entry(candidate)


def _cpu_operands():
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    pool = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    return q, pool, pool


KNOB_ERRORS = [
    ("tree_attention:packed_tree_attention_gqa", {"query_tile": 3}, "query_tile must be 1, 2 or 4"),
    ("tree_attention:packed_tree_attention_gqa", {"num_warps": 2}, "num_warps must be 4, 8 or 16"),
    ("tree_attention:packed_tree_attention_gqa", {"query_tile": True}, "query_tile must be 1, 2 or 4"),
    ("tree_attention:packed_tree_attention_register_tuned", {"maxnreg": 100}, "maxnreg must be 64, 80, 96, 112 or 128"),
    ("tree_gqa:packed_tree_attention_gqa", {"query_tile": 2}, "GQA query tile must be 1 or 4"),
    ("tree_dot:packed_tree_attention_dot", {"query_tile": 16}, "query_tile must be 1, 2, 4 or 8"),
    ("tree_dot:packed_tree_attention_dot", {"num_warps": 32}, "num_warps must be 4, 8 or 16"),
    ("tree_prefix:packed_tree_attention_prefix", {"num_warps": 5}, "num_warps must be 4, 8 or 16"),
    ("tree_prefix:packed_tree_attention_prefix_single_loop", {"num_warps": 5}, "num_warps must be 4, 8 or 16"),
    ("tree_prefix:packed_tree_attention_prefix_split_exact", {"num_warps": 5}, "num_warps must be 4, 8 or 16"),
    ("paged_backend:packed_tree_attention", {"backend": "triton"},
     "tree attention backend must be auto, reference, prefix or gqa"),
    ("paged_backend:packed_tree_attention", {"output_dtype": torch.float16},
     "output dtype must match input or be FP32 for qualification"),
]


@pytest.mark.parametrize("candidate,options,message", KNOB_ERRORS)
def test_entry_knob_validation(candidate, options, message):
    q, k, v = _cpu_operands()
    with pytest.raises(ValueError, match=message):
        candidate_entry(candidate)(q, k, v, None, 128 ** -0.5, 4, **options)


def test_grouped_entry_requires_half_precision_before_geometry():
    """tree_gqa.py:123-126: dtype and grouping are checked before the metadata."""
    from jetspec_amd.tree_gqa import packed_tree_attention_gqa

    q = torch.zeros(2, 32, 128, dtype=torch.float32)
    with pytest.raises(ValueError, match="requires BF16 or FP16"):
        packed_tree_attention_gqa(q, q, q, None, 1.0, 4)
    q = q.to(torch.bfloat16)
    with pytest.raises(ValueError, match="power-of-two GQA <=16"):
        packed_tree_attention_gqa(q, q, q, None, 1.0, 3)


def test_legacy_entry_rejections_before_any_device_work():
    """paged_backend.py:323-325: more than one sequence is refused; the block-table form (no
    logical slots or no bias) runs the external jetspec kernel, which this build lacks."""
    from jetspec_amd import paged_tree_attention

    q, k, v = _cpu_operands()
    with pytest.raises(ValueError, match="multi-request tree verification requires explicit PackedTreeMetadata"):
        paged_tree_attention(q, k, v, None, None, torch.zeros(2), None, 1.0, 4, 256)
    with pytest.raises(ValueError, match="external jetspec kernel"):
        paged_tree_attention(q, k, v, None, None, torch.zeros(1), None, 1.0, 4, 256)


def test_kernel_choice_follows_the_mfma_geometry():
    """The drop-in's per-batch kernel choice (host logic): the MFMA kernel for bf16/f16,
    head_dim 128 with 1-8 or 16 query heads per KV head or head_dim 64 or 256 with 1, 2, 4, 8 or 16,
    page sizes that are multiples of 32, trees of at most 2048 nodes and 16-byte aligned K/V
    rows; the FP32 kernel otherwise."""
    from types import SimpleNamespace

    from jetspec_amd.paged_backend import _mfma_geometry

    def case(*, dtype=torch.bfloat16, groups=4, head_dim=128, block=256, nodes=(64,), kv=8, pool=None):
        q = torch.zeros(2, groups * kv, head_dim, dtype=dtype)
        k = torch.zeros(4, block, kv, head_dim, dtype=dtype) if pool is None else pool
        meta = SimpleNamespace(block_size=block, node_counts_host=tuple(nodes))
        return _mfma_geometry(q, k, k, meta)

    assert case()
    assert case(dtype=torch.float16)
    for groups in (1, 2, 3, 5, 6, 7, 8, 16):
        assert case(groups=groups), groups
    assert case(nodes=(1024, 3)) and case(nodes=(2048, 1025)) and case(block=32) and case(block=512)
    assert not case(dtype=torch.float32)
    for groups in (9, 12, 32):
        assert not case(groups=groups), groups
    for head_dim in (64, 256):
        for groups in (1, 2, 4, 8, 16):
            assert case(head_dim=head_dim, groups=groups), (head_dim, groups)
        for groups in (3, 5, 6, 7):
            assert not case(head_dim=head_dim, groups=groups), (head_dim, groups)
    for head_dim in (32, 96, 512):
        assert not case(head_dim=head_dim), head_dim
    assert not case(block=16) and not case(block=48)
    assert not case(nodes=(64, 2049))
    wide = torch.zeros(4, 256, 8, 256, dtype=torch.bfloat16)
    assert not case(pool=wide[..., ::2])                     # strided head dimension
    assert not case(pool=wide[..., 1:129])                   # rows not 16-byte aligned
    assert case(pool=wide[..., 128:])                        # aligned view of a wider row
