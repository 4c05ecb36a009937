"""Every named operator entry on the GPU, called the way the qualification harness calls it.

benchmarks/jetspec_tree_kernel_qualification.py:33-55 resolves ``module:function``,
passes ``query_tile`` / ``num_warps`` only when the entry takes them, and an explicit
``output_dtype``.  Each entry here runs on the reference's NaN-poisoned fixture and
must meet the north-star gate against the fp64 oracle, with bf16 and with FP32 output;
the FP32 output rounded to bf16 equals the bf16 output bit for bit (one kernel, one
arithmetic).  The dispatcher's backend names route to the same entries.
"""
from __future__ import annotations

import inspect

import pytest
import torch

from gpu_helpers import assert_within_gate, oracle_rows
from jetspec_amd import packed_tree_attention, read_and_clear_status
from test_attention_gpu import reference_fixture
from test_entries import ENTRIES, candidate_entry

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def candidate_options(function, *, query_tile, num_warps, output_dtype=None):
    """jetspec_tree_kernel_qualification.py:47-53."""
    supported = inspect.signature(function).parameters
    options = {name: value for name, value in (("query_tile", query_tile), ("num_warps", num_warps))
               if name in supported}
    if output_dtype is not None:
        options["output_dtype"] = output_dtype
    return options


@pytest.mark.parametrize("candidate", ENTRIES)
def test_named_entry_meets_gate_in_bf16_and_fp32(candidate):
    q, k, v, meta, *_ = reference_fixture()
    function = candidate_entry(candidate)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    out16 = function(q, k, v, meta, SCALE, 4, **candidate_options(function, query_tile=1, num_warps=4))
    out32 = function(q, k, v, meta, SCALE, 4, **candidate_options(function, query_tile=4, num_warps=4,
                                                                   output_dtype=torch.float32))
    torch.cuda.synchronize()
    assert out16.dtype == torch.bfloat16 and out32.dtype == torch.float32
    assert torch.isfinite(out32).all().item(), f"{candidate}: NaN padding was read"
    assert_within_gate(out16, expect, f"{candidate} bf16")
    assert_within_gate(out32, expect, f"{candidate} fp32")
    assert torch.equal(out32.to(torch.bfloat16).view(torch.int16), out16.view(torch.int16))
    assert read_and_clear_status(q.device) == 0


@pytest.mark.parametrize("backend", ["auto", "reference", "prefix", "gqa"])
def test_dispatcher_backends(backend):
    q, k, v, meta, *_ = reference_fixture(seed=88)
    out = packed_tree_attention(q, k, v, meta, SCALE, 4, backend=backend)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    assert_within_gate(out, expect, f"backend {backend}")
    assert read_and_clear_status(q.device) == 0
