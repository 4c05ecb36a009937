"""Legacy single-request slot-addressed attention and the exact-probability mode (GPU).

* paged_tree_attention (paged_backend.py:309-415) as the legacy c1 path calls it
  (models/qwen3.py:270-302): the pool viewed as 16-token sub-pages, a logical slot per key
  (prefix through the page table, then the tree's scratch slots) and a 0 / -inf bias.  Where
  its plan splits the prefix as the page plan does, it must equal the packed exact entry on
  the same request byte for byte (the reference's "packed == per-request legacy" test,
  tests/test_jetspec_packed_attention.py:156-188); it must always meet the gate against the
  fp64 oracle.
* The FP32 entries keep probabilities exact: their FP32 output meets the reference's FP32
  qualification bound (FP32_ATTENTION_BOUND = 1e-4 on max-abs and relative RMS,
  benchmarks/jetspec_numeric_oracles.py:21,108-168) against the fp64 oracle, which the
  bf16-probability mode does not.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import assert_within_gate, metrics, oracle_rows
from jetspec_amd import (PackedTreeMetadata, packed_tree_attention, packed_tree_attention_reference,
                         paged_tree_attention, read_and_clear_status, workloads)
from test_attention_gpu import reference_fixture

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5


def legacy_call(q, k, v, prefix, table, slots, mask):
    """models/qwen3.py:270-302's call for one request."""
    positions = torch.arange(prefix, device=DEV, dtype=torch.int64)
    pages = torch.tensor(table, device=DEV, dtype=torch.int64)
    prefix_slots = pages[positions // 256] * 256 + positions % 256 if prefix else positions
    logical = torch.cat((prefix_slots, slots.to(torch.int64)))
    total = prefix + q.shape[0]
    bias = torch.where(mask, 0.0, float("-inf")).float()
    return paged_tree_attention(
        q, k.view(-1, 16, k.shape[2], k.shape[3]), v.view(-1, 16, v.shape[2], v.shape[3]),
        torch.zeros((1, (total + 15) // 16), device=DEV, dtype=torch.int32),
        torch.tensor([0, q.shape[0]], device=DEV, dtype=torch.int32),
        torch.tensor([total], device=DEV, dtype=torch.int32), bias, SCALE, q.shape[1] // k.shape[2], 16,
        logical.reshape(1, -1), torch.tensor([0], device=DEV, dtype=torch.int32),
        torch.tensor([total], device=DEV, dtype=torch.int32))


@pytest.mark.parametrize("prefixes,counts", [((65, 0, 257), (63, 31, 47)), ((5000, 1, 2049), (16, 7, 64))])
def test_legacy_c1_equals_packed_fp32_entry_bytewise(prefixes, counts):
    q, k, v, meta, slots, masks, _ = reference_fixture(prefixes=prefixes, counts=counts)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    for r in range(meta.num_requests):
        rows = meta.request_slice(r)
        local_q = q[rows].contiguous()
        legacy = legacy_call(local_q, k, v, meta.prefix_lengths[r], meta.block_tables_host[r], slots[r], masks[r])
        solo = PackedTreeMetadata.build([meta.prefix_lengths[r]], [meta.block_tables_host[r]], [slots[r]],
                                        [masks[r]], 256)
        packed = packed_tree_attention_reference(local_q, k, v, solo, SCALE, 4)
        torch.cuda.synchronize()
        assert torch.isfinite(legacy.float()).all().item(), f"request {r}: NaN padding was read"
        assert torch.equal(legacy.view(torch.int16), packed.view(torch.int16)), f"request {r}"
        full = torch.zeros_like(q)
        full[rows] = legacy
        assert_within_gate(full, {r: expect[r]}, f"legacy c1 request {r} (P={meta.prefix_lengths[r]})")
    assert read_and_clear_status(DEV) == 0


def test_legacy_long_prefix_with_differently_split_plans_meets_the_gate():
    """One request with a long prefix, 8 KV heads x 16 query heads and 200 nodes: the page plan
    splits the prefix into chunks above the 2048 slots a slot-addressed item caches, so the
    legacy entry's plan splits it finer and its split-K merges round differently.  The result
    then stays within the gate of the fp64 oracle and within bf16 rounding of the packed entry."""
    q, k, v, meta, slots, masks, _ = reference_fixture(prefixes=(9000,), counts=(200,), kv_heads=8, groups=16)
    legacy = legacy_call(q, k, v, 9000, meta.block_tables_host[0], slots[0], masks[0])
    packed = packed_tree_attention_reference(q, k, v, meta, SCALE, 16)
    torch.cuda.synchronize()
    assert torch.isfinite(legacy.float()).all().item(), "NaN padding was read"
    assert (legacy.float() - packed.float()).abs().max().item() < 2e-3
    assert_within_gate(legacy, oracle_rows(q, k, v, meta, SCALE, [0], rows_per_request=16),
                       "legacy c1 P=9000 T=200 kv=8 G=16")
    assert read_and_clear_status(DEV) == 0


def test_legacy_rejections():
    q, k, v, meta, slots, masks, _ = reference_fixture()
    rows = meta.request_slice(0)
    local_q = q[rows].contiguous()
    with pytest.raises(ValueError, match="multi-request"):
        paged_tree_attention(local_q, k, v, None, None, torch.tensor([3, 4], device=DEV), None, SCALE, 4, 256)
    with pytest.raises(ValueError, match="external jetspec kernel"):
        paged_tree_attention(local_q, k, v, None, None, torch.tensor([3], device=DEV), None, SCALE, 4, 256)
    # A finite bias is added to the score (paged_backend.py:82-91): it runs on the FP32
    # kernel and moves only its own row (tests/test_fp32_kernel_gpu.py checks the values).
    bias = torch.where(masks[0], 0.0, float("-inf")).float()
    bias[5, 0] = 0.5
    logical = torch.cat((torch.arange(65, device=DEV) + 256 * meta.block_tables_host[0][0], slots[0]))
    biased = paged_tree_attention(local_q, k.view(-1, 16, 2, 128), v.view(-1, 16, 2, 128), None, None,
                                  torch.tensor([65 + local_q.shape[0]], device=DEV), bias, SCALE, 4, 16,
                                  logical.view(1, -1))
    plain = legacy_call(local_q, k, v, 65, meta.block_tables_host[0], slots[0], masks[0])
    diff = (biased.float() - plain.float()).abs().amax(dim=(1, 2))
    assert diff[5].item() > 1e-3
    assert torch.cat((diff[:5], diff[6:])).max().item() < 2e-2
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("case", ["fixture", "config2", "forced_split", "config5_sampled"])
def test_exact_probabilities_meet_the_fp32_bound(case):
    if case == "fixture":
        q, k, v, meta, *_ = reference_fixture()
        requests, rows_per, kwargs = list(range(meta.num_requests)), None, {}
    elif case == "forced_split":
        q, k, v, meta, *_ = reference_fixture(prefixes=(1500, 0, 700))
        requests, rows_per, kwargs = list(range(meta.num_requests)), None, {"chunk_keys": 64}
    else:
        batch = workloads.config2(DEV) if case == "config2" else workloads.config5(DEV)
        q, k, v, meta = batch.q, batch.k_pool, batch.v_pool, batch.metadata
        requests = list(range(meta.num_requests)) if case == "config2" else [0, 5, 16, 40]
        rows_per, kwargs = (None if case == "config2" else 6), {}
    expect = oracle_rows(q, k, v, meta, SCALE, requests, rows_per_request=rows_per)
    if kwargs:
        exact = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        from jetspec_amd.paged_backend import _launch
        _launch(q, k, v, meta, SCALE, exact, exact=True, **kwargs)
    else:
        exact = packed_tree_attention_reference(q, k, v, meta, SCALE, 4, output_dtype=torch.float32)
    fast = packed_tree_attention(q, k, v, meta, SCALE, 4, output_dtype=torch.float32, **kwargs)
    torch.cuda.synchronize()
    m_exact, m_fast = metrics(exact, expect), metrics(fast, expect)
    print(f"[exact {case}] max-abs {m_exact['max_abs_error']:.3e} rel-RMS {m_exact['relative_rms_error']:.3e} "
          f"(bound {m_exact['max_abs_bound']:.1e}); bf16-P: max-abs {m_fast['max_abs_error']:.3e} "
          f"rel-RMS {m_fast['relative_rms_error']:.3e}", flush=True)
    assert m_exact["within_fixed_bound"], m_exact
    assert not m_fast["within_fixed_bound"]
    assert read_and_clear_status(DEV) == 0
