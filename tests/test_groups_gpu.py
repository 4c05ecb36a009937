"""Every query-group size the MFMA kernel is built for, G in 1..8 and 16 (GPU).

The reference's grouped kernel takes any power of two up to 16 query heads per KV head
(tree_gqa.py:124-126) and its FP32 kernel any divisor; this build instantiates the MFMA
kernel for G = 1..8 and 16 (the powers of two and the GQA ratios of other Qwen-family
checkpoints) and runs other ratios on the FP32 kernel.  A work item is 8 waves x 32 score
rows, so it holds (8 / HPW) * floor(32 / G) tree nodes of each of its HPW KV heads: 256
nodes at G = 1 down to 16 at G = 16, with two KV heads per item for trees of at most
half that; when G does not divide 32, each wave's last 32 - floor(32 / G) * G rows are
padding.  The node counts below sit on both sides of those limits for every G.

Per G:
  * bf16 output within the north-star gate of the fp64 oracle on every row (auto
    backend), with NaN in every unused pool row;
  * the exact-probability mode (the reference's FP32 entries) within the FP32 bound;
  * a forced split of the prefix (partials + merge) within the gate and equal to the
    unsplit launch up to the merge's rounding;
  * the device planner writes the host planner's items;
  * the graphed launch equals the eager one bit for bit;
  * the legacy slot-addressed entry equals the packed FP32 entry byte for byte.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import assert_within_gate, metrics, oracle_rows
from jetspec_amd import (PackedTreeMetadata, packed_tree_attention, packed_tree_attention_reference,
                         read_and_clear_status)
from jetspec_amd import _device
from jetspec_amd.paged_backend import _launch, _mfma_geometry, make_plan
from jetspec_amd.target_graph import GraphedTreeAttention
from test_attention_gpu import reference_fixture
from test_graph_gpu import device_plan
from test_legacy_exact_gpu import legacy_call

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5
GROUPS = (1, 2, 3, 5, 6, 7, 8, 16)   # G = 4 is covered by every other GPU test


def nodes_per_item(hpw, groups):
    return (8 // hpw) * (32 // groups)


def threshold_counts(groups):
    """Node counts on both sides of the two-head and one-head item sizes for this G."""
    two, one = nodes_per_item(2, groups), nodes_per_item(1, groups)
    return tuple(min(n, 1024) for n in (1, two, two + 1, one, one + 1, 2 * one + 3))


def fixture(groups, prefixes=None, kv_heads=2, seed=900):
    counts = threshold_counts(groups)
    if prefixes is None:
        prefixes = (0, 65, 257, 1500, 31, 4097)[:len(counts)]
    return reference_fixture(prefixes=prefixes, counts=counts, kv_heads=kv_heads, seed=seed + groups,
                             groups=groups)


@pytest.mark.parametrize("groups", GROUPS)
@pytest.mark.parametrize("kv_heads", [1, 2])
def test_every_row_meets_the_gate(groups, kv_heads):
    q, k, v, meta, *_ = fixture(groups, kv_heads=kv_heads)
    print(f"[G{groups} kv{kv_heads}] nodes {meta.node_counts_host} prefixes {meta.prefix_lengths}", flush=True)
    out = packed_tree_attention(q, k, v, meta, SCALE, groups)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all().item(), "NaN padding was read"
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    assert_within_gate(out, expect, f"G{groups} kv{kv_heads}")
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
def test_exact_mode_meets_the_fp32_bound(groups):
    q, k, v, meta, *_ = fixture(groups)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    exact = packed_tree_attention_reference(q, k, v, meta, SCALE, groups, output_dtype=torch.float32)
    torch.cuda.synchronize()
    m = metrics(exact, expect)
    print(f"[exact G{groups}] max-abs {m['max_abs_error']:.3e} rel-RMS {m['relative_rms_error']:.3e}", flush=True)
    assert m["within_fixed_bound"], m
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
def test_forced_prefix_split_meets_the_gate(groups):
    q, k, v, meta, *_ = fixture(groups, prefixes=(3000, 700, 2049, 1500, 64, 4097))
    plan = make_plan(meta.prefix_lengths, meta.node_counts_host, 2, meta.block_size,
                     _device.compute_units(torch.cuda.current_device()), 64, queries_per_kv=groups)
    assert plan["num_partial_slots"] > 0 and plan["num_groups"] > 0
    split = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    _launch(q, k, v, meta, SCALE, split, chunk_keys=64, exact=True)
    whole = packed_tree_attention_reference(q, k, v, meta, SCALE, groups, output_dtype=torch.float32)
    torch.cuda.synchronize()
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)), rows_per_request=8)
    m = metrics(split, expect)
    print(f"[split G{groups}] items {plan['num_items']} merges {plan['num_groups']} "
          f"max-abs {m['max_abs_error']:.3e} rel-RMS {m['relative_rms_error']:.3e}", flush=True)
    assert m["within_fixed_bound"], m
    assert (split - whole).abs().max().item() < 1e-5
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
@pytest.mark.parametrize("chunk_keys", [0, 64])
def test_device_plan_equals_host_plan(groups, chunk_keys):
    _, _, _, meta, *_ = fixture(groups, prefixes=(3000, 700, 2049, 1500, 64, 4097))
    cus = _device.compute_units(torch.cuda.current_device())
    for kv in (1, 2, 8):
        host = make_plan(meta.prefix_lengths, meta.node_counts_host, kv, meta.block_size, cus, chunk_keys,
                         queries_per_kv=groups)
        print(f"[plan G{groups} kv{kv} chunk {chunk_keys}] items {host['num_items']}", flush=True)
        items, merges, counts, _ = device_plan(meta, kv_heads=kv, chunk_keys=chunk_keys, queries_per_kv=groups)
        assert counts == [host["num_items"], host["num_groups"], host["num_partial_slots"], 0]
        assert np.array_equal(items[:host["num_items"]], host["items"])
        assert np.array_equal(merges[:host["num_groups"]], host["groups"][:host["num_groups"]])


@pytest.mark.parametrize("groups", GROUPS)
def test_graphed_attention_equals_eager(groups):
    q, k, v, meta, *_ = fixture(groups)
    eager = packed_tree_attention(q, k, v, meta, SCALE, groups)
    attn = GraphedTreeAttention(meta.node_counts_host, 2, 256, max_prefix=max(meta.prefix_lengths), device=DEV,
                                queries_per_kv=groups)
    out = torch.empty_like(q)
    attn(q, k, v, meta, SCALE, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
    with pytest.raises(ValueError, match="query head count"):
        attn(q[:, :groups], k, v, meta, SCALE, out[:, :groups])
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", [1, 5, 16])
def test_legacy_entry_equals_packed_fp32_entry(groups):
    q, k, v, meta, slots, masks, _ = fixture(groups)
    for r in range(meta.num_requests):
        rows = meta.request_slice(r)
        local_q = q[rows].contiguous()
        legacy = legacy_call(local_q, k, v, meta.prefix_lengths[r], meta.block_tables_host[r], slots[r], masks[r])
        solo = PackedTreeMetadata.build([meta.prefix_lengths[r]], [meta.block_tables_host[r]], [slots[r]],
                                        [masks[r]], 256)
        packed = packed_tree_attention_reference(local_q, k, v, solo, SCALE, groups)
        torch.cuda.synchronize()
        assert torch.equal(legacy.view(torch.int16), packed.view(torch.int16)), f"G{groups} request {r}"
    assert read_and_clear_status(DEV) == 0


def test_other_group_sizes_take_the_fp32_kernel():
    """Group sizes outside 1-8 and 16 run the FP32 kernel (tests/test_fp32_kernel_gpu.py
    checks its values); the grouped entry refuses them as the reference's does."""
    q, k, v, meta, *_ = reference_fixture(kv_heads=1, groups=4)
    assert _mfma_geometry(q, k, v, meta)
    for heads in (9, 12, 32):
        other = torch.randn((q.shape[0], heads, 128), device=DEV).to(q.dtype)
        assert not _mfma_geometry(other, k, v, meta)
        out = packed_tree_attention(other, k, v, meta, SCALE, heads)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all().item()
        with pytest.raises(ValueError, match="power-of-two GQA"):
            packed_tree_attention(other, k, v, meta, SCALE, heads, backend="gqa")
    assert read_and_clear_status(DEV) == 0
