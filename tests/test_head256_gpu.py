"""The MFMA kernel at head size 256 (GPU).

The reference's grouped kernel takes any head size, padded to a power of two
(tree_gqa.py:132-135), for power-of-two query groups up to 16 (:124-126).  This build
instantiates the MFMA kernel at head size 256 for G = 1, 2, 4, 8 and 16.  A wave's Q operands
and O accumulators double there, so a work item's 256 score rows run as two 4-wave workgroups
(one wave per SIMD): a one-head item's halves split its nodes and share its K/V stream, a
two-head item's halves are its two heads.  A tile is staged as four 64-dim parts, one DMA per
part and lane.  Per G, on the reference fixture's layout (shuffled pages, scattered scratch
slots, NaN in every unused pool row) with node counts on both sides of the half, two-head and
one-head item sizes:
  * bf16 output within the north-star gate of the fp64 oracle on every row, for 1, 2 and 3 KV
    heads (3: a two-head item whose second head does not exist leaves its second half idle);
  * the exact-probability mode within the reference's FP32 bound;
  * a forced split of the prefix (partials + merge at the 256-float partial row);
  * the graphed launch (device plan, capacity grid) bit for bit equal to the eager one;
  * the legacy slot-addressed entry byte for byte equal to the packed FP32 entry.
"""
from __future__ import annotations

import pytest
import torch

from gpu_helpers import assert_within_gate, metrics, oracle_rows
from jetspec_amd import (PackedTreeMetadata, packed_tree_attention, packed_tree_attention_reference,
                         read_and_clear_status, workloads)
from jetspec_amd import _device
from jetspec_amd.paged_backend import _launch, _mfma_geometry, make_plan
from jetspec_amd.target_graph import GraphedTreeAttention
from test_attention_gpu import reference_fixture
from test_legacy_exact_gpu import legacy_call

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 256
SCALE = D ** -0.5
GROUPS = (1, 2, 4, 8, 16)


def nodes_per_item(hpw, groups):
    return (8 // hpw) * (32 // groups)


def fixture(groups, prefixes=None, kv_heads=2, seed=2560, dtype=torch.bfloat16):
    two, one = nodes_per_item(2, groups), nodes_per_item(1, groups)
    half = one // 2
    counts = tuple(min(n, 1024) for n in (1, two, two + 1, one, one + 1, half + 1, 2 * one + 3))
    if prefixes is None:
        prefixes = (0, 65, 257, 1500, 31, 700, 4097)
    return reference_fixture(prefixes=prefixes, counts=counts, kv_heads=kv_heads, seed=seed + groups,
                             groups=groups, head_dim=D, dtype=dtype)


@pytest.mark.parametrize("groups", GROUPS)
@pytest.mark.parametrize("kv_heads", [1, 2, 3])
def test_every_row_meets_the_gate(groups, kv_heads):
    q, k, v, meta, *_ = fixture(groups, kv_heads=kv_heads)
    assert _mfma_geometry(q, k, v, meta)
    print(f"[D256 G{groups} kv{kv_heads}] nodes {meta.node_counts_host} prefixes {meta.prefix_lengths}", flush=True)
    out = packed_tree_attention(q, k, v, meta, SCALE, groups)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all().item(), "NaN padding was read"
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    assert_within_gate(out, expect, f"D256 G{groups} kv{kv_heads}")
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
def test_exact_mode_meets_the_fp32_bound(groups):
    q, k, v, meta, *_ = fixture(groups)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    exact = packed_tree_attention_reference(q, k, v, meta, SCALE, groups, output_dtype=torch.float32)
    torch.cuda.synchronize()
    m = metrics(exact, expect)
    print(f"[D256 exact G{groups}] max-abs {m['max_abs_error']:.3e} rel-RMS {m['relative_rms_error']:.3e}", flush=True)
    assert m["within_fixed_bound"], m
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
def test_forced_prefix_split_meets_the_bound(groups):
    q, k, v, meta, *_ = fixture(groups, prefixes=(3000, 700, 2049, 1500, 64, 900, 4097))
    plan = make_plan(meta.prefix_lengths, meta.node_counts_host, 2, meta.block_size,
                     _device.compute_units(torch.cuda.current_device()), 64, queries_per_kv=groups)
    assert plan["num_partial_slots"] > 0 and plan["num_groups"] > 0
    split = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    _launch(q, k, v, meta, SCALE, split, chunk_keys=64, exact=True)
    whole = packed_tree_attention_reference(q, k, v, meta, SCALE, groups, output_dtype=torch.float32)
    torch.cuda.synchronize()
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)), rows_per_request=8)
    m = metrics(split, expect)
    print(f"[D256 split G{groups}] items {plan['num_items']} merges {plan['num_groups']} "
          f"max-abs {m['max_abs_error']:.3e} rel-RMS {m['relative_rms_error']:.3e}", flush=True)
    assert m["within_fixed_bound"], m
    assert (split - whole).abs().max().item() < 1e-5
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", GROUPS)
def test_graphed_attention_equals_eager(groups):
    q, k, v, meta, *_ = fixture(groups)
    eager = packed_tree_attention(q, k, v, meta, SCALE, groups)
    attn = GraphedTreeAttention(meta.node_counts_host, 2, 256, max_prefix=max(meta.prefix_lengths), device=DEV,
                                queries_per_kv=groups, head_dim=D)
    out = torch.empty_like(q)
    attn(q, k, v, meta, SCALE, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
    assert read_and_clear_status(DEV) == 0


def test_graphed_split_equals_eager_split():
    """Split prefixes under the device plan: the workspace sized for head size 256."""
    q, k, v, meta, *_ = fixture(4, prefixes=(3000, 700, 2049, 1500, 64, 900, 4097))
    eager = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    _launch(q, k, v, meta, SCALE, eager, chunk_keys=128, exact=True)
    attn = GraphedTreeAttention(meta.node_counts_host, 2, 256, max_prefix=max(meta.prefix_lengths), device=DEV,
                                queries_per_kv=4, chunk_keys=128, head_dim=D)
    assert attn.slot_capacity > 0
    out = torch.empty_like(eager)
    attn(q, k, v, meta, SCALE, out, exact=True)
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    small = GraphedTreeAttention(meta.node_counts_host, 2, 256, max_prefix=max(meta.prefix_lengths), device=DEV,
                                 queries_per_kv=4, chunk_keys=128)
    with pytest.raises(ValueError, match="head size 256"):
        small(q, k, v, meta, SCALE, out, exact=True)
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("groups", [1, 4, 16])
def test_legacy_entry_equals_packed_fp32_entry(groups):
    q, k, v, meta, slots, masks, _ = fixture(groups)
    for r in range(meta.num_requests):
        rows = meta.request_slice(r)
        local_q = q[rows].contiguous()
        legacy = legacy_call(local_q, k, v, meta.prefix_lengths[r], meta.block_tables_host[r], slots[r], masks[r])
        solo = PackedTreeMetadata.build([meta.prefix_lengths[r]], [meta.block_tables_host[r]], [slots[r]],
                                        [masks[r]], 256)
        packed = packed_tree_attention_reference(local_q, k, v, solo, 128 ** -0.5, groups)
        torch.cuda.synchronize()
        assert torch.equal(legacy.view(torch.int16), packed.view(torch.int16)), f"G{groups} request {r}"
    assert read_and_clear_status(DEV) == 0


def test_grouped_entry_takes_head_size_256():
    """backend="gqa" (the reference's grouped kernel pads any head size, tree_gqa.py:132-135)."""
    q, k, v, meta, *_ = fixture(8)
    out = packed_tree_attention(q, k, v, meta, SCALE, 8, backend="gqa")
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    assert_within_gate(out, expect, "D256 gqa")
    assert torch.equal(out.view(torch.int16), packed_tree_attention(q, k, v, meta, SCALE, 8).view(torch.int16))
    assert read_and_clear_status(DEV) == 0


def test_fp16_operands():
    q, k, v, meta, *_ = fixture(4, dtype=torch.float16)
    out = packed_tree_attention(q, k, v, meta, SCALE, 4)
    expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
    assert_within_gate(out, expect, "D256 fp16")
    assert read_and_clear_status(DEV) == 0


def test_long_context_batch_sampled_rows():
    """16 requests of 4k-20k keys with 64-node trees in a 90 % full permuted pool, at head size 256
    (the streaming loop's page walk over many pages; each item's halves share its stream)."""
    import numpy as np

    rng = np.random.default_rng(256)
    prefixes = [int(x) for x in rng.integers(4096, 20481, size=16)]
    trees = [workloads.random_parents(64, 8, rng) for _ in range(16)]
    batch = workloads.build_verify_batch(prefixes, trees, device=DEV, seed=256, pool_fill=0.9, poison=False,
                                         head_dim=D)
    out = packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, batch.metadata, batch.scale, 4)
    expect = oracle_rows(batch.q, batch.k_pool, batch.v_pool, batch.metadata, batch.scale, [0, 5, 11, 15],
                         rows_per_request=6)
    assert_within_gate(out, expect, "D256 long context")
    assert read_and_clear_status(DEV) == 0


def test_other_groups_at_head_size_256_take_the_fp32_kernel():
    for groups in (3, 6):
        q, k, v, meta, *_ = reference_fixture(kv_heads=1, groups=groups, head_dim=D)
        assert not _mfma_geometry(q, k, v, meta)
        out = packed_tree_attention(q, k, v, meta, SCALE, groups)
        expect = oracle_rows(q, k, v, meta, SCALE, list(range(meta.num_requests)))
        assert_within_gate(out, expect, f"D256 G{groups} (FP32 kernel)")
    assert read_and_clear_status(DEV) == 0
