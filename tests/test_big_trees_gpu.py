"""Trees of 1025 to 2048 nodes on the MFMA kernel (GPU).

A work item caches its tree's scratch slots in LDS; beside a page-table prefix that cache
holds 2048 of them (csrc/tv_attention.h), so chunked-prefill rows of up to 2048 tokens
(chain trees, prefill.py:14-26) and large draft trees stay on the MFMA kernel instead of
the FP32 one.  Checked against the fp64 oracle on sampled rows and against the float32
torch restatement of paged_backend.py:116-213 on every row, for head sizes 64, 128 and
256; the plan built on the device equals the host plan item for item; the serving
constructor (which builds such trees' visibility on the host) equals the validating one.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import assert_within_gate, assert_within_gate_dense, oracle_rows, torch_fp32_rows
from jetspec_amd import PackedTreeMetadata, packed_tree_attention, read_and_clear_status, workloads
from jetspec_amd.paged_backend import _mfma_geometry, make_plan

pytestmark = pytest.mark.gpu
DEV = "cuda"


def big_batch(seed, prefixes, parent_lists, kv_heads=8, groups=4, head_dim=128, block=256):
    """Shuffled pages and scratch slots, N(0, 1) bf16 operands."""
    rng = np.random.default_rng(seed)
    counts = [len(p) for p in parent_lists]
    need = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    order = rng.permutation(sum(need) + scratch_pages + 5)
    tables, cursor = [], 0
    for n in need:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    pool_slots = (scratch[:, None] * block + np.arange(block)).reshape(-1)[rng.permutation(scratch_pages * block)]
    slots, off = [], 0
    for n in counts:
        slots.append(torch.as_tensor(pool_slots[off:off + n].astype(np.int64), device=DEV))
        off += n
    masks = [torch.as_tensor(workloads.ancestor_mask(p), device=DEV) for p in parent_lists]
    meta = PackedTreeMetadata.build(list(prefixes), tables, slots, masks, block)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    pages = int(order.size)
    k = torch.randn((pages, block, kv_heads, head_dim), generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn((pages, block, kv_heads, head_dim), generator=gen, device=DEV).to(torch.bfloat16)
    q = torch.randn((meta.total_queries, kv_heads * groups, head_dim), generator=gen, device=DEV).to(torch.bfloat16)
    return q, k, v, meta


def trees(seed):
    rng = np.random.default_rng(seed)
    return [workloads.chain_parents(2048), workloads.random_parents(1500, 8, rng), workloads.chain_parents(1025),
            workloads.random_parents(24, 5, rng)]


@pytest.mark.parametrize("head_dim,groups,kv_heads", [(128, 4, 8), (64, 4, 2), (256, 4, 2), (128, 8, 2)])
def test_trees_up_to_2048_nodes_match_the_references(head_dim, groups, kv_heads):
    prefixes = [3000, 0, 700, 5000]
    q, k, v, meta = big_batch(11, prefixes, trees(11), kv_heads=kv_heads, groups=groups, head_dim=head_dim)
    assert _mfma_geometry(q, k, v, meta)
    scale = head_dim ** -0.5
    out = packed_tree_attention(q, k, v, meta, scale, groups)
    reference = torch_fp32_rows(q, k, v, meta, scale)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 0
    label = f"D={head_dim} G={groups} Hkv={kv_heads} trees {list(meta.node_counts_host)}"
    pins = oracle_rows(q, k, v, meta, scale, [0, 1, 2, 3], rows_per_request=4)
    assert_within_gate(reference, pins, f"{label}: torch fp32 vs fp64 oracle", max_abs=1e-4, mean_abs=1e-5)
    assert_within_gate(out, pins, f"{label}: kernel vs fp64 oracle")
    assert_within_gate_dense(out, reference, f"{label}: kernel vs torch fp32")
    # The exact-probability entry (the reference's FP32 entries) on the same batch, f32 output.
    exact = packed_tree_attention(q, k, v, meta, scale, groups, backend="reference", output_dtype=torch.float32)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 0
    assert_within_gate_dense(exact, reference, f"{label}: exact entry vs torch fp32", max_abs=1e-4, mean_abs=1e-5)


def test_big_tree_plans_cover_every_block():
    """Every node block of a 2048-node tree has an item over the tree's slots up to its end."""
    counts = [2048, 1500, 1025, 24]
    plan = make_plan([3000, 0, 700, 5000], counts, 8, 256, 256, 0, queries_per_kv=4)
    blocks = {(r, h0, n0) for r, h0, n0, *_ in plan["items"].tolist()}
    for r, t in enumerate(counts):
        hpw = 2 if t <= 32 else 1
        npw = (8 // hpw) * 8
        assert {(r, h, n) for h in range(0, 8, hpw) for n in range(0, t, npw)} <= blocks, r


def test_serving_constructor_takes_big_trees():
    """from_host_trees builds visibility on the device up to 1024 nodes and, like the
    reference (packed_metadata.py:185-195), from the host masks above that; either way the
    metadata and the attention equal the validating constructor's."""
    from test_metadata_gpu import host_trees

    parent_lists = [workloads.chain_parents(2048), workloads.random_parents(40, 6, np.random.default_rng(2))]
    counts = [len(p) for p in parent_lists]
    prefixes, tables, arena = [300, 0], [[1, 2], []], [10, 11, 12, 13, 14, 15, 16, 17, 18, 19]
    fast = PackedTreeMetadata.from_host_trees(prefixes, tables, host_trees(parent_lists), arena, 256, device=DEV,
                                              request_ids=[0, 1])
    slots, offset = [], 0
    for n in counts:
        slots.append(torch.tensor([arena[(offset + j) // 256] * 256 + (offset + j) % 256 for j in range(n)],
                                  device=DEV))
        offset += n
    masks = [torch.as_tensor(workloads.ancestor_mask(p), device=DEV) for p in parent_lists]
    full = PackedTreeMetadata.build(prefixes, tables, slots, masks, 256, request_ids=[0, 1])
    assert torch.equal(fast.qq_bias.cpu().view(torch.int32), full.qq_bias.cpu().view(torch.int32))
    g = torch.Generator(device=DEV).manual_seed(9)
    pool = torch.randn(2, 24, 256, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(sum(counts), 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    a = packed_tree_attention(q, pool[0], pool[1], fast, 128 ** -0.5, 4)
    b = packed_tree_attention(q, pool[0], pool[1], full, 128 ** -0.5, 4)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert read_and_clear_status(DEV) == 0
