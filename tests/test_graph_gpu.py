"""Graph-capturable verify: the device planner and HIP-graph replay (GPU).

* tv_tree_attention_plan_device writes the host planner's items and merge groups,
  item for item, for the benchmark batches, ragged batches (trees of up to 2048 nodes
  among them; 100, 128, 140 and 160 requests for each form of the device planner) and
  forced chunk lengths.
* GraphedTreeAttention (device plan, capacity grids, no allocation) equals
  packed_tree_attention bit for bit.
* PackedVerifyGraph: one capture, then replays with new prefix lengths, page tables,
  scratch slots, positions and inputs of the same execution geometry; every replay is
  compared with the eager path (rotated Q, attention output and the K/V rows written),
  with eager work and synchronisations between replays.
"""
from __future__ import annotations

import ctypes
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from gpu_helpers import assert_within_gate, oracle_rows
from jetspec_amd import (PackedTreeMetadata, _device, _lib, packed_tree_attention, read_and_clear_status,
                         rope_scatter_prevalidated, workloads)
from jetspec_amd.paged_backend import make_plan
from jetspec_amd.target_graph import GraphedTreeAttention, PackedVerifyGraph

pytestmark = pytest.mark.gpu
DEV = "cuda"


def device_plan(meta, kv_heads=8, chunk_keys=0, max_prefix=None, queries_per_kv=4):
    lib = _lib.library()
    count = meta.num_requests
    nodes = (ctypes.c_int32 * count)(*meta.node_counts_host)
    info = _lib.PlanInfo()
    bound = max(meta.prefix_lengths) if max_prefix is None else max_prefix
    cus = _device.compute_units(torch.cuda.current_device())
    _lib.check(lib.tv_tree_attention_plan_capacity(nodes, count, kv_heads, queries_per_kv, meta.block_size, cus,
                                                   chunk_keys, bound, ctypes.byref(info)), "capacity")
    items = torch.full((info.num_items, 8), -7, dtype=torch.int32, device=DEV)
    groups = torch.full((max(info.num_groups, 1), 8), -7, dtype=torch.int32, device=DEV)
    counts = torch.full((4,), -7, dtype=torch.int32, device=DEV)
    _lib.check(lib.tv_tree_attention_plan_device(meta.prefix_lens.data_ptr(), meta.node_counts.data_ptr(), count,
                                                 kv_heads, queries_per_kv, meta.block_size, cus, chunk_keys,
                                                 info.num_items, info.num_groups, info.num_partial_slots, items.data_ptr(),
                                                 groups.data_ptr(), counts.data_ptr(),
                                                 _device.stream_handle(items.device)), "plan_device")
    counts = counts.tolist()
    return items.cpu().numpy(), groups.cpu().numpy(), counts, cus


def ragged_metadata(seed, prefixes, counts, pool_pages=4096):
    rng = np.random.default_rng(seed)
    pages = rng.permutation(pool_pages)
    cursor = 0
    tables, slots, masks = [], [], []
    for p, n in zip(prefixes, counts):
        need = (p + 255) // 256
        tables.append([int(x) for x in pages[cursor:cursor + need]])
        cursor += need
    scratch = [int(x) for x in pages[cursor:cursor + (sum(counts) + 255) // 256 + 1]]
    offset = 0
    for n in counts:
        slots.append(torch.tensor([scratch[(offset + j) // 256] * 256 + (offset + j) % 256 for j in range(n)],
                                  device=DEV))
        offset += n
        parents = workloads.random_parents(n, 8, rng)
        masks.append(torch.from_numpy(workloads.ancestor_mask(parents)).to(DEV))
    return PackedTreeMetadata.build(list(prefixes), tables, slots, masks, 256)


def batches():
    yield "cfg1", workloads.config1(DEV).metadata
    yield "cfg2", workloads.config2(DEV).metadata
    yield "cfg5", workloads.config5(DEV).metadata
    yield "ragged", ragged_metadata(1, [0, 1, 63, 64, 65, 255, 256, 257, 9000], [1, 2, 16, 17, 32, 33, 64, 65, 512])
    yield "long", ragged_metadata(2, [150000, 3], [64, 16])
    yield "big", ragged_metadata(4, [3000, 0, 700], [2048, 1500, 16])
    # Above 128 requests the device planner sorts item keys instead of ranking cost classes.
    rng = np.random.default_rng(6)
    yield "wide", ragged_metadata(5, [int(x) for x in rng.integers(0, 3000, size=160)],
                                  [int(x) for x in rng.choice([1, 16, 32, 64], size=160)])


def plan_inputs(seed, requests, choices, max_prefix):
    """Just what the planners read (prefix lengths and node counts, host and device)."""
    rng = np.random.default_rng(seed)
    prefixes = [int(x) for x in rng.integers(0, max_prefix, size=requests)]
    counts = [int(x) for x in rng.choice(choices, size=requests)]
    return SimpleNamespace(prefix_lengths=prefixes, node_counts_host=counts, num_requests=requests, block_size=256,
                           prefix_lens=torch.tensor(prefixes, dtype=torch.int32, device=DEV),
                           node_counts=torch.tensor(counts, dtype=torch.int32, device=DEV))


def shard_batches():
    """(name, metadata, KV heads): one- and two-head shards, where the planner refits its
    chunk target to fill whole rounds of work items, and batches for each of the device
    planner's forms: above 64 requests the per-request steps use the whole block (and the
    refit its 5-way search), 128 requests fill the cost-class ranking, and above it the
    items' keys are sorted, with unaligned (65-node) and aligned (512-node) multi-block
    trees."""
    yield "cfg4/kv1", workloads.config4(DEV, kv_heads=1, requests=64).metadata, 1
    yield "cfg5/kv2", workloads.config5(DEV, kv_heads=2).metadata, 2
    rng = np.random.default_rng(8)
    prefixes = [int(x) for x in rng.integers(0, 30000, size=34)]
    counts = [int(x) for x in rng.choice([16, 32, 64], size=34)]
    yield "ragged34", ragged_metadata(3, prefixes, counts, pool_pages=8192), 8
    yield "r100", plan_inputs(7, 100, [1, 16, 32, 64], 30000), 8
    yield "r100/kv1", plan_inputs(11, 100, [16, 32, 64], 20000), 1
    yield "r128", plan_inputs(12, 128, [16, 32], 30000), 8
    yield "r140/unaligned", plan_inputs(9, 140, [1, 16, 65, 512], 2000), 8
    yield "r140/aligned", plan_inputs(10, 140, [16, 512], 2000), 4


@pytest.mark.parametrize("chunk_keys", [0, 64, 256])
def test_device_plan_equals_host_plan(chunk_keys):
    cus = _device.compute_units(torch.cuda.current_device())
    cases = [(name, meta, 8) for name, meta in batches()] + (list(shard_batches()) if chunk_keys == 0 else [])
    for name, meta, kv in cases:
        host = make_plan(meta.prefix_lengths, meta.node_counts_host, kv, meta.block_size, cus, chunk_keys,
                         queries_per_kv=4)
        print(f"[plan] {name} chunk={chunk_keys} items={host['num_items']} groups={host['num_groups']}", flush=True)
        if host["num_items"] > 8192:
            # Beyond the device planner's 8192 items (its LDS arrays): refused up front, never overrun.
            with pytest.raises(ValueError, match="exceed"):
                device_plan(meta, kv_heads=kv, chunk_keys=chunk_keys)
            continue
        try:
            items, groups, counts, _ = device_plan(meta, kv_heads=kv, chunk_keys=chunk_keys)
        except ValueError as err:
            # A forced chunk length's capacity bound (every block at the largest prefix) can pass
            # the sort's limit before the plan does; the planner's own chunking never does here.
            assert chunk_keys > 0 and "exceed" in str(err), name
            continue
        assert counts == [host["num_items"], host["num_groups"], host["num_partial_slots"], 0], name
        assert np.array_equal(items[:host["num_items"]], host["items"]), name
        assert np.array_equal(groups[:host["num_groups"]], host["groups"][:host["num_groups"]]), name


def test_device_plan_equals_host_plan_on_random_batches():
    """Seeded random batches over every form of the device planner: request counts on both
    sides of its one-wave (64), cost-class (128) and sort limits, one to eight KV heads,
    1 to 16 query heads per KV head, trees of 1 to 2048 nodes (aligned and unaligned
    multi-block ones), prefixes from empty to 200k keys, pages of 32 and 256 and forced
    chunk lengths.  Batches whose plan either planner refuses (capacity) are counted, not
    compared; most are compared."""
    rng = np.random.default_rng(2024)
    cus = _device.compute_units(torch.cuda.current_device())
    compared = refused = 0
    for trial in range(240):
        requests = int(rng.choice([1, 2, 3, 7, 8, 16, 33, 63, 64, 65, 100, 127, 128, 129, 200, 300]))
        kv = int(rng.choice([1, 2, 4, 8]))
        qpk = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
        kind = trial % 4
        if kind == 0:
            counts = rng.integers(1, 65, size=requests)
        elif kind == 1:
            counts = rng.choice([1, 16, 32, 64, 65, 100, 512, 1024], size=requests)
        elif kind == 2:
            counts = rng.choice([8, 512], size=requests)
        else:
            counts = rng.integers(1, 2049, size=requests)
        prefixes = rng.integers(0, int(rng.choice([1, 100, 3000, 30000, 200000])), size=requests)
        chunk = int(rng.choice([0, 0, 0, 64, 256]))
        block = int(rng.choice([32, 256]))
        meta = SimpleNamespace(prefix_lengths=[int(x) for x in prefixes], node_counts_host=[int(x) for x in counts],
                               num_requests=requests, block_size=block,
                               prefix_lens=torch.tensor(prefixes, dtype=torch.int32, device=DEV),
                               node_counts=torch.tensor(counts, dtype=torch.int32, device=DEV))
        case = f"trial {trial}: R={requests} kv={kv} G={qpk} kind={kind} chunk={chunk} page={block}"
        try:
            host = make_plan(meta.prefix_lengths, meta.node_counts_host, kv, block, cus, chunk, queries_per_kv=qpk)
            items, groups, got, _ = device_plan(meta, kv_heads=kv, chunk_keys=chunk, queries_per_kv=qpk)
        except ValueError:
            refused += 1
            continue
        compared += 1
        assert got == [host["num_items"], host["num_groups"], host["num_partial_slots"], 0], case
        assert np.array_equal(items[:host["num_items"]], host["items"]), case
        assert np.array_equal(groups[:host["num_groups"]], host["groups"][:host["num_groups"]]), case
    print(f"[plan fuzz] compared {compared}, refused {refused}", flush=True)
    assert compared >= 150


def test_capacity_overflow_writes_zero_counts():
    meta = ragged_metadata(3, [100000], [64])
    lib = _lib.library()
    items = torch.zeros((2, 8), dtype=torch.int32, device=DEV)
    counts = torch.full((4,), -7, dtype=torch.int32, device=DEV)
    _lib.check(lib.tv_tree_attention_plan_device(meta.prefix_lens.data_ptr(), meta.node_counts.data_ptr(), 1, 8, 4,
                                                 256, 256, 64, 2, 0, 0, items.data_ptr(), None, counts.data_ptr(),
                                                 None), "plan_device")
    assert counts.tolist() == [0, 0, 0, 1]


@pytest.mark.parametrize("name", ["cfg1", "cfg2", "cfg5", "ragged", "big"])
def test_graphed_attention_equals_eager(name):
    meta = dict(batches())[name]
    g = torch.Generator(device=DEV).manual_seed(4)
    pages = int(max(max((max(t) for t in meta.block_tables_host if t), default=0),
                    max(meta.tree_slot_ids) // 256)) + 1
    pool = torch.randn(2, pages, 256, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(meta.total_queries, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    eager = packed_tree_attention(q, pool[0], pool[1], meta, 128 ** -0.5, 4)
    attn = GraphedTreeAttention(meta.node_counts_host, 8, 256, max_prefix=max(meta.prefix_lengths), device=DEV)
    out = torch.empty_like(q)
    attn(q, pool[0], pool[1], meta, 128 ** -0.5, out)
    assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
    assert read_and_clear_status(DEV) == 0
    reference = oracle_rows(q, pool[0], pool[1], meta, 128 ** -0.5, list(range(meta.num_requests)),
                            rows_per_request=8)
    assert_within_gate(out, reference, f"graphed {name}")


def verify_round(seed, counts, pages, max_prefix):
    """One round's metadata and per-layer inputs over a shared pool of `pages` pages."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(pages)
    prefixes = [int(x) for x in rng.integers(1, max_prefix, size=len(counts))]
    cursor, tables, slots, masks, depth_lists = 0, [], [], [], []
    for p in prefixes:
        need = (p + 255) // 256
        tables.append([int(x) for x in perm[cursor:cursor + need]])
        cursor += need
    scratch = [int(x) for x in perm[cursor:cursor + (sum(counts) + 255) // 256 + 1]]
    offset = 0
    for n in counts:
        slots.append(torch.tensor([scratch[(offset + j) // 256] * 256 + (offset + j) % 256 for j in range(n)],
                                  device=DEV))
        offset += n
        parents = workloads.random_parents(n, 8, rng)
        masks.append(torch.from_numpy(workloads.ancestor_mask(parents)).to(DEV))
        depth_lists.append(workloads.depths_of(parents))
    meta = PackedTreeMetadata.build(prefixes, tables, slots, masks, 256)
    positions = torch.tensor([prefixes[r] + d for r, depths in enumerate(depth_lists) for d in depths], device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed)
    rows = sum(counts)
    q = torch.randn(2, rows, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(2, rows, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(2, rows, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    return meta, positions, q, k, v


def eager_round(kv_pool, cache, meta, positions, q, k, v):
    outs, rotations = [], []
    for layer in range(q.shape[0]):
        rotated = torch.empty_like(q[layer])
        rope_scatter_prevalidated(q[layer], k[layer], v[layer], positions, cache, kv_pool[0, layer],
                                  kv_pool[1, layer], meta.tree_slots, rotated)
        rotations.append(rotated)
        outs.append(packed_tree_attention(rotated, kv_pool[0, layer], kv_pool[1, layer], meta, 128 ** -0.5, 4))
    return torch.stack(outs), torch.stack(rotations)


def test_verify_graph_replays_match_eager():
    counts = [64, 32, 16, 64]
    pages, max_prefix = 96, 4000
    g = torch.Generator(device=DEV).manual_seed(9)
    pool = torch.randn(2, 2, pages, 256, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    angles = torch.arange(8192, device=DEV, dtype=torch.float32)[:, None] * (
        torch.arange(64, device=DEV, dtype=torch.float32)[None, :] + 1) * 1e-3
    cache = torch.cat((angles.cos(), angles.sin()), -1).unsqueeze(1)
    graph = PackedVerifyGraph(pool, cache, 128 ** -0.5, max_model_len=4096)
    for round_index in range(4):
        meta, positions, q, k, v = verify_round(100 + round_index, counts, pages, max_prefix)
        reference_pool = pool.clone()
        expected, rotated = eager_round(reference_pool, cache, meta, positions, q, k, v)
        torch.cuda.synchronize()
        got = graph.verify(q, k, v, positions, meta).clone()
        torch.cuda.synchronize()
        print(f"[graph] round {round_index}: prefixes {meta.prefix_lengths} {graph.snapshot()}", flush=True)
        assert torch.equal(got.view(torch.int16), expected.view(torch.int16)), f"round {round_index} output"
        assert torch.equal(pool.view(torch.int16), reference_pool.view(torch.int16)), f"round {round_index} pool"
        # The replay against the fp64 oracle on the same rotated queries and pool rows.
        for layer in range(q.shape[0]):
            reference = oracle_rows(rotated[layer], pool[0, layer], pool[1, layer], meta, 128 ** -0.5,
                                    list(range(meta.num_requests)))
            assert_within_gate(got[layer], reference, f"graph replay round {round_index} layer {layer}")
        # Eager work between replays (a different stream state and allocator traffic).
        torch.randn(1 << 20, device=DEV).sum().item()
    assert graph.captures == 1 and graph.replays == 4
    assert read_and_clear_status(DEV) == 0
    graph.close()
