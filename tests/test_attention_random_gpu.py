"""Seeded random batches of the packed tree-verify attention vs the fp64 oracle (GPU).

Each case draws the request count, prefix lengths (0 to a few thousand keys), tree sizes
and depths, page size (a multiple of 32), KV heads (1, 2 or 8 with 4 query heads each),
a forced prefix chunk length (0 = the planner's own), operand dtype and output dtype.
Pages and scratch slots come from a shuffled pool whose unused rows are NaN, so a wrong
page, slot, mask bit or chunk boundary shows up either as NaN or as a gate failure
(max-abs 2e-2, mean-abs 2e-3 against the oracle).  Together the cases cross the
kernel's streaming and general loops, one- and two-head work items, page changes every
1-16 tiles and chunk starts inside a page.  A second set draws larger batches (up to 48
requests, prefixes up to 40k keys, trees up to 200 nodes) whose plans split prefixes and
run several rounds of work items; there the oracle checks sampled rows of three requests
per case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import assert_within_gate, oracle_rows
from jetspec_amd import PackedTreeMetadata, packed_tree_attention, read_and_clear_status, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def random_case(seed):
    rng = np.random.default_rng(seed)
    requests = int(rng.integers(1, 7))
    block = int(rng.choice([32, 64, 96, 128, 256, 512]))
    kv_heads = int(rng.choice([1, 2, 8], p=[0.4, 0.4, 0.2]))
    chunk = int(rng.choice([0, 0, 64, 96, 320]))
    dtype = torch.float16 if rng.random() < 0.25 else torch.bfloat16
    prefixes = [int(x) for x in rng.integers(0, 3000, size=requests)]
    if rng.random() < 0.3:
        prefixes[0] = 0
    counts = [int(rng.choice([1, 5, 16, 31, 32, 33, 64, 65, 100])) for _ in range(requests)]
    parents = [workloads.random_parents(n, int(rng.integers(1, 9)), rng) if rng.random() < 0.8
               else workloads.chain_parents(n) for n in counts]
    prefix_pages = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    total = sum(prefix_pages) + scratch_pages + 2
    order = rng.permutation(total)
    tables, cursor = [], 0
    for n in prefix_pages:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    pool_slots = (scratch[:, None] * block + np.arange(block)).reshape(-1)[rng.permutation(scratch_pages * block)]
    slots, off = [], 0
    for n in counts:
        slots.append(torch.as_tensor(pool_slots[off:off + n].astype(np.int64), device=DEV))
        off += n
    masks = [torch.as_tensor(workloads.ancestor_mask(p), device=DEV) for p in parents]
    meta = PackedTreeMetadata.build(prefixes, tables, slots, masks, block)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.full((total, block, kv_heads, 128), float("nan"), device=DEV, dtype=dtype)
    v = torch.full_like(k, float("nan"))
    live = [torch.as_tensor(np.asarray(t, dtype=np.int64)[np.arange(p) // block] * block + np.arange(p) % block,
                            device=DEV) for t, p in zip(tables, prefixes)]
    live = torch.cat(live + slots)
    k.view(-1, kv_heads, 128)[live] = torch.randn((live.numel(), kv_heads, 128), generator=gen, device=DEV).to(dtype)
    v.view(-1, kv_heads, 128)[live] = torch.randn((live.numel(), kv_heads, 128), generator=gen, device=DEV).to(dtype)
    q = torch.randn((meta.total_queries, 4 * kv_heads, 128), generator=gen, device=DEV).to(dtype)
    out_dtype = torch.float32 if rng.random() < 0.25 else None
    label = (f"seed {seed}: R={requests} block={block} kv_heads={kv_heads} chunk={chunk} {dtype} "
             f"prefixes={prefixes} nodes={counts} out={out_dtype}")
    return q, k, v, meta, chunk, out_dtype, label


@pytest.mark.parametrize("seed", range(40))
def test_random_batch_matches_oracle(seed):
    q, k, v, meta, chunk, out_dtype, label = random_case(7000 + seed)
    print(f"[random] {label}", flush=True)
    kwargs = {"chunk_keys": chunk}
    if out_dtype is not None:
        kwargs["output_dtype"] = out_dtype
    out = packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4, **kwargs)
    torch.cuda.synchronize()
    assert out.dtype == (out_dtype or q.dtype)
    assert torch.isfinite(out).all().item(), f"{label}: NaN padding was read"
    expect = oracle_rows(q, k, v, meta, 128 ** -0.5, list(range(meta.num_requests)))
    assert_within_gate(out, expect, label)
    assert read_and_clear_status(q.device) == 0


def large_case(seed):
    rng = np.random.default_rng(seed)
    requests = int(rng.integers(1, 49))
    block = int(rng.choice([32, 64, 128, 256, 512]))
    kv_heads = int(rng.choice([1, 2, 8], p=[0.3, 0.3, 0.4]))
    prefixes = [int(x) for x in rng.integers(0, 40000, size=requests)]
    counts = [int(rng.choice([1, 7, 16, 32, 33, 64, 100, 200])) for _ in range(requests)]
    parents = [workloads.random_parents(n, int(rng.integers(1, 12)), rng) for n in counts]
    prefix_pages = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    total = sum(prefix_pages) + scratch_pages + 2
    order = rng.permutation(total)
    tables, cursor = [], 0
    for n in prefix_pages:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    pool_slots = (scratch[:, None] * block + np.arange(block)).reshape(-1)[rng.permutation(scratch_pages * block)]
    slots, off = [], 0
    for n in counts:
        slots.append(torch.as_tensor(pool_slots[off:off + n].astype(np.int64), device=DEV))
        off += n
    masks = [torch.as_tensor(workloads.ancestor_mask(p), device=DEV) for p in parents]
    meta = PackedTreeMetadata.build(prefixes, tables, slots, masks, block)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    q = torch.randn((meta.total_queries, 4 * kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    picks = sorted({int(x) for x in rng.choice(requests, size=min(3, requests), replace=False)})
    label = (f"seed {seed}: R={requests} block={block} kv_heads={kv_heads} max prefix={max(prefixes)} "
             f"max nodes={max(counts)} checked requests={picks}")
    return q, k, v, meta, picks, label


@pytest.mark.parametrize("seed", range(8))
def test_large_random_batch_matches_oracle_on_sampled_rows(seed):
    q, k, v, meta, picks, label = large_case(9100 + seed)
    print(f"[random-large] {label}", flush=True)
    out = packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item(), label
    assert_within_gate(out, oracle_rows(q, k, v, meta, 128 ** -0.5, picks, rows_per_request=8), label)
    assert read_and_clear_status(q.device) == 0


@pytest.mark.parametrize("requests,seed", [(600, 11), (1500, 12)])
def test_many_requests_match_oracle_on_sampled_rows(requests, seed):
    """Hundreds of small requests in one launch: thousands of work items, mostly two-head
    items of short trees, every request's rows at a different packed offset; sampled
    requests against the fp64 oracle, the whole output finite over a NaN-free pool."""
    rng = np.random.default_rng(seed)
    block, kv_heads = 256, 8
    prefixes = [int(x) for x in rng.integers(0, 2500, size=requests)]
    counts = [int(rng.choice([1, 2, 9, 16, 32, 33, 64])) for _ in range(requests)]
    parents = [workloads.random_parents(n, int(rng.integers(1, 8)), rng) for n in counts]
    prefix_pages = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    total = sum(prefix_pages) + scratch_pages + 1
    order = rng.permutation(total)
    tables, cursor = [], 0
    for n in prefix_pages:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    pool_slots = (scratch[:, None] * block + np.arange(block)).reshape(-1)[rng.permutation(scratch_pages * block)]
    slots, off = [], 0
    for n in counts:
        slots.append(torch.as_tensor(pool_slots[off:off + n].astype(np.int64), device=DEV))
        off += n
    masks = [torch.as_tensor(workloads.ancestor_mask(p), device=DEV) for p in parents]
    meta = PackedTreeMetadata.build(prefixes, tables, slots, masks, block)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    q = torch.randn((meta.total_queries, 4 * kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    picks = sorted({0, requests - 1} | {int(x) for x in rng.choice(requests, size=4, replace=False)})
    print(f"[many] R={requests} rows={meta.total_queries} pages={total} checked={picks}", flush=True)
    out = packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    assert_within_gate(out, oracle_rows(q, k, v, meta, 128 ** -0.5, picks), f"{requests} requests")
    assert read_and_clear_status(q.device) == 0
