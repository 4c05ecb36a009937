"""The MFMA kernel against the FP32 kernel on every row of large random batches (GPU).

The fp64 oracle checks sampled rows at these sizes; here the MFMA kernel's exact-
probability mode (the reference's FP32 entries) is compared on every row with the FP32
kernel, an independent implementation of the same semantics (one wave per row and KV
head, scalar fp32 arithmetic, no plan, no ancestor bits: it reads qq_bias).  Both are
pinned to the oracle elsewhere (tests/test_groups_gpu.py, tests/test_fp32_kernel_gpu.py);
agreement within 5e-5 on every row and head of batches with split prefixes, several
rounds of work items, one- and two-head items, every MFMA group size and page sizes from
32 to 512 extends that pin to rows the oracle does not reach.  The bf16-probability mode
(auto) is compared with the same FP32 output within the north-star gate.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import MAX_ABS, MEAN_ABS
from jetspec_amd import PackedTreeMetadata, packed_tree_attention, packed_tree_attention_reference, \
    read_and_clear_status, workloads
from jetspec_amd.paged_backend import SUPPORTED_GROUPS, _fp32_template, _launch_fp32, _mfma_geometry

pytestmark = pytest.mark.gpu
DEV = "cuda"
EXACT_AGREEMENT = 5e-5


def random_batch(seed, big=False):
    """A seeded random batch; `big` draws 1 to 4 requests, the first with a tree of 1025 to
    2048 nodes (the MFMA kernel's large-tree range)."""
    rng = np.random.default_rng(seed)
    requests = int(rng.integers(1, 5)) if big else int(rng.integers(1, 49))
    block = int(rng.choice([32, 64, 128, 256, 512]))
    kv_heads = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice(SUPPORTED_GROUPS))
    dtype = torch.float16 if rng.random() < 0.25 else torch.bfloat16
    prefixes = [int(x) for x in rng.integers(0, 40000 if requests < 16 else 12000, size=requests)]
    counts = [int(rng.choice([1, 7, 16, 24, 33, 48, 64, 96, 129, 256, 500, 1024])) if rng.random() < 0.9 else 1
              for _ in range(requests)]
    if big:
        counts[0] = int(rng.integers(1025, 2049))
        prefixes = [min(p, 6000) for p in prefixes]
    parents = [workloads.random_parents(n, int(rng.integers(1, 12)), rng) if rng.random() < 0.7
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
    k = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(dtype)
    v = torch.randn((total, block, kv_heads, 128), generator=gen, device=DEV).to(dtype)
    q = torch.randn((meta.total_queries, groups * kv_heads, 128), generator=gen, device=DEV).to(dtype)
    label = (f"seed {seed}: R={requests} block={block} kv={kv_heads} G={groups} {dtype} rows={meta.total_queries} "
             f"max P={max(prefixes)} max T={max(counts)}")
    return q, k, v, meta, groups, label


@pytest.mark.parametrize("seed", range(16))
def test_mfma_kernel_equals_fp32_kernel(seed):
    q, k, v, meta, groups, label = random_batch(9100 + seed)
    print(f"[crosscheck] {label}", flush=True)
    assert _mfma_geometry(q, k, v, meta)
    scale = 128 ** -0.5
    stream = torch.cuda.current_stream().cuda_stream
    reference = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    _launch_fp32(_fp32_template(meta, k, v, groups, q.device), q, reference, scale, stream)
    exact = packed_tree_attention_reference(q, k, v, meta, scale, groups, output_dtype=torch.float32)
    fast = packed_tree_attention(q, k, v, meta, scale, groups)
    torch.cuda.synchronize()
    assert torch.isfinite(reference).all().item()
    d_exact = (exact - reference).abs()
    d_fast = (fast.float() - reference).abs()
    print(f"[crosscheck] exact max {d_exact.max().item():.2e} mean {d_exact.mean().item():.2e}; "
          f"bf16-P max {d_fast.max().item():.2e} mean {d_fast.mean().item():.2e}", flush=True)
    assert d_exact.max().item() <= EXACT_AGREEMENT
    assert d_fast.max().item() <= MAX_ABS and d_fast.mean().item() <= MEAN_ABS
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("seed", range(6))
def test_big_trees_mfma_kernel_equals_fp32_kernel(seed):
    q, k, v, meta, groups, label = random_batch(9300 + seed, big=True)
    print(f"[crosscheck big] {label}", flush=True)
    assert _mfma_geometry(q, k, v, meta)
    scale = 128 ** -0.5
    stream = torch.cuda.current_stream().cuda_stream
    reference = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    _launch_fp32(_fp32_template(meta, k, v, groups, q.device), q, reference, scale, stream)
    exact = packed_tree_attention_reference(q, k, v, meta, scale, groups, output_dtype=torch.float32)
    fast = packed_tree_attention(q, k, v, meta, scale, groups)
    torch.cuda.synchronize()
    d_exact = (exact - reference).abs()
    d_fast = (fast.float() - reference).abs()
    print(f"[crosscheck big] exact max {d_exact.max().item():.2e}; bf16-P max {d_fast.max().item():.2e} "
          f"mean {d_fast.mean().item():.2e}", flush=True)
    assert d_exact.max().item() <= EXACT_AGREEMENT
    assert d_fast.max().item() <= MAX_ABS and d_fast.mean().item() <= MEAN_ABS
    assert read_and_clear_status(DEV) == 0


def test_many_random_batches_agree():
    """250 more random batches in one pass, every row: a guard against rare ordering faults (a race
    between waves shows as one row off by the weight of one key, ~1e-4, only now and then)."""
    scale = 128 ** -0.5
    stream = torch.cuda.current_stream().cuda_stream
    failures = []
    for seed in range(40000, 40250):
        q, k, v, meta, groups, label = random_batch(seed)
        reference = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        _launch_fp32(_fp32_template(meta, k, v, groups, q.device), q, reference, scale, stream)
        exact = packed_tree_attention_reference(q, k, v, meta, scale, groups, output_dtype=torch.float32)
        fast = packed_tree_attention(q, k, v, meta, scale, groups)
        torch.cuda.synchronize()
        d_exact = (exact - reference).abs().max().item()
        d_fast = (fast.float() - reference).abs()
        if not (d_exact <= EXACT_AGREEMENT and d_fast.max().item() <= MAX_ABS and d_fast.mean().item() <= MEAN_ABS):
            failures.append(f"{label}: exact {d_exact:.2e}, bf16-P {d_fast.max().item():.2e}")
    print(f"[crosscheck] 250 batches, {len(failures)} disagreements", flush=True)
    assert not failures, failures[:5]
    assert read_and_clear_status(DEV) == 0
