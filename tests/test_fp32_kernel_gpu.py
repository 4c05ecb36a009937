"""The FP32 kernel (tv_tree_attention_fp32): every geometry outside the MFMA kernel (GPU).

The reference's dispatcher runs its scalar FP32 kernel for every batch outside its fast
kernel's geometry (paged_backend.py:288-306), and its FP32 entries accept f32 operands
(tree_attention.py:31-37).  This build's drop-in sends those batches to the FP32 kernel.
Each case below is outside the MFMA kernel's geometry and is checked against the fp64
oracle: FP32 output within the reference's FP32 qualification bound
(FP32_ATTENTION_BOUND = 1e-4, benchmarks/jetspec_numeric_oracles.py:21,108-168), bf16
output within the north-star gate.  Pools carry NaN in every unused row.

Cases: f32 Q/K/V through every FP32 entry; head sizes 64, 96, 256 and 512; query groups
9, 12 and 32; page sizes 16 and 48; a 1500-node causal chunk; a K/V pool whose head
dimension is strided; finite qq_bias values (legacy entry; the packed MFMA path flags
them); bad pages; and a captured launch that follows staged metadata.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

import oracle
from gpu_helpers import MAX_ABS, MEAN_ABS, errors, metrics, oracle_rows
from jetspec_amd import (PackedTreeMetadata, _lib, packed_tree_attention, packed_tree_attention_gqa,
                         packed_tree_attention_prefix_split_exact, packed_tree_attention_reference,
                         paged_tree_attention, read_and_clear_status, workloads)
from jetspec_amd.paged_backend import _mfma_geometry

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_case(prefixes, counts, *, kv_heads=2, groups=4, head_dim=128, block=256, dtype=torch.bfloat16, seed=0,
              chain=False, pool_dim=None):
    """Shuffled pages, scattered scratch slots, NaN in every unused pool row.  `pool_dim`
    > head_dim stores each head in a wider row (the kernel then reads a strided view)."""
    rng = np.random.default_rng(seed)
    prefix_pages = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    total = sum(prefix_pages) + scratch_pages + 3
    order = rng.permutation(total)
    tables, cursor = [], 0
    for n in prefix_pages:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    pool_slots = (scratch[:, None] * block + np.arange(block)).reshape(-1)[rng.permutation(scratch_pages * block)]
    slots, masks, off = [], [], 0
    for n in counts:
        slots.append(torch.as_tensor(pool_slots[off:off + n].astype(np.int64), device=DEV))
        parents = workloads.chain_parents(n) if chain else workloads.random_parents(n, 8, rng)
        masks.append(torch.as_tensor(workloads.ancestor_mask(parents), device=DEV))
        off += n
    meta = PackedTreeMetadata.build(list(prefixes), tables, slots, masks, block)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    width = pool_dim or head_dim
    k_full = torch.full((total, block, kv_heads, width), float("nan"), device=DEV, dtype=dtype)
    v_full = torch.full_like(k_full, float("nan"))
    live = [torch.as_tensor(np.asarray(t, dtype=np.int64)[np.arange(p) // block] * block + np.arange(p) % block,
                            device=DEV) for t, p in zip(tables, prefixes)]
    live = torch.cat(live + slots)
    for pool in (k_full, v_full):
        pool.view(-1, kv_heads, width)[live] = torch.randn((live.numel(), kv_heads, width), generator=gen,
                                                           device=DEV).to(dtype)
    k, v = (k_full, v_full) if pool_dim is None else (k_full[..., ::2], v_full[..., ::2])
    q = torch.randn((meta.total_queries, kv_heads * groups, head_dim), generator=gen, device=DEV).to(dtype)
    return q, k, v, meta, slots, masks


def check(out, q, k, v, meta, label, rows_per_request=None, scale=None):
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all().item(), f"{label}: NaN padding was read"
    expect = oracle_rows(q, k, v, meta, scale, list(range(meta.num_requests)), rows_per_request=rows_per_request)
    m = metrics(out, expect)
    mx, mean = errors(out, expect)
    print(f"[{label}] {out.dtype} max-abs {mx:.3e} mean-abs {mean:.3e} rel-RMS {m['relative_rms_error']:.3e}",
          flush=True)
    if out.dtype == torch.float32:
        assert m["within_fixed_bound"], (label, m)
    else:
        assert mx <= MAX_ABS and mean <= MEAN_ABS, label
    assert read_and_clear_status(DEV) == 0


def test_f32_operands_through_every_fp32_entry():
    q, k, v, meta, *_ = make_case((65, 0, 257), (63, 31, 47), dtype=torch.float32, seed=1)
    assert not _mfma_geometry(q, k, v, meta)
    scale = 128 ** -0.5
    for label, out in (
            ("auto", packed_tree_attention(q, k, v, meta, scale, 4)),
            ("reference", packed_tree_attention(q, k, v, meta, scale, 4, backend="reference")),
            ("prefix", packed_tree_attention(q, k, v, meta, scale, 4, backend="prefix")),
            ("reference entry", packed_tree_attention_reference(q, k, v, meta, scale, 4, output_dtype=torch.float32)),
            ("split exact", packed_tree_attention_prefix_split_exact(q, k, v, meta, scale, 4))):
        assert out.dtype == torch.float32
        check(out, q, k, v, meta, f"f32 {label}")
    with pytest.raises(ValueError, match="requires BF16 or FP16"):
        packed_tree_attention_gqa(q, k, v, meta, scale, 4)
    with pytest.raises(ValueError, match="requires BF16 or FP16"):
        packed_tree_attention(q, k, v, meta, scale, 4, backend="gqa")


@pytest.mark.parametrize("head_dim,groups", [(64, 3), (96, 4), (256, 3), (512, 4)])
def test_head_sizes(head_dim, groups):
    """Head sizes outside the MFMA kernel's (128 for every group, 64 and 256 for the power-of-two
    groups, tests/test_head64_gpu.py and tests/test_head256_gpu.py)."""
    q, k, v, meta, *_ = make_case((300, 0, 1025), (17, 40, 64), head_dim=head_dim, groups=groups, seed=head_dim)
    assert not _mfma_geometry(q, k, v, meta)
    scale = head_dim ** -0.5
    check(packed_tree_attention(q, k, v, meta, scale, groups), q, k, v, meta, f"D{head_dim} auto", scale=scale)
    check(packed_tree_attention(q, k, v, meta, scale, groups, output_dtype=torch.float32), q, k, v, meta,
          f"D{head_dim} f32 out", scale=scale)


@pytest.mark.parametrize("groups,kv_heads", [(9, 2), (12, 1), (32, 1)])
def test_query_groups_beyond_the_mfma_kernel(groups, kv_heads):
    q, k, v, meta, *_ = make_case((129, 7, 700), (9, 33, 20), kv_heads=kv_heads, groups=groups, seed=groups)
    assert not _mfma_geometry(q, k, v, meta)
    scale = 128 ** -0.5
    check(packed_tree_attention(q, k, v, meta, scale, groups), q, k, v, meta, f"G{groups}")
    check(packed_tree_attention_reference(q, k, v, meta, scale, groups, output_dtype=torch.float32), q, k, v, meta,
          f"G{groups} f32 out")
    with pytest.raises(ValueError, match="power-of-two GQA"):
        packed_tree_attention(q, k, v, meta, scale, groups, backend="gqa")


@pytest.mark.parametrize("block", [16, 48])
def test_page_sizes_that_are_not_multiples_of_32(block):
    q, k, v, meta, *_ = make_case((0, 47, 48, 49, 1000), (5, 16, 3, 64, 30), block=block, seed=block)
    assert not _mfma_geometry(q, k, v, meta)
    check(packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4), q, k, v, meta, f"B{block}")


def test_causal_chunk_above_2048_nodes():
    q, k, v, meta, *_ = make_case((2000, 100), (2100, 64), kv_heads=1, chain=True, seed=9)
    assert not _mfma_geometry(q, k, v, meta)
    check(packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4), q, k, v, meta, "2100-row chunk",
          rows_per_request=24)


def test_strided_head_dimension_in_the_pool():
    q, k, v, meta, *_ = make_case((500, 33), (20, 12), pool_dim=256, seed=12)
    assert k.stride(3) == 2 and not _mfma_geometry(q, k, v, meta)
    check(packed_tree_attention(q, k, v, meta, 128 ** -0.5, 4), q, k, v, meta, "strided head dim")


def test_finite_bias_legacy_entry_adds_it_and_packed_path_flags_it():
    q, k, v, meta, slots, masks = make_case((65, 0), (24, 9), kv_heads=2, seed=13)
    scale = 128 ** -0.5
    rows = meta.request_slice(0)
    local_q = q[rows].contiguous()
    n, prefix = rows.stop - rows.start, meta.prefix_lengths[0]
    rng = np.random.default_rng(14)
    bias_host = np.where(masks[0].cpu().numpy(), rng.uniform(-2.0, 1.0, size=(n, n)), -np.inf).astype(np.float32)
    bias = torch.as_tensor(bias_host, device=DEV)
    pages = torch.tensor(meta.block_tables_host[0], device=DEV, dtype=torch.int64)
    positions = torch.arange(prefix, device=DEV)
    logical = torch.cat((pages[positions // 256] * 256 + positions % 256, slots[0]))
    out = paged_tree_attention(local_q, k, v, None, None, torch.tensor([prefix + n], device=DEV), bias, scale, 4, 256,
                               logical.view(1, -1))
    torch.cuda.synchronize()
    # fp64 oracle with the finite bias: one request, the whole (small) pool.
    q64 = local_q.float().cpu().numpy()
    meta_arrays = oracle.metadata_arrays([prefix], [meta.block_tables_host[0]], [slots[0].tolist()],
                                         [masks[0].cpu().numpy()], 256)
    meta_arrays["qq_bias"] = bias_host.reshape(-1)
    expect = oracle.tree_attention_f64(q64, k.float().cpu().numpy(), v.float().cpu().numpy(), scale=scale,
                                       **meta_arrays)
    err = np.abs(out.float().cpu().numpy() - expect)
    print(f"[finite bias legacy] max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS
    # The same bias cannot be carried as visibility bits: the packed MFMA path says so.
    assert read_and_clear_status(DEV) == 0
    biased = replace(meta, qq_bias=meta.qq_bias.clone())
    biased.qq_bias[:n * n] = bias.view(-1)
    packed_tree_attention(q, k, v, biased, scale, 4)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == _lib.TV_STATUS_BAD_BIAS


def test_bad_pages_set_status_without_faulting():
    q, k, v, meta, *_ = make_case((300, 20), (16, 8), head_dim=96, seed=15)
    bad = replace(meta, block_tables=meta.block_tables.clone())
    bad.block_tables[0, 0] = 10 ** 6
    out = packed_tree_attention(q, k, v, bad, 96 ** -0.5, 4)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) & _lib.TV_STATUS_BAD_PAGE
    rows = bad.request_slice(1)
    good = packed_tree_attention(q, k, v, meta, 96 ** -0.5, 4)
    assert torch.equal(out[rows].view(torch.int16), good[rows].view(torch.int16))   # other requests untouched
    assert read_and_clear_status(DEV) == 0


FIELDS = ("cu_seqlens_q", "query_to_request", "query_local_row", "prefix_lens", "block_tables", "tree_slots",
          "qq_bias", "qq_bias_offsets", "node_counts")


def test_captured_fp32_route_follows_staged_metadata():
    """A head size the MFMA kernel does not take, under the reference's graph flow:
    capture against a staged metadata object, then replay after copy_-ing rounds with
    other prefixes and trees of the same signature (target_graph.py:55-75,150-167)."""
    rounds = [((12, 60, 72), (300, 70, 500)), ((24, 36, 84), (510, 25, 257)), ((72, 12, 60), (1, 800, 96))]
    cases = [make_case(p, c, head_dim=96, seed=40 + i) for i, (c, p) in enumerate(rounds)]
    pages = max(int(c[1].shape[0]) for c in cases)
    k = torch.randn((pages, 256, 2, 96), device=DEV).to(torch.bfloat16)
    v = torch.randn_like(k)
    width = 4
    staged = None
    q_in = torch.empty_like(cases[0][0])
    for index, (q, _, _, meta, *_) in enumerate(cases):
        if staged is None:
            tensors = {name: torch.empty_like(getattr(meta, name)) for name in FIELDS if name != "block_tables"}
            tensors["block_tables"] = torch.full((meta.num_requests, width), -1, dtype=torch.int32, device=DEV)
            staged = replace(meta, **tensors)
        for name in FIELDS:
            dst, src = getattr(staged, name), getattr(meta, name)
            if name == "block_tables":
                dst[:, :src.shape[1]].copy_(src)
            else:
                dst.copy_(src)
        q_in.copy_(q)
        if index == 0:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                packed_tree_attention(q_in, k, v, staged, 0.125, 4)    # warm-up
            torch.cuda.current_stream().wait_stream(stream)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                captured = packed_tree_attention(q_in, k, v, staged, 0.125, 4)
        graph.replay()
        torch.cuda.synchronize()
        eager = packed_tree_attention(q, k, v, meta, 0.125, 4)
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), f"round {index}"
        check(captured.clone(), q, k, v, meta, f"captured D96 round {index}", scale=0.125)
        torch.randn(1 << 20, device=DEV).sum().item()   # eager work between replays
