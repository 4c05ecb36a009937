"""The drop-in packed_tree_attention under the reference's CUDA-graph runner flow (GPU).

speculative/jetspec/target_graph.py:55-167 (PackedTargetGraph) builds a staged metadata
object with dataclasses.replace (fresh device tensors, a fixed-width block table),
warms the forward up on it, captures the forward once, and for every later round of
the same signature (requests, packed rows, qq_bias elements; :24-27) copy_s the
round's metadata into the staged tensors and replays.  The forward calls the rebound
module attributes exactly as models/qwen3.py:223-240 does:
rope_scatter_prevalidated, then packed_tree_attention(..., backend=...).

Each replay here has different prefix lengths (longer and shorter than at capture,
crossing page ends, including an empty prefix), different pages, trees and node
counts (same signature: (12, 60, 72) and (24, 36, 84) have equal sums and equal sums
of squares), and is checked
  * within the north-star gate against the fp64 oracle on the replay's own inputs,
  * bitwise against the eager drop-in path on the round's real metadata,
with eager work and synchronisations between replays.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from gpu_helpers import assert_within_gate, oracle_rows
from jetspec_amd import (PackedTreeMetadata, packed_tree_attention, read_and_clear_status,
                         rope_scatter_prevalidated, workloads)

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIELDS = ("cu_seqlens_q", "query_to_request", "query_local_row", "prefix_lens", "block_tables", "tree_slots",
          "qq_bias", "qq_bias_offsets", "node_counts")
SCALE = 128 ** -0.5
PAGES = 160
TABLE_WIDTH = 32          # max_model_len 8192 at 256-token pages
LAYERS = 2

# Same request count, packed rows (144) and qq_bias elements (8928) in every round.
ROUNDS = [
    ((12, 60, 72), (3000, 700, 5000)),
    ((24, 36, 84), (5100, 255, 257)),
    ((72, 12, 60), (1, 8000, 4096)),
    ((84, 24, 36), (0, 512, 7777)),
]


def round_inputs(seed, counts, prefixes, groups=4):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(PAGES)
    cursor, tables, slots, masks, depths = 0, [], [], [], []
    for p in prefixes:
        need = (p + 255) // 256
        tables.append([int(x) for x in perm[cursor:cursor + need]])
        cursor += need
    scratch = [int(x) for x in perm[cursor:cursor + (sum(counts) + 255) // 256 + 1]]
    order = rng.permutation(sum(counts))   # scattered scratch slots
    offset = 0
    for n in counts:
        local = order[offset:offset + n]
        slots.append(torch.tensor([scratch[int(j) // 256] * 256 + int(j) % 256 for j in local], device=DEV))
        offset += n
        parents = workloads.random_parents(n, 8, rng)
        masks.append(torch.from_numpy(workloads.ancestor_mask(parents)).to(DEV))
        depths.append(workloads.depths_of(parents))
    meta = PackedTreeMetadata.build(list(prefixes), tables, slots, masks, 256)
    positions = torch.tensor([prefixes[r] + d for r, ds in enumerate(depths) for d in ds], device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed)
    rows = sum(counts)
    q = torch.randn(LAYERS, rows, 8 * groups, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(LAYERS, rows, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(LAYERS, rows, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    return meta, positions, q, k, v


def stage(staged, metadata):
    """target_graph.py:63-75."""
    for name in FIELDS:
        dst, src = getattr(staged, name), getattr(metadata, name)
        if name == "block_tables":
            dst[:, :src.shape[1]].copy_(src)
        else:
            dst.copy_(src)


def staged_from(metadata):
    """target_graph.py:77-87."""
    tensors = {name: torch.empty_like(getattr(metadata, name)) for name in FIELDS if name != "block_tables"}
    tensors["block_tables"] = torch.full((metadata.num_requests, TABLE_WIDTH), -1, dtype=torch.int32, device=DEV)
    staged = replace(metadata, **tensors)
    stage(staged, metadata)
    return staged


def forward(kv_pool, cache, metadata, positions, q, k, v, backend):
    """The per-layer calls of models/qwen3.py:223-240 (RMS norm and projections aside)."""
    rotated, outs = [], []
    for layer in range(LAYERS):
        kp, vp = kv_pool[0, layer], kv_pool[1, layer]
        rq = rope_scatter_prevalidated(q[layer], k[layer], v[layer], positions, cache, kp, vp, metadata.tree_slots,
                                       torch.empty_like(q[layer]))
        rotated.append(rq)
        outs.append(packed_tree_attention(rq, kp, vp, metadata, SCALE, q.shape[2] // kp.shape[2], backend=backend))
    return torch.stack(rotated), torch.stack(outs)


def rope_cache():
    angles = torch.arange(8192, device=DEV, dtype=torch.float32)[:, None] * (
        torch.arange(64, device=DEV, dtype=torch.float32)[None, :] + 1) * 1e-3
    return torch.cat((angles.cos(), angles.sin()), -1).unsqueeze(1)


@pytest.mark.parametrize("backend,groups", [("auto", 4), ("gqa", 4), ("auto", 1), ("gqa", 16)])
def test_captured_dropin_follows_staged_metadata(backend, groups):
    g = torch.Generator(device=DEV).manual_seed(21)
    pool = torch.randn(2, LAYERS, PAGES, 256, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    cache = rope_cache()
    meta0, pos0, q0, k0, v0 = round_inputs(500, *ROUNDS[0], groups=groups)
    staged = staged_from(meta0)
    inputs = {"positions": pos0.clone(), "q": q0.clone(), "k": k0.clone(), "v": v0.clone()}
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):   # warm-up on the staged object, eagerly (target_graph.py:141-143)
            forward(pool, cache, staged, inputs["positions"], inputs["q"], inputs["k"], inputs["v"], backend)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured = forward(pool, cache, staged, inputs["positions"], inputs["q"], inputs["k"], inputs["v"], backend)
    torch.cuda.synchronize()
    for index, (counts, prefixes) in enumerate(ROUNDS):
        meta, positions, q, k, v = (meta0, pos0, q0, k0, v0) if index == 0 else round_inputs(
            500 + index, counts, prefixes, groups=groups)
        reference_pool = pool.clone()
        expect_rotated, expect_out = forward(reference_pool, cache, meta, positions, q, k, v, backend)
        torch.cuda.synchronize()
        stage(staged, meta)
        for name, value in (("positions", positions), ("q", q), ("k", k), ("v", v)):
            inputs[name].copy_(value)
        graph.replay()
        torch.cuda.synchronize()
        print(f"[capture/{backend}/G{groups}] round {index}: nodes {counts} prefixes {prefixes}", flush=True)
        rotated, out = captured[0].clone(), captured[1].clone()
        assert torch.equal(rotated.view(torch.int16), expect_rotated.view(torch.int16)), f"round {index} rope"
        assert torch.equal(pool.view(torch.int16), reference_pool.view(torch.int16)), f"round {index} pool"
        assert torch.equal(out.view(torch.int16), expect_out.view(torch.int16)), f"round {index} vs eager"
        for layer in range(LAYERS):
            expected = oracle_rows(rotated[layer], pool[0, layer], pool[1, layer], meta, SCALE,
                                   list(range(meta.num_requests)))
            assert_within_gate(out[layer], expected, f"capture/{backend}/G{groups} round {index} layer {layer}")
        assert read_and_clear_status(DEV) == 0
        torch.randn(1 << 20, device=DEV).sum().item()   # eager work between replays

