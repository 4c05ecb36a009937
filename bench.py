#!/usr/bin/env python3
"""Tree-verify throughput on one MI355X: one verify step = tree K/V append + packed tree attention.

    python bench.py [--steps K] [--warmup W] [--config 4] [--cpu-requests 16]

Default workload is BASELINE config 4 (the long-context, bandwidth-bound verify):
64 requests, prefix ~ U[8k, 32k], 64-node trees of depth <= 8, Qwen3-8B attention
geometry (32 q / 8 kv heads x 128, bf16), 256-token pages from a ~90 % full permuted
pool, N(0, 1) operands, synthetic and seeded.  One step is what one decoder layer
does per verify round on this hot path: store_kvcache of the 4096 tree K/V rows into
their scratch slots, then one packed_tree_attention launch.  Inputs are resident in
HBM before timing starts.

Prints ONE JSON line.  `value` = query rows (tree tokens) verified per second.
`roofline` is for the dominant kernel (tree attention): algorithmic bytes per launch
(K/V of every visible position once per request and KV head + Q + O) over its mean
duration from HIP events on the launch stream.  `cpu_baseline` times the reference's
PyTorch CPU path (oracle/cpu_path.py) on a bounded sample of the same batch.
Other configs (--config 1/2/3/5) are for measurement only.  `--kv-heads 1` measures one
tensor-parallel shard of the same batch (1 of the 8 KV heads with its 4 query heads, every
request's full context): the share of one GPU in an 8-way split over KV heads.
"""
from __future__ import annotations

import argparse
import json
import os
from pathlib import Path
import statistics
import sys
import time

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "nano-vllm-jetspec_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA, MI355X
METRIC = "tree-verify tokens/sec + achieved HBM GB/s (% of peak) on 1 MI355X"
WORKLOADS = {
    1: "cfg1: 1 request, P=512, 16-node tree depth<=5 (+ append)",
    2: "cfg2: 8 requests, P~U[256,4096], trees of {16,32,64} nodes depth<=8",
    3: "cfg3: accepted-only commit, 36 layers, 64 requests x 32-node scratch trees, P~U[1k,8k]",
    4: "cfg4: 64 requests, P~U[8k,32k], 64-node trees depth<=8, ~90% full permuted pool",
    5: "cfg5: 16 x 512-row causal chunks on P~U[0,16k] + 32 x 32-node trees on P~U[2k,8k]",
}


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", type=int, default=4, choices=sorted(WORKLOADS))
    parser.add_argument("--cpu-requests", type=int, default=16,
                        help="requests of the batch timed on the CPU path (0 disables the CPU baseline)")
    parser.add_argument("--seed", type=int, default=None)
    parser.add_argument("--kv-heads", type=int, default=8, choices=(1, 2, 4, 8),
                        help="KV heads of the batch (4 query heads each); below 8 it is one tensor-parallel "
                             "shard, measured on the verify step only")
    parser.add_argument("--groups", type=int, default=4, choices=(1, 2, 3, 4, 5, 6, 7, 8, 16),
                        help="query heads per KV head (4 in the Qwen3-8B geometry; 8 for Qwen3-32B, 16 for "
                             "Qwen3-235B-A22B); other than 4 it is measured on the verify step only")
    parser.add_argument("--head-dim", type=int, default=128, choices=(64, 128, 256),
                        help="head size of the batch (128 in the Qwen3 geometry); 64 and 256 run the MFMA "
                             "kernel's instances for those sizes, measured on the verify step only")
    parser.add_argument("--legs", choices=("all", "verify", "graph"), default="all",
                        help="'verify' measures only the verify step (for a kernel profile of exactly the timed "
                             "launches); 'graph' adds only the graph leg (a profile of the replayed round, device "
                             "planner included); 'all' adds the rope_scatter, accept, graph, exact and round legs")
    parser.add_argument("--operands", choices=("normal", "constant", "zero", "zero-q", "zero-kv"), default="normal",
                        help="diagnostic: replace the N(0,1) Q/K/V values by constants or zeros (same shapes, "
                             "pages, trees, instructions and bytes) to show the part's data-dependent clock; "
                             "'zero-q' zeroes only Q (random K/V still cross HBM and LDS), 'zero-kv' only the "
                             "K/V pool and new rows (random Q); the headline is 'normal'")
    parser.add_argument("--sustain", type=float, default=0.0,
                        help="diagnostic: after the timed steps, run the attention back to back for this many "
                             "seconds (so power and clock telemetry can be read while it runs) and report the "
                             "sustained time per launch")
    return parser.parse_args()


def source_digest(paths) -> str:
    """sha256 over the named source files (relative to the repository root), in order."""
    import hashlib

    digest = hashlib.sha256()
    for rel in paths:
        digest.update((ROOT / rel).read_bytes())
    return digest.hexdigest()[:16]


def traffic_bytes(key: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters (committed summary), or None
    when the kernel sources changed since that measurement (the entry's `source_sha` no longer
    matches), so a stale count is never reported."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(key)
    if entry is None or "sources" not in entry or entry.get("source_sha") != source_digest(entry["sources"]):
        return None
    return entry.get("hbm_bytes_per_launch")


def cpu_baseline(batch, requests: int) -> dict:
    """The reference's PyTorch CPU path on the first `requests` requests of the same batch."""
    import torch

    from oracle import cpu_path  # CPU baseline leg only
    from jetspec_amd import PackedTreeMetadata, workloads

    meta = batch.metadata
    chosen = list(range(min(requests, meta.num_requests)))
    block = meta.block_size
    slots_all = meta.tree_slots.cpu()
    pages = sorted({p for r in chosen for p in meta.block_tables_host[r]} |
                   {int(s) // block for r in chosen for s in slots_all[meta.request_slice(r)].tolist()})
    remap = {p: i for i, p in enumerate(pages)}
    index = torch.tensor(pages, device=batch.k_pool.device)
    k_pool = batch.k_pool.index_select(0, index).cpu()
    v_pool = batch.v_pool.index_select(0, index).cpu()
    rows = torch.cat([torch.arange(meta.request_slice(r).start, meta.request_slice(r).stop) for r in chosen])
    q = batch.q[rows.to(batch.q.device)].cpu()
    new_k = batch.new_k[rows.to(batch.q.device)].cpu()
    new_v = batch.new_v[rows.to(batch.q.device)].cpu()
    slots = [torch.tensor([remap[int(s) // block] * block + int(s) % block
                           for s in slots_all[meta.request_slice(r)].tolist()]) for r in chosen]
    ancestors = [torch.from_numpy(workloads.ancestor_mask(batch.parents[r])) for r in chosen]
    sub = PackedTreeMetadata.build([meta.prefix_lengths[r] for r in chosen],
                                   [[remap[p] for p in meta.block_tables_host[r]] for r in chosen],
                                   slots, ancestors, block)
    # Every host core of the box (torch.set_num_threads(os.cpu_count()), the CPU baseline plan).
    previous = torch.get_num_threads()
    threads = os.cpu_count() or previous
    torch.set_num_threads(threads)

    def step():
        cpu_path.append(k_pool, v_pool, new_k, new_v, sub.tree_slots)
        cpu_path.packed_attention(q, k_pool, v_pool, sub, ancestors, batch.scale)

    step()  # warmup
    samples = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        samples.append(time.perf_counter() - t0)
    seconds = statistics.median(samples)
    torch.set_num_threads(previous)
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = threads
    return {"value": sub.total_queries / seconds, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpus_in_affinity_mask": affinity,
            "sample": f"requests 0..{len(chosen) - 1} of the same batch ({sub.total_queries} tree rows, "
                      f"{sum(sub.prefix_lengths)} prefix tokens); append + bf16 SDPA over page-table-gathered K/V; "
                      f"median of 3 after 1 warmup, samples_s={[round(s, 3) for s in samples]}"}


def copy_probe(torch, gib: int = 2, reps: int = 10) -> dict:
    """Device-to-device copy of a known size: the measured HBM ceiling next to the 8 TB/s
    vendor peak, and the reference kernel for calibrating rocprofv3 FETCH/WRITE_SIZE."""
    n = gib << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    del src, dst
    return {"bytes_read": n, "bytes_written": n, "ms": ms, "gbs": 2 * n / (ms * 1e-3) / 1e9}


def samples(ms: list[float]) -> dict:
    """Per-launch device times of a GPU leg in the reference benchmark's style
    (jetspec_tree_kernel_benchmark.py:292-297,421-431): the median, with every sample kept."""
    return {"median_ms": statistics.median(ms), "mean_ms": statistics.mean(ms), "min_ms": min(ms),
            "max_ms": max(ms), "samples_ms": [round(x, 5) for x in ms]}


def event_times(events) -> list[float]:
    return [e[0].elapsed_time(e[1]) for e in events]


def rope_cache(torch, max_positions: int = 40960, dim: int = 128, base: float = 1e6):
    """Qwen3-8B's cos/sin cache (rope_theta 1e6, 40960 positions) as layers/rotary_embedding.py:28-35 builds it."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))
    freqs = torch.arange(max_positions, dtype=torch.float)[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1).to("cuda")


def rope_leg(batch, torch, steps: int, warmup: int) -> dict:
    """The fused HF-order RoPE + tree K/V scatter (tree_fusion.py:181-199) on the same tree rows.

    Positions are prefix length + node depth; the rotated K and raw V go to the batch's
    scratch slots, the rotated Q to a separate buffer.  Bytes per row: Q read and written,
    K and V read and written to the pool, one cos/sin cache row, the position and slot.
    """
    from jetspec_amd import rope_scatter_prevalidated, workloads

    meta = batch.metadata
    positions = torch.tensor([meta.prefix_lengths[r] + d for r in range(meta.num_requests)
                              for d in workloads.depths_of(batch.parents[r])], dtype=torch.int32, device="cuda")
    cache = rope_cache(torch)
    out = torch.empty_like(batch.q)
    stream = torch.cuda.current_stream()

    def launch():
        rope_scatter_prevalidated(batch.q, batch.new_k, batch.new_v, positions, cache, batch.k_pool, batch.v_pool,
                                  meta.tree_slots, out)

    for _ in range(warmup):
        launch()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for e in events:
        e[0].record(stream)
        launch()
        e[1].record(stream)
    torch.cuda.synchronize()
    times = event_times(events)
    ms = statistics.mean(times)
    rows, hq, dim = batch.q.shape
    hkv = batch.new_k.shape[1]
    elem = batch.q.element_size()
    per_row = 2 * hq * dim * elem + 4 * hkv * dim * elem + dim * cache.element_size() + 4 + meta.tree_slots.element_size()
    algo = rows * per_row
    gbs = algo / (ms * 1e-3) / 1e9
    return {"kernel": "rope_scatter_kernel", "rows": rows, "ms": ms, "algorithmic_bytes": algo, "achieved": gbs,
            "unit": "GB/s", "peak": HBM_PEAK_GBS, "frac": gbs / HBM_PEAK_GBS, **samples(times)}


def accept_leg(batch, torch, steps: int, warmup: int, vocab: int = 151936) -> dict:
    """Greedy acceptance on the device for the same tree rows: the argmax over Qwen3's
    vocabulary (bf16 synthetic logits) and the per-request walk.  torch.argmax on the same
    logits is timed beside it (the reference's own device step, serving_ops.py:62)."""
    from jetspec_amd import accept_batch_device, greedy_argmax, workloads

    meta = batch.metadata
    rows = meta.total_queries
    logits = torch.randn(rows, vocab, device="cuda", dtype=torch.bfloat16)
    tokens = torch.randint(0, vocab, (rows,), device="cuda")
    parents = torch.tensor([p for r in range(meta.num_requests) for p in batch.parents[r]], device="cuda")
    depths = torch.tensor([d for r in range(meta.num_requests) for d in workloads.depths_of(batch.parents[r])],
                          device="cuda")
    cu = meta.cu_seqlens_q
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(warmup):
            fn()
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
        for e in events:
            e[0].record(stream)
            fn()
            e[1].record(stream)
        torch.cuda.synchronize()
        return event_times(events)

    argmax_times = timed(lambda: greedy_argmax(logits))
    torch_times = timed(lambda: logits.argmax(-1))
    accept_times = timed(lambda: accept_batch_device(logits, tokens, parents, depths, cu, 15))
    argmax_ms, torch_ms, accept_ms = (statistics.mean(t) for t in (argmax_times, torch_times, accept_times))
    algo = rows * vocab * logits.element_size()
    gbs = algo / (argmax_ms * 1e-3) / 1e9
    del logits
    return {"kernel": "argmax_rows_kernel", "rows": rows, "vocab": vocab, "argmax_ms": argmax_ms,
            "torch_argmax_ms": torch_ms, "argmax_plus_walk_ms": accept_ms, "algorithmic_bytes": algo,
            "achieved": gbs, "unit": "GB/s", "peak": HBM_PEAK_GBS, "frac": gbs / HBM_PEAK_GBS,
            **samples(argmax_times), "torch_argmax_median_ms": statistics.median(torch_times),
            "argmax_plus_walk_median_ms": statistics.median(accept_times)}


def graph_leg(batch, torch, steps: int, warmup: int, layers: int = 36) -> dict:
    """A verify round's attention part for all 36 Qwen3-8B layers, eager vs one HIP-graph replay.

    Per layer: the fused RoPE + scatter and the drop-in packed attention, called the way
    models/qwen3.py:223-240 calls them.  The graph is the reference runner's form
    (target_graph.py:135-167): the same calls captured once against the round's metadata and
    replayed; under capture the attention plans on the device, so the graph stays valid while
    prefix lengths, trees and node counts change.  Every layer reuses the batch's pool and
    inputs (the work per layer is the same; 36 distinct pools of config 4 would not fit the
    memory twice).  Wall-clock per round, host launch cost included: the quantity a graph
    removes."""
    from jetspec_amd import packed_tree_attention, rope_scatter_prevalidated, workloads

    meta = batch.metadata
    positions = torch.tensor([meta.prefix_lengths[r] + d for r in range(meta.num_requests)
                              for d in workloads.depths_of(batch.parents[r])], dtype=torch.int32, device="cuda")
    cache = rope_cache(torch)

    def round_():
        out = None
        for _ in range(layers):
            rotated = rope_scatter_prevalidated(batch.q, batch.new_k, batch.new_v, positions, cache, batch.k_pool,
                                                batch.v_pool, meta.tree_slots, torch.empty_like(batch.q))
            out = packed_tree_attention(rotated, batch.k_pool, batch.v_pool, meta, batch.scale, batch.groups)
        return out

    def wall(fn, rounds):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(rounds):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / rounds

    rounds = max(3, min(steps, 20))
    eager_ms = wall(round_, rounds)
    expected = round_()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        round_()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured = round_()
    replay_ms = wall(graph.replay, rounds)
    same = bool(torch.equal(captured.view(torch.int16), expected.view(torch.int16)))
    return {"layers": layers, "eager_ms_per_round": eager_ms, "graph_replay_ms_per_round": replay_ms,
            "speedup": eager_ms / replay_ms, "bitwise_equal": same}


COMMIT_SPIN_CYCLES = 400_000   # ~0.2-0.3 ms at the part's clock


def round_leg(batch, torch, rounds: int, layers: int = 36, vocab: int = 151936) -> dict:
    """One whole verify round of the hot path on the batch's requests: for each of the 36 layers
    the tree K/V append (store_kvcache into the scratch slots) and the packed attention, then
    greedy acceptance (device argmax over Qwen3's vocabulary + tree walk), the max_new_tokens /
    EOS cut, the commit maps and the accepted-only commit of every layer (copy_accepted_kv).

    The reference's round (batch_runtime.py:496-655, state.py:800-926) runs these per layer and
    then once per round.  Every layer's attention reads the batch's pool: its K/V (GBs) is far
    larger than the 256 MB Infinity Cache, so each layer streams it from HBM as 36 distinct
    layers would (36 of config 4's pools would need ~230 GB).  The commit moves rows of a
    36-layer pool holding the tree scratch pages (the batch's scratch pages renumbered) and two
    fresh pages per request after its prefix.  Tree tokens are set so that each request accepts
    the ancestor chain of one seeded node (1 to depth + 1 rows, as config 3 draws them).  As in
    the reference, the host reads the accepted row count once, before the commit.  Device time
    (events, the host turnaround excluded) and wall time per round; the median over rounds,
    every round kept."""
    import numpy as np

    from jetspec_amd import (accept_batch_device, commit_slots, copy_accepted_kv, packed_tree_attention,
                             store_kvcache, truncate_accepted, workloads)

    meta = batch.metadata
    requests, rows, block = meta.num_requests, meta.total_queries, meta.block_size
    rng = np.random.default_rng(17)
    logits = torch.randn(rows, vocab, device="cuda", dtype=torch.bfloat16)
    greedy = logits.argmax(-1).cpu().numpy()
    tokens = rng.integers(0, vocab, size=rows)
    parents_flat, depths_flat, chosen = [], [], []
    for r, parents in enumerate(batch.parents):
        base = meta.request_slice(r).start
        depth = workloads.depths_of(parents)
        # The walk accepts at most max_depth + 1 = 16 nodes (serving_ops.py:78-83).
        length = int(rng.integers(1, min(max(depth), 15) + 2))
        candidates = [n for n in range(len(parents)) if depth[n] == length - 1]
        node = int(candidates[rng.integers(len(candidates))])
        chain = [node]
        while parents[chain[-1]] != -1:
            chain.append(parents[chain[-1]])
        chain = chain[::-1]
        on_chain = set(chain)
        # The chain's children carry their parent's argmax; no other child of a chain node does,
        # so the walk takes exactly the chain and stops at its end.
        for n in range(1, len(parents)):
            want = greedy[base + parents[n]]
            if n in on_chain:
                tokens[base + n] = want
            elif parents[n] in on_chain and tokens[base + n] == want:
                tokens[base + n] = (want + 1) % vocab
        parents_flat += list(parents)
        depths_flat += list(depth)
        chosen.append(chain)
    accepted_rows = sum(len(c) for c in chosen)
    tokens_dev = torch.as_tensor(tokens, dtype=torch.int64, device="cuda")
    parents_dev = torch.as_tensor(parents_flat, dtype=torch.int64, device="cuda")
    depths_dev = torch.as_tensor(depths_flat, dtype=torch.int64, device="cuda")
    budgets = torch.full((requests,), 1 << 20, dtype=torch.int32, device="cuda")
    ignore_eos = torch.ones(requests, dtype=torch.uint8, device="cuda")
    # The commit's 36-layer pool: the batch's tree scratch pages, then two pages per request that
    # hold positions prefix .. prefix + 16 (a request's next positions, state.py:782-785).
    slot_ids = np.asarray(meta.tree_slot_ids, dtype=np.int64)
    scratch_pages = sorted(set((slot_ids // block).tolist()))
    renumber = {page: i for i, page in enumerate(scratch_pages)}
    commit_tree_slots = torch.as_tensor(
        np.array([renumber[s // block] * block + s % block for s in slot_ids.tolist()], dtype=np.int64), device="cuda")
    width = max(p // block for p in meta.prefix_lengths) + 2
    tables = np.full((requests, width), -1, dtype=np.int32)
    for r, prefix in enumerate(meta.prefix_lengths):
        tables[r, prefix // block] = len(scratch_pages) + 2 * r
        tables[r, prefix // block + 1] = len(scratch_pages) + 2 * r + 1
    pages = len(scratch_pages) + 2 * requests
    kv36 = torch.empty((2, layers, pages, block, batch.kv_heads, 128), dtype=batch.k_pool.dtype, device="cuda")
    kv36.normal_(generator=torch.Generator(device="cuda").manual_seed(36))
    tables_dev = torch.as_tensor(tables, device="cuda")
    cache_lens = torch.as_tensor(meta.prefix_lengths, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def one_round(events):
        events[0].record(stream)
        for _ in range(layers):
            store_kvcache(batch.new_k, batch.new_v, batch.k_pool, batch.v_pool, meta.tree_slots)
            packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, meta, batch.scale, batch.groups)
        events[1].record(stream)
        _, paths, lengths, corrections = accept_batch_device(logits, tokens_dev, parents_dev, depths_dev,
                                                             meta.cu_seqlens_q, 15)
        _, _, commit_paths, commit_offsets = truncate_accepted(paths, lengths, corrections, tokens_dev,
                                                               meta.cu_seqlens_q, budgets, ignore_eos, [])
        source, destination = commit_slots(commit_tree_slots, meta.cu_seqlens_q, commit_paths, commit_offsets,
                                           tables_dev, cache_lens, block, pages)
        events[2].record(stream)
        n = int(commit_offsets[-1].item())   # the one host read of the round
        # A short GPU spin ahead of the commit, so that its launch reaches the stream before the
        # GPU does and events 3-4 bracket the commit's device time, not the host's launch latency
        # (the spin lies outside every timed interval; the wall time includes it).
        torch.cuda._sleep(COMMIT_SPIN_CYCLES)
        events[3].record(stream)
        payload = copy_accepted_kv(kv36, source[:n], destination[:n], block)
        events[4].record(stream)
        return n, payload

    for _ in range(2):
        one_round([torch.cuda.Event(enable_timing=True) for _ in range(5)])
    torch.cuda.synchronize()
    record, walls = [], []
    for _ in range(rounds):
        events = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        t0 = time.perf_counter()
        n, payload = one_round(events)
        torch.cuda.synchronize()
        walls.append((time.perf_counter() - t0) * 1e3)
        record.append((events[0].elapsed_time(events[1]), events[1].elapsed_time(events[2]),
                       events[3].elapsed_time(events[4])))
    if n != accepted_rows:
        raise RuntimeError(f"round leg accepted {n} rows, expected {accepted_rows}")
    layer_ms = [a for a, _, _ in record]
    accept_ms = [b for _, b, _ in record]
    commit_ms = [c for _, _, c in record]
    device_ms = [a + b + c for a, b, c in record]
    layer_bytes = layers * (batch.algorithmic_bytes() + batch.append_bytes())
    accept_bytes = rows * vocab * logits.element_size()
    commit_bytes = 2 * payload   # every payload byte read once and written once
    total = layer_bytes + accept_bytes + commit_bytes
    ms = statistics.median(device_ms)
    del logits, kv36
    return {"layers": layers, "requests": requests, "tree_rows": rows, "accepted_rows": n,
            "device_ms_median": ms, "wall_ms_median": statistics.median(walls),
            "layers_ms_median": statistics.median(layer_ms), "accept_ms_median": statistics.median(accept_ms),
            "commit_ms_median": statistics.median(commit_ms),
            "algorithmic_bytes": total, "layers_bytes": layer_bytes, "accept_bytes": accept_bytes,
            "commit_bytes": commit_bytes, "achieved_gbs": total / (ms * 1e-3) / 1e9,
            "frac": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "device_samples_ms": [round(x, 4) for x in device_ms], "wall_samples_ms": [round(x, 4) for x in walls]}


def exact_leg(batch, torch, steps: int, warmup: int) -> dict:
    """The explicit FP32-probability entry (backend="reference", paged_backend.py:248-256) on the
    same batch: probabilities kept to ~2^-17 relative in the P.V product (two MFMAs per P.V
    step), HIP events on the launch stream."""
    from jetspec_amd import packed_tree_attention

    meta, stream = batch.metadata, torch.cuda.current_stream()

    def call():
        return packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, meta, batch.scale, batch.groups,
                                     backend="reference")
    for _ in range(warmup):
        call()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    torch.cuda.synchronize()
    for e in events:
        e[0].record(stream)
        call()
        e[1].record(stream)
    torch.cuda.synchronize()
    times = event_times(events)
    ms = statistics.mean(times)
    algo = batch.algorithmic_bytes()
    gbs = algo / (ms * 1e-3) / 1e9
    return {"kernel": "tree_attention_kernel (exact probabilities)", "backend": "reference", "ms": ms,
            "algorithmic_bytes": algo, "achieved": gbs, "unit": "GB/s", "peak": HBM_PEAK_GBS,
            "frac": gbs / HBM_PEAK_GBS, **samples(times)}


def sustain_leg(batch, torch, seconds: float) -> dict:
    """The verify attention back to back for `seconds` of wall time, synchronising every 50
    launches (a steady load for reading the part's power and clock telemetry)."""
    from jetspec_amd import packed_tree_attention

    meta = batch.metadata
    print(f"[sustain] attention back to back for {seconds:.1f} s", file=sys.stderr, flush=True)
    launches, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, meta, batch.scale, batch.groups)
        torch.cuda.synchronize()
        launches += 50
    wall = time.perf_counter() - t0
    return {"seconds": wall, "launches": launches, "ms_per_launch": wall * 1e3 / launches}


def run_verify(args, torch):
    from jetspec_amd import packed_tree_attention, read_and_clear_status, store_kvcache, workloads

    builder = {1: workloads.config1, 2: workloads.config2, 4: workloads.config4, 5: workloads.config5}[args.config]
    kwargs = {} if args.seed is None else {"seed": args.seed}
    if args.kv_heads != 8:
        kwargs["kv_heads"] = args.kv_heads
    if args.groups != 4:
        kwargs["groups"] = args.groups
    if args.head_dim != 128:
        kwargs["head_dim"] = args.head_dim
    batch = builder("cuda", **kwargs)
    meta = batch.metadata
    stream = torch.cuda.current_stream()
    if args.operands != "normal":
        # The chosen tensors get one value in every element (zeros, or 0.5 / 0.25 / -0.5):
        # the work is unchanged, only those operand bits stop toggling.
        values = {"constant": (0.5, 0.25, -0.5), "zero": (0.0, 0.0, 0.0), "zero-q": (0.0, None, None),
                  "zero-kv": (None, 0.0, 0.0)}[args.operands]
        for tensor, value in zip((batch.q, batch.k_pool, batch.v_pool), values):
            if value is not None:
                tensor.fill_(value)
        if values[1] is not None:
            batch.new_k.fill_(values[1])
            batch.new_v.fill_(values[2])

    def step(events=None):
        if events is not None:
            events[0].record(stream)
        store_kvcache(batch.new_k, batch.new_v, batch.k_pool, batch.v_pool, meta.tree_slots)
        if events is not None:
            events[1].record(stream)
        out = packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, meta, batch.scale, batch.groups)
        if events is not None:
            events[2].record(stream)
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    status = read_and_clear_status("cuda")
    if status:
        raise RuntimeError(f"kernel status bits {status}: an index was out of range")
    attn_times = [e[1].elapsed_time(e[2]) for e in events]
    append_times = [e[0].elapsed_time(e[1]) for e in events]
    attn_ms, append_ms = statistics.mean(attn_times), statistics.mean(append_times)
    algo_bytes = batch.algorithmic_bytes()
    algo_flops = batch.algorithmic_flops()
    achieved = algo_bytes / (attn_ms * 1e-3) / 1e9
    tflops = algo_flops / (attn_ms * 1e-3) / 1e12
    # The roof that bounds the kernel: HBM below the ridge point (peak flop/s / peak B/s),
    # the matrix cores above it (config 5's 512-row causal chunks).
    mfma_bound = algo_flops / algo_bytes > MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    tokens = meta.total_queries
    result = {
        "metric": METRIC, "value": tokens * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": ("synthetic (seeded N(0,1) bf16 Q/K/V, seeded parent arrays, permuted page pool)"
                 if args.operands == "normal" else
                 f"synthetic, diagnostic {args.operands} Q/K/V values (seeded parent arrays, permuted page pool)"),
        "config": {"workload": WORKLOADS[args.config], "requests": meta.num_requests,
                   "tree_rows_per_step": tokens, "prefix_tokens": sum(meta.prefix_lengths),
                   "q_heads": batch.q_heads, "kv_heads": batch.kv_heads, "head_dim": batch.head_dim,
                   "page": meta.block_size, "layers_per_step": 1, "pool_pages": batch.info["pages"]},
        "roofline": {"bound": "mfma" if mfma_bound else "hbm",
                     "achieved": tflops if mfma_bound else achieved,
                     "peak": MFMA_BF16_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBS,
                     "unit": "TFLOP/s" if mfma_bound else "GB/s",
                     "frac": tflops / MFMA_BF16_PEAK_TFLOPS if mfma_bound else achieved / HBM_PEAK_GBS,
                     "traffic": (traffic_bytes(f"cfg{args.config}")
                                 if args.kv_heads == 8 and args.groups == 4 and args.head_dim == 128 else None),
                     "kernel": "tree_attention_kernel", "kernel_ms": attn_ms, "algorithmic_bytes": algo_bytes,
                     "algorithmic_flops": algo_flops, "achieved_gbs": achieved, "achieved_tflops": tflops,
                     "append_ms": append_ms, "append_gbs": batch.append_bytes() / (append_ms * 1e-3) / 1e9,
                     "kernel_ms_median": statistics.median(attn_times),
                     "kernel_samples_ms": [round(x, 5) for x in attn_times],
                     "append_ms_median": statistics.median(append_times),
                     "append_samples_ms": [round(x, 5) for x in append_times]},
    }
    if args.kv_heads != 8:
        result["config"]["shard"] = f"tensor-parallel shard: {batch.kv_heads} of 8 KV heads"
    if args.groups != 4:
        result["config"]["geometry"] = f"{args.groups} query heads per KV head"
    if args.legs != "verify" and args.kv_heads == 8 and args.groups == 4 and args.head_dim == 128:
        if args.legs == "all":
            result["rope_scatter"] = rope_leg(batch, torch, args.steps, args.warmup)
            result["accept"] = accept_leg(batch, torch, args.steps, args.warmup)
        result["graph"] = graph_leg(batch, torch, args.steps, args.warmup)
        if args.legs == "all":
            result["exact"] = exact_leg(batch, torch, args.steps, args.warmup)
            result["round"] = round_leg(batch, torch, rounds=3 if args.config == 4 else 5)
    if args.sustain > 0:
        result["sustained"] = sustain_leg(batch, torch, args.sustain)
    probe = copy_probe(torch)
    result["roofline"]["measured_copy_gbs"] = probe["gbs"]
    result["roofline"]["frac_of_measured_copy"] = achieved / probe["gbs"]
    if (args.cpu_requests > 0 and args.config in (1, 2, 4, 5) and args.operands == "normal"
            and args.groups == 4 and args.kv_heads == 8 and args.head_dim == 128):
        result["cpu_baseline"] = cpu_baseline(batch, args.cpu_requests)
    return result


def run_commit(args, torch):
    from jetspec_amd import copy_accepted_kv, read_and_clear_status, workloads

    batch = workloads.config3("cuda") if args.seed is None else workloads.config3("cuda", seed=args.seed)
    pool, src, dst = batch.kv_pool, batch.source, batch.destination
    for _ in range(args.warmup):
        copy_accepted_kv(pool, src, dst, pool.shape[3])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        copy_accepted_kv(pool, src, dst, pool.shape[3])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Device time per commit: a second pass, queued behind a GPU spin so the launches
    # reach the stream before the GPU does and the events bracket only device work (a
    # commit takes less GPU time than its host-side call).  MI355X's 256 MB Infinity
    # Cache would hold a 68 MB commit's rows from one repetition to the next, which a
    # served round (36 layers of multi-GB attention reads before its commit) never sees:
    # every timed commit is therefore preceded, outside its events, by a 1 GiB read that
    # evicts the cache and leaves it clean, as the attention's reads of the pool would
    # ("cold", the reported rate).  The same pass without it is reported as "warm".
    flush = torch.ones(1 << 28, dtype=torch.float32, device="cuda")

    def device_ms(cold: bool) -> float:
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        for e in events:
            if cold:
                flush.amax()
            e[0].record(stream)
            copy_accepted_kv(pool, src, dst, pool.shape[3])
            e[1].record(stream)
        torch.cuda.synchronize()
        # Median: the first interval can also span the tail of the spin.
        return statistics.median(e[0].elapsed_time(e[1]) for e in events)

    ms = device_ms(cold=True)
    warm_ms = device_ms(cold=False)
    # The same bytes as one contiguous device copy (half read, half written), timed the
    # same way: the ceiling a gather/scatter of 2 KB rows is compared with at this size
    # and cache state.
    algo = batch.algorithmic_bytes()
    copy_src = torch.empty(algo // 2, dtype=torch.uint8, device="cuda")
    copy_dst = torch.empty_like(copy_src)

    def copy_ms(cold: bool) -> float:
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        for e in events:
            if cold:
                flush.amax()
            e[0].record(stream)
            copy_dst.copy_(copy_src)
            e[1].record(stream)
        torch.cuda.synchronize()
        return statistics.median(e[0].elapsed_time(e[1]) for e in events)

    copy_cold_ms, copy_warm_ms = copy_ms(cold=True), copy_ms(cold=False)
    del flush, copy_src, copy_dst
    if read_and_clear_status("cuda"):
        raise RuntimeError("commit reported an out-of-range slot")
    achieved = algo / (ms * 1e-3) / 1e9
    rows = int(src.numel())
    probe = copy_probe(torch)
    return {"metric": "accepted KV rows committed/sec (36 layers) + achieved HBM GB/s", "value": rows * args.steps / elapsed,
            "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": WORKLOADS[3], "accepted_rows": rows, "pool_pages": batch.info["pages"]},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_bytes("cfg3"), "kernel_ms": ms,
                         "cache": "cold (Infinity Cache evicted by a 1 GiB read before each timed commit)",
                         "warm_kernel_ms": warm_ms, "warm_gbs": algo / (warm_ms * 1e-3) / 1e9,
                         "algorithmic_bytes": algo, "measured_copy_gbs": probe["gbs"],
                         "frac_of_measured_copy": achieved / probe["gbs"],
                         "same_bytes_copy_cold_ms": copy_cold_ms, "same_bytes_copy_warm_ms": copy_warm_ms,
                         "frac_of_same_bytes_copy_cold": copy_cold_ms / ms,
                         "frac_of_same_bytes_copy_warm": copy_warm_ms / warm_ms}}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (--gpus {args.gpus} refused)",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 1
    result = run_commit(args, torch) if args.config == 3 else run_verify(args, torch)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
