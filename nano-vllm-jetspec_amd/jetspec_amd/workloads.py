"""Seeded synthetic verify batches at the shapes of the five benchmark configurations.

Qwen3-8B attention geometry (32 query heads, 8 KV heads, head_dim 128, bf16),
256-token pages drawn from a randomly permuted pool, N(0, 1) operands, trees from
seeded parent arrays (parent < child, bounded depth).  Mirrors the fixture style of
benchmarks/jetspec_tree_kernel_qualification.py:110-162: shuffled pages, scattered
scratch slots, unused pool rows optionally NaN so a read of them is detectable.

Index structures are generated on the host with numpy (seeded); K/V/Q payloads are
drawn on the target device with a seeded torch generator.
"""
from __future__ import annotations

from dataclasses import dataclass, field
import math

import numpy as np
import torch

from .packed_metadata import PackedTreeMetadata

Q_HEADS, KV_HEADS, HEAD_DIM, BLOCK = 32, 8, 128, 256


def random_parents(nodes: int, max_depth: int, rng: np.random.Generator) -> list[int]:
    """Parent array: root -1, every parent earlier than its child, depth <= max_depth."""
    parents = [-1]
    depth = [0]
    for node in range(1, nodes):
        eligible = [j for j in range(node) if depth[j] < max_depth]
        parent = int(eligible[rng.integers(len(eligible))])
        parents.append(parent)
        depth.append(depth[parent] + 1)
    return parents


def chain_parents(nodes: int) -> list[int]:
    """A causal chunk as a tree: node j's parent is j - 1 (prefill.py:14-26 visibility)."""
    return [-1] + list(range(nodes - 1))


def depths_of(parents: list[int]) -> list[int]:
    depth = [0] * len(parents)
    for node in range(1, len(parents)):
        depth[node] = depth[parents[node]] + 1
    return depth


def ancestor_mask(parents: list[int]) -> np.ndarray:
    """Self-inclusive ancestor matrix: row i marks i and every ancestor of i."""
    n = len(parents)
    mask = np.zeros((n, n), dtype=bool)
    for node in range(n):
        mask[node, node] = True
        if node:
            mask[node, :node] |= mask[parents[node], :node]
    return mask


@dataclass
class VerifyBatch:
    """One layer's packed verify inputs."""
    q: torch.Tensor                 # [Q, groups * KV heads, head_dim]
    k_pool: torch.Tensor            # [N, 256, 8, head_dim]
    v_pool: torch.Tensor
    metadata: PackedTreeMetadata
    new_k: torch.Tensor             # tree K/V to append into metadata.tree_slots
    new_v: torch.Tensor
    parents: list[list[int]]
    prefix_pages: list[list[int]]
    scale: float = HEAD_DIM ** -0.5
    groups: int = Q_HEADS // KV_HEADS
    head_dim: int = HEAD_DIM
    name: str = ""
    info: dict = field(default_factory=dict)

    @property
    def total_queries(self) -> int:
        return self.metadata.total_queries

    @property
    def kv_heads(self) -> int:
        return self.k_pool.shape[2]

    @property
    def q_heads(self) -> int:
        return self.q.shape[1]

    def algorithmic_bytes(self) -> int:
        """K/V of every visible position once per (request, KV head) + Q read + O write."""
        e = self.q.element_size()
        kv = sum(2 * (p + t) * self.kv_heads * self.head_dim * e
                 for p, t in zip(self.metadata.prefix_lengths, self.metadata.node_counts_host))
        qo = 2 * self.total_queries * self.q_heads * self.head_dim * e
        return kv + qo

    def algorithmic_flops(self) -> int:
        """4 * Hq * D per (row, visible key): QK^T and PV."""
        total = 0
        for prefix, parents in zip(self.metadata.prefix_lengths, self.parents):
            visible = sum(prefix + d + 1 for d in depths_of(parents))
            total += 4 * self.q_heads * self.head_dim * visible
        return total

    def append_bytes(self) -> int:
        return 2 * 2 * self.total_queries * self.kv_heads * self.head_dim * self.new_k.element_size()


def build_verify_batch(prefixes: list[int], trees: list[list[int]], *, device: torch.device | str,
                       seed: int, dtype: torch.dtype = torch.bfloat16, pool_fill: float = 1.0,
                       poison: bool = True, name: str = "", kv_heads: int = KV_HEADS,
                       groups: int = Q_HEADS // KV_HEADS, head_dim: int = HEAD_DIM) -> VerifyBatch:
    """Pages and slots from a permuted pool; payloads N(0,1); unused rows NaN if `poison`.

    `pool_fill` < 1 sizes the pool so live pages fill that fraction (fragmentation).
    Tree K/V are written into their scratch slots (the post-append state) and also
    returned as `new_k`/`new_v` for timing the append.  `kv_heads` < 8 builds one
    tensor-parallel shard: that many KV heads.  `groups` is the number of query heads
    per KV head (4 in the Qwen3-8B geometry), `head_dim` the head size (128 there).
    """
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    counts = [len(parents) for parents in trees]
    prefix_pages = [math.ceil(p / BLOCK) for p in prefixes]
    scratch_pages = math.ceil(sum(counts) / BLOCK) + 1
    live = sum(prefix_pages) + scratch_pages
    total_pages = max(live, math.ceil(live / pool_fill)) + (2 if pool_fill >= 1.0 else 0)
    order = rng.permutation(total_pages)
    tables = []
    cursor = 0
    for n in prefix_pages:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    scratch_slots = (scratch[:, None] * BLOCK + np.arange(BLOCK)[None, :]).reshape(-1)
    scratch_slots = scratch_slots[rng.permutation(scratch_slots.size)]
    slots, masks = [], []
    offset = 0
    for parents in trees:
        n = len(parents)
        slots.append(torch.as_tensor(scratch_slots[offset:offset + n].astype(np.int64), device=device))
        masks.append(torch.as_tensor(ancestor_mask(parents), device=device))
        offset += n
    metadata = PackedTreeMetadata.build(prefixes, tables, slots, masks, BLOCK)
    gen = torch.Generator(device=device).manual_seed(seed)
    shape = (total_pages, BLOCK, kv_heads, head_dim)
    k_pool = torch.empty(shape, dtype=dtype, device=device)
    v_pool = torch.empty(shape, dtype=dtype, device=device)
    k_pool.normal_(generator=gen)
    v_pool.normal_(generator=gen)
    if poison:
        used = np.zeros(total_pages * BLOCK, dtype=bool)
        for prefix, table in zip(prefixes, tables):
            pos = np.arange(prefix)
            used[np.asarray(table, dtype=np.int64)[pos // BLOCK] * BLOCK + pos % BLOCK] = True
        used[np.asarray(metadata.tree_slot_ids, dtype=np.int64)] = True
        unused = torch.as_tensor(np.flatnonzero(~used), device=device)
        k_pool.view(-1, kv_heads, head_dim)[unused] = float("nan")
        v_pool.view(-1, kv_heads, head_dim)[unused] = float("nan")
    total_q = metadata.total_queries
    q = torch.randn((total_q, groups * kv_heads, head_dim), generator=gen, device=device,
                    dtype=torch.float32).to(dtype)
    new_k = torch.randn((total_q, kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32).to(dtype)
    new_v = torch.randn((total_q, kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32).to(dtype)
    tree_slots = metadata.tree_slots
    k_pool.view(-1, kv_heads, head_dim)[tree_slots] = new_k
    v_pool.view(-1, kv_heads, head_dim)[tree_slots] = new_v
    return VerifyBatch(q=q, k_pool=k_pool, v_pool=v_pool, metadata=metadata, new_k=new_k, new_v=new_v,
                       parents=[list(p) for p in trees], prefix_pages=tables, name=name, groups=groups,
                       scale=head_dim ** -0.5, head_dim=head_dim,
                       info={"pages": total_pages, "pool_fill": pool_fill, "seed": seed})


def config1(device, seed: int = 1, **kw) -> VerifyBatch:
    """1 request, P=512, 16-node tree of depth <= 5."""
    rng = np.random.default_rng(seed)
    return build_verify_batch([512], [random_parents(16, 5, rng)], device=device, seed=seed, name="cfg1", **kw)


def config2(device, seed: int = 2, **kw) -> VerifyBatch:
    """8 requests, P ~ U[256, 4096], trees of {16, 32, 64} nodes, depth <= 8."""
    rng = np.random.default_rng(seed)
    prefixes = [int(x) for x in rng.integers(256, 4097, size=8)]
    trees = [random_parents(int(rng.choice([16, 32, 64])), 8, rng) for _ in range(8)]
    return build_verify_batch(prefixes, trees, device=device, seed=seed, name="cfg2", **kw)


def config4(device, seed: int = 4, requests: int = 64, **kw) -> VerifyBatch:
    """64 requests, P ~ U[8192, 32768], 64-node trees of depth <= 8, pool ~90 % full."""
    rng = np.random.default_rng(seed)
    prefixes = [int(x) for x in rng.integers(8192, 32769, size=requests)]
    trees = [random_parents(64, 8, rng) for _ in range(requests)]
    kw.setdefault("pool_fill", 0.9)
    kw.setdefault("poison", False)
    return build_verify_batch(prefixes, trees, device=device, seed=seed, name="cfg4", **kw)


def config5(device, seed: int = 5, **kw) -> VerifyBatch:
    """16 x 512-row causal prefill chunks on P ~ U[0, 16384] + 32 x 32-node trees on P ~ U[2048, 8192]."""
    rng = np.random.default_rng(seed)
    prefixes = [int(x) for x in rng.integers(0, 16385, size=16)]
    trees = [chain_parents(512) for _ in range(16)]
    prefixes += [int(x) for x in rng.integers(2048, 8193, size=32)]
    trees += [random_parents(32, 8, rng) for _ in range(32)]
    kw.setdefault("poison", False)
    return build_verify_batch(prefixes, trees, device=device, seed=seed, name="cfg5", **kw)


@dataclass
class CommitBatch:
    """Accepted-only commit across all layers (config 3)."""
    kv_pool: torch.Tensor            # [2, L, N, 256, 8, 128]
    source: torch.Tensor             # int64 [n]
    destination: torch.Tensor        # int64 [n]
    paths: list[list[int]]
    info: dict = field(default_factory=dict)

    def algorithmic_bytes(self) -> int:
        """Read + write of every accepted row, both KV axes, every layer."""
        layers = self.kv_pool.shape[1]
        row = self.kv_pool.shape[4] * self.kv_pool.shape[5] * self.kv_pool.element_size()
        return 2 * 2 * layers * int(self.source.numel()) * row


def config3(device, seed: int = 3, layers: int = 36, requests: int = 64, nodes: int = 32,
            dtype: torch.dtype = torch.bfloat16, fill: bool = True) -> CommitBatch:
    """64 requests with 32-node scratch trees; commit a root path of length 1..depth+1 per request.

    Destinations are the next slots after each prefix in that request's page list
    (a new page when the path crosses a page end), as state.py:782-785 builds them.
    """
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    prefixes = [int(x) for x in rng.integers(1024, 8193, size=requests)]
    trees = [random_parents(nodes, 8, rng) for _ in range(requests)]
    scratch_pages = math.ceil(requests * nodes / BLOCK)
    pages_needed = [math.ceil(p / BLOCK) for p in prefixes]
    paths, lengths = [], []
    for parents in trees:
        depth = depths_of(parents)
        length = int(rng.integers(1, max(depth) + 2))
        candidates = [n for n in range(len(parents)) if depth[n] == length - 1]
        node = int(candidates[rng.integers(len(candidates))])
        chain = [node]
        while parents[chain[-1]] != -1:
            chain.append(parents[chain[-1]])
        paths.append(chain[::-1])
        lengths.append(length)
    growth = [math.ceil((p + ln) / BLOCK) - math.ceil(p / BLOCK) for p, ln in zip(prefixes, lengths)]
    total_pages = sum(pages_needed) + sum(growth) + scratch_pages
    order = rng.permutation(total_pages)
    cursor = 0
    tables = []
    for need, grow in zip(pages_needed, growth):
        tables.append([int(x) for x in order[cursor:cursor + need + grow]])
        cursor += need + grow
    scratch = order[cursor:cursor + scratch_pages]
    scratch_slots = (scratch[:, None] * BLOCK + np.arange(BLOCK)[None, :]).reshape(-1)
    scratch_slots = scratch_slots[rng.permutation(scratch_slots.size)]
    source, destination = [], []
    for i, (prefix, path, table) in enumerate(zip(prefixes, paths, tables)):
        node_slots = scratch_slots[i * nodes:(i + 1) * nodes]
        source.extend(int(node_slots[j]) for j in path)
        for pos in range(prefix, prefix + len(path)):
            destination.append(table[pos // BLOCK] * BLOCK + pos % BLOCK)
    pool = torch.empty((2, layers, total_pages, BLOCK, KV_HEADS, HEAD_DIM), dtype=dtype, device=device)
    if fill:
        gen = torch.Generator(device=device).manual_seed(seed)
        pool.normal_(generator=gen)
    return CommitBatch(kv_pool=pool, source=torch.tensor(source, dtype=torch.int64, device=device),
                       destination=torch.tensor(destination, dtype=torch.int64, device=device), paths=paths,
                       info={"prefixes": prefixes, "pages": total_pages, "layers": layers, "seed": seed})
