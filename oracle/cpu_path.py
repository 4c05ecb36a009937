"""The reference's PyTorch CPU path for this hot path - TEST / BASELINE INFRASTRUCTURE ONLY.

Restates, on CPU tensors, what the reference runs when no Triton kernel is used:
  attention   gather committed K/V through the page table (layers/attention.py:87-93),
              append the tree K/V, build the bool visibility [T, P+T] with an all-visible
              prefix and the ancestor matrix over the tree (speculative/jetspec/
              runtime.py:486-488), turn it into an additive 0 / finfo.min mask, expand the
              KV heads to the query heads and call scaled_dot_product_attention
              (models/qwen3.py:161-189).  A causal chunk is a chain tree, whose ancestor
              matrix is the offset-causal mask of prefill.py:14-26.
  append      k_pool[blocks, offsets] = k  (models/qwen3.py:255-258)
  commit      advanced-index gather + scatter (speculative/jetspec/state.py:80-85)

bench.py times this as the CPU baseline (kind "port") on the host cores; tests use
the attention in float32 as a second reference next to the fp64 oracle.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def gather_paged(cache: torch.Tensor, pages, length: int) -> torch.Tensor:
    """Rows [0, length) of one request through its page list (layers/attention.py:87-93)."""
    block = cache.shape[1]
    pos = torch.arange(length)
    table = torch.as_tensor(list(pages), dtype=torch.long)
    return cache[table[pos // block], pos % block]


def request_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, pages, prefix: int,
                      tree_slots: torch.Tensor, ancestor: torch.Tensor, scale: float,
                      dtype: torch.dtype | None = None) -> torch.Tensor:
    """One request's tree rows: q [T, Hq, D] -> [T, Hq, D] (computed in `dtype`, default q.dtype)."""
    dtype = dtype or q.dtype
    block = k_pool.shape[1]
    n = q.shape[0]
    k_tree = k_pool[tree_slots // block, tree_slots % block]
    v_tree = v_pool[tree_slots // block, tree_slots % block]
    k_all = torch.cat((gather_paged(k_pool, pages, prefix), k_tree)).to(dtype)
    v_all = torch.cat((gather_paged(v_pool, pages, prefix), v_tree)).to(dtype)
    allowed = torch.zeros((n, prefix + n), dtype=torch.bool)
    allowed[:, :prefix] = True
    allowed[:, prefix:] = ancestor
    mask = torch.where(allowed, torch.zeros((), dtype=dtype), torch.full((), torch.finfo(dtype).min, dtype=dtype))
    groups = q.shape[1] // k_all.shape[1]
    qh = q.to(dtype).transpose(0, 1).unsqueeze(0)
    kh = k_all.transpose(0, 1).unsqueeze(0)
    vh = v_all.transpose(0, 1).unsqueeze(0)
    batch, heads, length, dim = kh.shape
    kh = kh[:, :, None].expand(batch, heads, groups, length, dim).reshape(batch, heads * groups, length, dim)
    vh = vh[:, :, None].expand(batch, heads, groups, length, dim).reshape(batch, heads * groups, length, dim)
    out = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask.view(1, 1, n, prefix + n), dropout_p=0.0,
                                         scale=scale)
    return out.squeeze(0).transpose(0, 1).contiguous()


def packed_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, metadata, ancestors,
                     scale: float, requests=None, dtype: torch.dtype | None = None) -> dict[int, torch.Tensor]:
    """Per-request outputs {request: [T, Hq, D]} for the packed batch (CPU tensors)."""
    slots = metadata.tree_slots.cpu()
    result = {}
    for r in (range(metadata.num_requests) if requests is None else requests):
        sl = metadata.request_slice(r)
        result[r] = request_attention(q[sl], k_pool, v_pool, metadata.block_tables_host[r],
                                      metadata.prefix_lengths[r], slots[sl], ancestors[r], scale, dtype)
    return result


def append(k_pool: torch.Tensor, v_pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
           slots: torch.Tensor) -> None:
    """Eager tree scatter (models/qwen3.py:255-258)."""
    block = k_pool.shape[1]
    blocks = torch.div(slots, block, rounding_mode="floor").long()
    offsets = torch.remainder(slots, block).long()
    k_pool[blocks, offsets] = k
    v_pool[blocks, offsets] = v


def copy_accepted_kv(kv_pool: torch.Tensor, source: torch.Tensor, destination: torch.Tensor, block_size: int) -> int:
    """Advanced-index gather then scatter (state.py:80-86); returns payload bytes."""
    accepted = kv_pool[:, :, torch.div(source, block_size, rounding_mode="floor"), source % block_size]
    kv_pool[:, :, torch.div(destination, block_size, rounding_mode="floor"), destination % block_size] = accepted
    return int(accepted.numel() * accepted.element_size())
