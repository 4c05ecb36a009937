"""Slot-mapped K/V append (drop-in for layers/attention.py:38-45)."""
from __future__ import annotations

import torch

from . import _device, _lib


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """Copy row i of key/value into cache slot ``slot_mapping[i]``; slot -1 skips the row.

    Same argument contract and AssertionError checks as the reference
    (layers/attention.py:38-44); the copy is one HIP launch (tv_store_kvcache) on
    torch's current stream, bit-exact.  Also used for the tree-node append into
    scratch slots (replacing models/qwen3.py:255-258) with ``metadata.tree_slots``.
    """
    n, num_heads, head_dim = key.shape
    row = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == row and v_cache.stride(1) == row
    assert slot_mapping.numel() == n
    device = _device.require_gpu(key, value, k_cache, v_cache, slot_mapping, what="store_kvcache")
    if not (key.dtype == value.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("store_kvcache copies bits: key, value and both caches must share one dtype")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("slot_mapping must be int32 or int64")
    if n == 0:
        return
    slots = slot_mapping if slot_mapping.is_contiguous() else slot_mapping.contiguous()
    cache_slots = min(k_cache.numel(), v_cache.numel()) // row
    status = _device.status_word(device)
    code = _lib.library().tv_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        cache_slots, slots.data_ptr(), int(slots.dtype == torch.int64), n, row, key.element_size(),
        status.data_ptr(), _device.stream_handle(device))
    _lib.check(code, "store_kvcache")
