"""Device plumbing shared by the operator wrappers: streams, dtypes, status words."""
from __future__ import annotations

from functools import lru_cache

import numpy as np
import torch

from . import _lib

_DTYPE_CODES = {torch.bfloat16: _lib.TV_BF16, torch.float16: _lib.TV_F16, torch.float32: _lib.TV_F32}
_status_words: dict[int, torch.Tensor] = {}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def require_gpu(*tensors: torch.Tensor, what: str) -> torch.device:
    """All tensors on one GPU; these operators have no CPU implementation."""
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError(f"{what} requires GPU tensors (got {device}); there is no CPU path")
    for tensor in tensors[1:]:
        if tensor.device != device:
            raise ValueError(f"{what} requires all tensors on one device")
    return device


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def status_word(device: torch.device) -> torch.Tensor:
    """Per-device int32 that kernels OR TV_STATUS_* bits into (zeroed once)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    word = _status_words.get(index)
    if word is None:
        word = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", index))
        _status_words[index] = word
    return word


def read_and_clear_status(device: torch.device | str | int = "cuda") -> int:
    """Synchronising diagnostic: the accumulated TV_STATUS_* bits, then reset."""
    device = torch.device(device) if not isinstance(device, torch.device) else device
    if device.type != "cuda":
        device = torch.device("cuda", int(device.index or 0))
    word = status_word(device)
    value = int(word.item())
    word.zero_()
    return value


@lru_cache(maxsize=None)
def compute_units(index: int) -> int:
    return int(torch.cuda.get_device_properties(index).multi_processor_count)


def upload_fields(fields: dict[str, np.ndarray], device: torch.device, *, pinned: bool) -> dict[str, torch.Tensor]:
    """All fields in one host-to-device transfer: a byte buffer with each field at an offset
    aligned to its element size (largest elements first), then typed device views by name."""
    order = sorted(fields, key=lambda name: -fields[name].itemsize)
    offsets, cursor = {}, 0
    for name in order:
        itemsize = fields[name].itemsize
        cursor = (cursor + itemsize - 1) // itemsize * itemsize
        offsets[name] = cursor
        cursor += fields[name].nbytes
    host = torch.empty(max(cursor, 8), dtype=torch.uint8, pin_memory=pinned)
    raw = host.numpy()
    for name in order:
        array = fields[name]
        raw[offsets[name]:offsets[name] + array.nbytes] = array.reshape(-1).view(np.uint8)
    blob = host.to(device, non_blocking=pinned)
    views = {}
    for name in order:
        array = fields[name]
        typed = torch.int64 if array.dtype == np.int64 else torch.int32
        views[name] = blob[offsets[name]:offsets[name] + array.nbytes].view(typed)
    return views
