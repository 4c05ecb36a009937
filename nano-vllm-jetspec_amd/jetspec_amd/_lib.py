"""ctypes binding of libtreeverify.so (the C ABI declared in include/treeverify.h).

The shared library is built in-tree by ``nano-vllm-jetspec_amd/build.py``.  There
is no fallback: if the library is missing or does not match this binding, every
device entry point raises ``RuntimeError`` naming the problem.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path
import threading

LIBRARY_PATH = Path(__file__).resolve().parent / "libtreeverify.so"
ABI_VERSION = 4

TV_OK = 0
TV_ERR_INVALID = -1
TV_ERR_UNSUPPORTED = -2
TV_ERR_LAUNCH = -3
TV_ERR_CAPACITY = -4

TV_BF16 = 0
TV_F16 = 1
TV_F32 = 2

TV_STATUS_BAD_PAGE = 1
TV_STATUS_BAD_SLOT = 2
TV_STATUS_BAD_REQUEST = 4
TV_STATUS_BAD_POSITION = 8
TV_STATUS_BAD_DEPTH = 16
TV_STATUS_BAD_BIAS = 32
TV_STATUS_STALE_PLAN = 64

# Every extern "C" symbol of include/treeverify.h.
EXPORTED_SYMBOLS = (
    "tv_abi_version",
    "tv_last_error",
    "tv_sizeof_tree_attention_args",
    "tv_store_kvcache",
    "tv_copy_accepted_kv_workspace_bytes",
    "tv_copy_accepted_kv",
    "tv_commit_slots",
    "tv_truncate_accepted",
    "tv_tree_attention_plan",
    "tv_tree_attention_plan_slots",
    "tv_pack_ancestor_words",
    "tv_tree_attention",
    "tv_sizeof_rope_scatter_args",
    "tv_rope_scatter",
    "tv_argmax_rows",
    "tv_tree_accept",
    "tv_ancestor_words_from_parents",
    "tv_bias_from_ancestor_words",
    "tv_tree_attention_plan_capacity",
    "tv_tree_attention_plan_device",
    "tv_tree_attention_plan_capacity_packed",
    "tv_stream_capture_info",
    "tv_tree_attention_noalloc",
    "tv_tree_attention_noalloc_max_workspace",
    "tv_tree_attention_workspace_bytes",
    "tv_tree_attention_fp32",
    "tv_sizeof_tree_attention_fp32_args",
)


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("num_items", c_int32),
        ("num_groups", c_int32),
        ("num_partial_slots", c_int32),
        ("ancestor_words_per_row", c_int32),
        ("workspace_bytes", c_int64),
    ]


class TreeAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p),
        ("q_stride_row", c_int64),
        ("q_stride_head", c_int64),
        ("k_pool", c_void_p),
        ("v_pool", c_void_p),
        ("k_stride", c_int64 * 4),
        ("v_stride", c_int64 * 4),
        ("num_blocks", c_int64),
        ("in_dtype", c_int32),
        ("out", c_void_p),
        ("out_stride_row", c_int64),
        ("out_stride_head", c_int64),
        ("out_dtype", c_int32),
        ("cu_seqlens_q", c_void_p),
        ("prefix_lens", c_void_p),
        ("node_counts", c_void_p),
        ("block_tables", c_void_p),
        ("block_table_stride", c_int64),
        ("tree_slots", c_void_p),
        ("ancestor_words", c_void_p),
        ("ancestor_words_per_row", c_int32),
        ("num_requests", c_int32),
        ("total_queries", c_int32),
        ("num_q_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("block_size", c_int32),
        ("scale", c_float),
        ("items", c_void_p),
        ("num_items", c_int32),
        ("groups", c_void_p),
        ("num_groups", c_int32),
        ("num_partial_slots", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_int64),
        ("status", c_void_p),
        ("device_counts", c_void_p),
        ("prefix_slots", c_void_p),
        ("prefix_slots_stride", c_int64),
        ("prefix_slots_is_int64", c_int32),
        ("exact_probabilities", c_int32),
    ]


class TreeAttentionFp32Args(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p),
        ("q_stride_row", c_int64),
        ("q_stride_head", c_int64),
        ("k_pool", c_void_p),
        ("v_pool", c_void_p),
        ("k_stride", c_int64 * 4),
        ("v_stride", c_int64 * 4),
        ("num_blocks", c_int64),
        ("in_dtype", c_int32),
        ("out", c_void_p),
        ("out_stride_row", c_int64),
        ("out_stride_head", c_int64),
        ("out_dtype", c_int32),
        ("cu_seqlens_q", c_void_p),
        ("query_to_request", c_void_p),
        ("query_local_row", c_void_p),
        ("prefix_lens", c_void_p),
        ("node_counts", c_void_p),
        ("block_tables", c_void_p),
        ("block_table_stride", c_int64),
        ("tree_slots", c_void_p),
        ("qq_bias", c_void_p),
        ("qq_bias_offsets", c_void_p),
        ("prefix_slots", c_void_p),
        ("prefix_slots_stride", c_int64),
        ("prefix_slots_is_int64", c_int32),
        ("num_requests", c_int32),
        ("total_queries", c_int32),
        ("num_q_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("block_size", c_int32),
        ("scale", c_float),
        ("status", c_void_p),
    ]


class RopeScatterArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p), ("q_stride", c_int64 * 3),
        ("k", c_void_p), ("k_stride", c_int64 * 3),
        ("v", c_void_p), ("v_stride", c_int64 * 3),
        ("positions", c_void_p), ("positions_stride", c_int64), ("positions_is_int64", c_int32),
        ("cache", c_void_p), ("cache_rows", c_int64), ("cache_stride_row", c_int64), ("cache_stride_elem", c_int64),
        ("cache_dtype", c_int32),
        ("k_pool", c_void_p), ("k_pool_stride", c_int64 * 4),
        ("v_pool", c_void_p), ("v_pool_stride", c_int64 * 4),
        ("pool_pages", c_int64), ("page_size", c_int64),
        ("node_slots", c_void_p), ("slots_stride", c_int64), ("slots_is_int64", c_int32),
        ("out", c_void_p), ("out_stride", c_int64 * 3),
        ("rows", c_int64),
        ("q_heads", c_int32), ("kv_heads", c_int32), ("head_dim", c_int32), ("dtype", c_int32),
        ("status", c_void_p),
    ]


_lock = threading.Lock()
_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    lib.tv_abi_version.restype = c_int32
    lib.tv_abi_version.argtypes = []
    lib.tv_last_error.restype = c_char_p
    lib.tv_last_error.argtypes = []
    lib.tv_sizeof_tree_attention_args.restype = c_int64
    lib.tv_sizeof_tree_attention_args.argtypes = []
    lib.tv_store_kvcache.restype = c_int32
    lib.tv_store_kvcache.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                     c_void_p, c_int32, c_int64, c_int64, c_int32, c_void_p, c_void_p]
    lib.tv_copy_accepted_kv_workspace_bytes.restype = c_int64
    lib.tv_copy_accepted_kv_workspace_bytes.argtypes = [c_int64, c_int64, c_int64, c_int32]
    lib.tv_copy_accepted_kv.restype = c_int32
    lib.tv_copy_accepted_kv.argtypes = [c_void_p, POINTER(c_int64), POINTER(c_int64), c_int32, c_void_p,
                                        c_void_p, c_int64, c_void_p, c_int64, POINTER(c_int64), c_void_p,
                                        c_void_p]
    lib.tv_commit_slots.restype = c_int32
    lib.tv_commit_slots.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p,
                                    c_int32, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]
    lib.tv_truncate_accepted.restype = c_int32
    lib.tv_truncate_accepted.argtypes = [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_int32,
                                         c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_void_p]
    lib.tv_tree_attention_plan.restype = c_int32
    lib.tv_tree_attention_plan.argtypes = [POINTER(c_int32), POINTER(c_int32), c_int32, c_int32, c_int32,
                                           c_int32, c_int32, c_int32, POINTER(c_int32), POINTER(c_int32),
                                           POINTER(PlanInfo)]
    lib.tv_tree_attention_plan_slots.restype = c_int32
    lib.tv_tree_attention_plan_slots.argtypes = [POINTER(c_int32), POINTER(c_int32), c_int32, c_int32, c_int32,
                                                 c_int32, c_int32, POINTER(c_int32), POINTER(c_int32),
                                                 POINTER(PlanInfo)]
    lib.tv_pack_ancestor_words.restype = c_int32
    lib.tv_pack_ancestor_words.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                           c_int32, c_void_p, c_void_p, c_void_p]
    lib.tv_tree_attention.restype = c_int32
    lib.tv_tree_attention.argtypes = [POINTER(TreeAttentionArgs), c_void_p]
    lib.tv_tree_attention_noalloc.restype = c_int32
    lib.tv_tree_attention_noalloc.argtypes = [POINTER(TreeAttentionArgs), c_void_p]
    lib.tv_tree_attention_noalloc_max_workspace.restype = c_int64
    lib.tv_tree_attention_noalloc_max_workspace.argtypes = []
    lib.tv_tree_attention_workspace_bytes.restype = c_int64
    lib.tv_tree_attention_workspace_bytes.argtypes = [c_int32, c_int32]
    lib.tv_tree_attention_fp32.restype = c_int32
    lib.tv_tree_attention_fp32.argtypes = [POINTER(TreeAttentionFp32Args), c_void_p]
    lib.tv_sizeof_tree_attention_fp32_args.restype = c_int64
    lib.tv_sizeof_tree_attention_fp32_args.argtypes = []
    lib.tv_sizeof_rope_scatter_args.restype = c_int64
    lib.tv_sizeof_rope_scatter_args.argtypes = []
    lib.tv_rope_scatter.restype = c_int32
    lib.tv_rope_scatter.argtypes = [POINTER(RopeScatterArgs), c_void_p]
    lib.tv_argmax_rows.restype = c_int32
    lib.tv_argmax_rows.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int32, c_void_p, c_void_p]
    lib.tv_ancestor_words_from_parents.restype = c_int32
    lib.tv_ancestor_words_from_parents.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                                   c_void_p]
    lib.tv_bias_from_ancestor_words.restype = c_int32
    lib.tv_bias_from_ancestor_words.argtypes = [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                                c_void_p, c_void_p]
    lib.tv_tree_attention_plan_capacity.restype = c_int32
    lib.tv_tree_attention_plan_capacity.argtypes = [POINTER(c_int32), c_int32, c_int32, c_int32, c_int32, c_int32,
                                                    c_int32, c_int64, POINTER(PlanInfo)]
    lib.tv_tree_attention_plan_device.restype = c_int32
    lib.tv_tree_attention_plan_device.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                                  c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                                  c_void_p]
    lib.tv_tree_attention_plan_capacity_packed.restype = c_int32
    lib.tv_tree_attention_plan_capacity_packed.argtypes = [c_int32, c_int32, c_int64, c_int32, c_int32, c_int32,
                                                           c_int32, c_int32, c_int64, POINTER(PlanInfo)]
    lib.tv_stream_capture_info.restype = c_int32
    lib.tv_stream_capture_info.argtypes = [c_void_p, POINTER(c_int32), POINTER(c_uint64)]
    lib.tv_tree_accept.restype = c_int32
    lib.tv_tree_accept.argtypes = [c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_int32, c_void_p,
                                   c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]


def library() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"{LIBRARY_PATH} is missing: build it with `python nano-vllm-jetspec_amd/build.py` "
                "(there is no non-HIP fallback)")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        missing = [name for name in EXPORTED_SYMBOLS if not hasattr(lib, name)]
        if missing:
            raise RuntimeError(f"{LIBRARY_PATH} lacks symbols {missing}; rebuild it")
        _declare(lib)
        version = lib.tv_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libtreeverify ABI {version} != binding ABI {ABI_VERSION}; rebuild it")
        if lib.tv_sizeof_tree_attention_args() != ctypes.sizeof(TreeAttentionArgs):
            raise RuntimeError("tv_tree_attention_args layout differs between library and binding")
        if lib.tv_sizeof_rope_scatter_args() != ctypes.sizeof(RopeScatterArgs):
            raise RuntimeError("tv_rope_scatter_args layout differs between library and binding")
        _lib = lib
        return lib


def check(code: int, what: str) -> None:
    """Raise for a nonzero C-ABI return code, with the library's message."""
    if code == TV_OK:
        return
    message = library().tv_last_error().decode(errors="replace")
    if code in (TV_ERR_INVALID, TV_ERR_UNSUPPORTED, TV_ERR_CAPACITY):
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message} (code {code})")
