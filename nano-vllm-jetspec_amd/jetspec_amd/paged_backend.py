"""Packed ragged tree-verify attention on MI355X (drop-in for paged_backend.py:240-306).

Every public entry keeps the reference's signature, argument meaning and ValueError
conditions, and runs hand-written HIP kernels (libtreeverify).  The reference's
numerical variants (frozen FP32 ``reference``, ``prefix``, grouped ``gqa``) differ only
in tiling and precision knobs; here they are one MFMA kernel (tv_tree_attention) with
bf16/f16 products, fp32 accumulation and online softmax, in two probability modes:
``auto`` and ``gqa`` round each probability to the operand type for the P.V product
(as the reference's gqa backend, tree_gqa.py:102-105); the explicit FP32 entries
(``reference``, ``prefix``, and their modules' other entries) keep it to about 2^-17
relative (two MFMAs: its rounding and the rounding of the remainder) and sum it in
fp32, the reference's "never BF16 probabilities" (paged_backend.py:248-256).

Batches outside the MFMA kernel's geometry (f32 operands, head sizes other than 64, 128
and 256, query groups other than 1-8 and 16 (1, 2, 4, 8 and 16 at head sizes 64 and 256),
page sizes that are not multiples of 32, trees above MFMA_MAX_TREE_NODES nodes, unaligned
pools) run the FP32 kernel (tv_tree_attention_fp32), as the
reference's dispatcher runs its scalar FP32 kernel outside its fast kernel's geometry
(paged_backend.py:288-306).  It reads every metadata value from device memory, needs
no plan, and is capturable as is.

Two launch modes, chosen per call:

* Eager (the stream is not capturing).  Per metadata object the wrapper derives,
  once: the work plan (tv_tree_attention_plan over the host prefix/node counts) and
  the ancestor bit rows (tv_pack_ancestor_words over qq_bias, or the words the
  serving constructor built on the device).  Per (metadata, K/V pool, stream) it
  keeps a filled argument block and, when the plan splits prefixes, one partial-
  result workspace that the 36 per-layer launches of a round reuse in stream order.
  A steady-state call allocates only its output, and the first call on a new object
  queues the plan's upload (pinned, asynchronous) without waiting for the stream.
  Metadata objects are treated as immutable here, as the reference's frozen dataclass
  is: an object whose device tensors are rewritten in place must be replayed through a
  captured graph.  The kernel checks every item against the live prefix lengths and
  node counts, so a plan that an in-place change outgrew sets TV_STATUS_STALE_PLAN
  (read_and_clear_status) instead of passing silently.
* Captured (torch.cuda.is_current_stream_capturing()).  The reference's
  PackedTargetGraph (target_graph.py:55-167) captures the forward once against a
  staged metadata object and replays it after copy_-ing each round's metadata into
  that object; its kernels read prefix lengths and node counts from device memory
  (paged_backend.py:138).  So under capture this wrapper plans on the device too:
  the first call of a capture on a metadata object enqueues the ancestor words
  (from the live qq_bias) and the device planner (from the live prefix_lens and
  node_counts), sized for every batch of the graph signature (request count,
  packed rows, qq_bias elements); each call then launches the attention and merge
  kernels on capacity grids that read the live counts.  Replays therefore follow
  the staged metadata.  The capture-mode buffers belong to the metadata object,
  which must outlive the graphs that captured it (PackedTargetGraph keeps it in the
  graph entry), and graphs sharing one metadata object must not replay concurrently.
"""
from __future__ import annotations

import ctypes
import threading
import weakref

import numpy as np
import torch

from . import _device, _lib

_BACKENDS = ("auto", "reference", "prefix", "gqa")
# Query heads per KV head the MFMA kernel is built for (the reference's grouped kernel takes
# powers of two up to 16, tree_gqa.py:124-126; 3, 5, 6 and 7 are the GQA ratios of other
# Qwen-family checkpoints, e.g. 40 query over 8 KV heads).  Other ratios run the FP32 kernel.
SUPPORTED_GROUPS = (1, 2, 3, 4, 5, 6, 7, 8, 16)
# Head sizes 64 and 256 run the MFMA kernel for the power-of-two groups of the reference's grouped
# kernel (tree_gqa.py:124-135).
SUPPORTED_GROUPS_D64 = (1, 2, 4, 8, 16)
SUPPORTED_GROUPS_D256 = (1, 2, 4, 8, 16)


def mfma_head(head_size: int, groups: int) -> bool:
    """Head size and query group the MFMA kernel is built for."""
    return ((head_size == 128 and groups in SUPPORTED_GROUPS) or (head_size == 64 and groups in SUPPORTED_GROUPS_D64)
            or (head_size == 256 and groups in SUPPORTED_GROUPS_D256))


def workspace_bytes(plan_bytes: int, partial_slots: int, head_dim: int) -> int:
    """Split-prefix workspace of a plan at this head size (a plan's own figure holds up to 128)."""
    if not partial_slots:
        return int(plan_bytes)
    return max(int(plan_bytes), int(_lib.library().tv_tree_attention_workspace_bytes(partial_slots, head_dim)))


_FP32_ROUTE = "fp32"     # cache entries of batches that run the FP32 kernel
_derived: dict[int, dict] = {}
_derived_lock = threading.Lock()


def _validate(q, k_pool, v_pool, metadata, groups, output_dtype) -> torch.dtype:
    """Geometry/device/dtype checks of tree_attention.py:21-37; returns the output dtype."""
    if q.ndim != 3 or q.shape[0] != metadata.total_queries:
        raise ValueError("packed queries do not match the metadata")
    if k_pool.ndim != 4 or k_pool.shape != v_pool.shape or k_pool.shape[1] != metadata.block_size:
        raise ValueError("packed K/V page geometry does not match metadata")
    if (not q.is_cuda or q.device != k_pool.device or q.device != v_pool.device
            or q.device != metadata.tree_slots.device):
        raise ValueError("packed attention requires CUDA queries, KV and metadata on one device")
    if q.stride(-1) != 1 or k_pool.shape[-1] != q.shape[-1]:
        raise ValueError("unsupported packed query/KV head geometry")
    if isinstance(groups, bool) or not isinstance(groups, int) or groups <= 0 or q.shape[1] != k_pool.shape[2] * groups:
        raise ValueError("invalid packed GQA head grouping")
    if q.dtype != k_pool.dtype or k_pool.dtype != v_pool.dtype or q.dtype not in (
            torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("packed Q/K/V must use one supported floating dtype")
    dtype = q.dtype if output_dtype is None else output_dtype
    if dtype not in (q.dtype, torch.float32):
        raise ValueError("output dtype must match input or be FP32 for qualification")
    if q.shape[-1] > 512:
        raise ValueError("the MI355X tree-attention kernels take head sizes up to 512")
    return dtype


def _aligned_rows(t: torch.Tensor) -> bool:
    """16-byte aligned base and row/page/head strides (the MFMA kernel's 16-byte loads)."""
    return t.data_ptr() % 16 == 0 and all(t.stride(i) % 8 == 0 for i in range(t.ndim - 1))


# Tree nodes per request the MFMA kernel takes with page-table prefixes (its work items
# cache the tree's scratch slots in LDS; csrc/tv_attention.h kMaxTreeNodes), and beside the
# legacy entry's slot-addressed prefixes (kMaxTreeSlots).
MFMA_MAX_TREE_NODES = 2048
MFMA_MAX_TREE_NODES_SLOTS = 1024


def _mfma_geometry(q, k_pool, v_pool, metadata) -> bool:
    """True when the MFMA kernel (tv_tree_attention) takes this batch; the others run the
    FP32 kernel.  Mirrors the MFMA entry's limits (csrc/tv_attention.hip)."""
    if q.dtype not in (torch.bfloat16, torch.float16):
        return False
    kv_heads = int(k_pool.shape[2])
    if q.shape[1] % kv_heads or not mfma_head(int(q.shape[-1]), q.shape[1] // kv_heads):
        return False
    if metadata.block_size % 32 or max(metadata.node_counts_host, default=0) > MFMA_MAX_TREE_NODES:
        return False
    if k_pool.stride(3) != 1 or v_pool.stride(3) != 1 or not _aligned_rows(k_pool) or not _aligned_rows(v_pool):
        return False
    # 32-bit page, head and 32-key-tile byte offsets.
    return all(0 <= t.stride(0) * 2 < (1 << 32) and 0 <= t.stride(1) * 64 < (1 << 31)
               and 0 <= t.stride(2) * 2 < (1 << 31) for t in (k_pool, v_pool)) and (
        int(k_pool.shape[0]) * metadata.block_size < (1 << 31))


def _fp32_template(metadata, k_pool, v_pool, queries_per_kv: int, device):
    """Filled FP32-kernel argument block of one (metadata, K/V pool): all but Q, O and scale."""
    a = _lib.TreeAttentionFp32Args()
    a.k_pool, a.v_pool = k_pool.data_ptr(), v_pool.data_ptr()
    for i in range(4):
        a.k_stride[i] = k_pool.stride(i)
        a.v_stride[i] = v_pool.stride(i)
    a.num_blocks = int(k_pool.shape[0])
    a.in_dtype = _device.dtype_code(k_pool.dtype)
    a.cu_seqlens_q = metadata.cu_seqlens_q.data_ptr()
    a.query_to_request = metadata.query_to_request.data_ptr()
    a.query_local_row = metadata.query_local_row.data_ptr()
    a.prefix_lens = metadata.prefix_lens.data_ptr()
    a.node_counts = metadata.node_counts.data_ptr()
    a.block_tables = metadata.block_tables.data_ptr()
    a.block_table_stride = metadata.block_tables.stride(0)
    a.tree_slots = metadata.tree_slots.data_ptr()
    a.qq_bias = metadata.qq_bias.data_ptr()
    a.qq_bias_offsets = metadata.qq_bias_offsets.data_ptr()
    a.num_requests = metadata.num_requests
    a.total_queries = metadata.total_queries
    a.num_kv_heads = int(k_pool.shape[2])
    a.num_q_heads = queries_per_kv * a.num_kv_heads
    a.head_dim = int(k_pool.shape[3])
    a.block_size = metadata.block_size
    a.status = _device.status_word(device).data_ptr()
    return a


def _launch_fp32(a, q, out, scale, stream: int) -> torch.Tensor:
    """Complete a copy of an FP32-kernel argument block with Q, O and scale, and launch."""
    a = _lib.TreeAttentionFp32Args.from_buffer_copy(a)
    if q.stride(-1) != 1 or out.stride(-1) != 1:
        raise ValueError("unsupported packed query/KV head geometry")
    a.q = q.data_ptr()
    a.q_stride_row, a.q_stride_head = q.stride(0), q.stride(1)
    a.out = out.data_ptr()
    a.out_stride_row, a.out_stride_head = out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.scale = float(scale)
    _lib.check(_lib.library().tv_tree_attention_fp32(ctypes.byref(a), stream), "tree_attention_fp32")
    return out


_METADATA_LAYOUT = (
    ("cu_seqlens_q", torch.int32), ("query_to_request", torch.int32), ("query_local_row", torch.int32),
    ("prefix_lens", torch.int32), ("tree_slots", torch.int64), ("qq_bias", torch.float32),
    ("qq_bias_offsets", torch.int64), ("node_counts", torch.int32),
)


def _check_metadata_buffers(metadata) -> None:
    """The kernel reads these buffers raw: dtypes, 1-D contiguity and sizes must hold."""
    r, q = metadata.num_requests, metadata.total_queries
    sizes = {"cu_seqlens_q": r + 1, "query_to_request": q, "query_local_row": q, "prefix_lens": r,
             "tree_slots": q, "qq_bias_offsets": r + 1, "node_counts": r,
             "qq_bias": sum(n * n for n in metadata.node_counts_host)}
    for name, dtype in _METADATA_LAYOUT:
        t = getattr(metadata, name)
        if t.dtype != dtype or t.ndim != 1 or not t.is_contiguous() or t.numel() != sizes[name]:
            raise ValueError(f"metadata.{name} must be a contiguous {dtype} vector of {sizes[name]} entries")
    tables = metadata.block_tables
    width = max(1, max(len(t) for t in metadata.block_tables_host))
    if (tables.dtype != torch.int32 or tables.ndim != 2 or tables.shape[0] != r or tables.shape[1] < width
            or tables.stride(1) != 1):
        raise ValueError("metadata.block_tables must be int32 [requests, pages] with unit column stride")


def _release(key: int) -> None:
    with _derived_lock:
        _derived.pop(key, None)


def _per_metadata(metadata) -> dict:
    """The derived-state dictionary of one metadata object (dropped with the object)."""
    key = id(metadata)
    per_meta = _derived.get(key)
    if per_meta is not None:
        return per_meta
    _check_metadata_buffers(metadata)
    with _derived_lock:
        per_meta = _derived.get(key)
        if per_meta is None:
            per_meta = _derived[key] = {}
            weakref.finalize(metadata, _release, key)
    return per_meta


def derived_state(metadata, num_kv_heads: int, *, queries_per_kv: int, chunk_keys: int = 0) -> dict:
    """Work plan and ancestor bits of `metadata` for one head geometry, built once per object."""
    per_meta = _per_metadata(metadata)
    lib = _lib.library()
    device = metadata.tree_slots.device
    words = per_meta.get("ancestor_words")
    prebuilt = getattr(metadata, "ancestor_words", None)
    if words is None and prebuilt is not None:
        per_meta["ancestor_words"] = words = prebuilt
        per_meta["words_per_row"] = int(prebuilt.shape[1])
    if words is None:
        count = max(metadata.node_counts_host)
        per_row = (count + 63) // 64
        total = metadata.total_queries
        words = torch.empty((max(total, 1), per_row), dtype=torch.int64, device=device)
        status = _device.status_word(device)
        _lib.check(lib.tv_pack_ancestor_words(
            metadata.qq_bias.data_ptr(), metadata.qq_bias_offsets.data_ptr(),
            metadata.query_to_request.data_ptr(), metadata.query_local_row.data_ptr(),
            metadata.node_counts.data_ptr(), total, metadata.num_requests, per_row,
            words.data_ptr(), status.data_ptr(), _device.stream_handle(device)), "pack_ancestor_words")
        per_meta["ancestor_words"] = words
        per_meta["words_per_row"] = per_row
    plan_key = ("plan", int(num_kv_heads), int(queries_per_kv), int(chunk_keys))
    plan = per_meta.get(plan_key)
    if plan is None:
        plan = make_plan(metadata.prefix_lengths, metadata.node_counts_host, num_kv_heads, metadata.block_size,
                         _device.compute_units(device.index), chunk_keys, queries_per_kv=queries_per_kv)
        # One pinned staging buffer and an asynchronous copy: the serving loop builds a new
        # metadata object every round, and a pageable copy here would wait for every kernel
        # already queued on the stream before the round's first attention could be enqueued.
        staged = _device.upload_fields({"items": plan["items"], "groups": plan["groups"][:plan["num_groups"]]}, device,
                         pinned=True)
        plan["items_dev"] = staged["items"]
        plan["groups_dev"] = staged["groups"] if plan["num_groups"] else None
        per_meta[plan_key] = plan
    return {"ancestor_words": per_meta["ancestor_words"], "words_per_row": per_meta["words_per_row"], **plan}


def make_plan(prefix_lengths, node_counts, num_kv_heads: int, block_size: int, compute_units: int,
              chunk_keys: int = 0, *, queries_per_kv: int) -> dict:
    """Host work plan from tv_tree_attention_plan (items/groups as int32 [n, 8])."""
    lib = _lib.library()
    count = len(prefix_lengths)
    prefixes = (ctypes.c_int32 * count)(*prefix_lengths)
    nodes = (ctypes.c_int32 * count)(*node_counts)
    info = _lib.PlanInfo()
    _lib.check(lib.tv_tree_attention_plan(prefixes, nodes, count, num_kv_heads, queries_per_kv, block_size,
                                          compute_units, chunk_keys, None, None, ctypes.byref(info)),
               "tree_attention_plan")
    items = np.zeros((max(info.num_items, 1), 8), dtype=np.int32)
    groups = np.zeros((max(info.num_groups, 1), 8), dtype=np.int32)
    _lib.check(lib.tv_tree_attention_plan(
        prefixes, nodes, count, num_kv_heads, queries_per_kv, block_size, compute_units, chunk_keys,
        items.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), groups.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
        ctypes.byref(info)), "tree_attention_plan")
    return {"items": items[:info.num_items], "groups": groups[:info.num_groups],
            "num_items": info.num_items, "num_groups": info.num_groups,
            "num_partial_slots": info.num_partial_slots, "workspace_bytes": int(info.workspace_bytes)}


def fill_pool_args(a, metadata, k_pool, v_pool, num_kv_heads: int, queries_per_kv: int, status) -> None:
    """The metadata, K/V pool and geometry fields of a tv_tree_attention_args block."""
    a.k_pool, a.v_pool = k_pool.data_ptr(), v_pool.data_ptr()
    for i in range(4):
        a.k_stride[i] = k_pool.stride(i)
        a.v_stride[i] = v_pool.stride(i)
    a.num_blocks = int(k_pool.shape[0])
    a.in_dtype = _device.dtype_code(k_pool.dtype)
    a.cu_seqlens_q = metadata.cu_seqlens_q.data_ptr()
    a.prefix_lens = metadata.prefix_lens.data_ptr()
    a.node_counts = metadata.node_counts.data_ptr()
    a.block_tables = metadata.block_tables.data_ptr()
    a.block_table_stride = metadata.block_tables.stride(0)
    a.tree_slots = metadata.tree_slots.data_ptr()
    a.num_requests = metadata.num_requests
    a.total_queries = metadata.total_queries
    a.num_q_heads = queries_per_kv * num_kv_heads
    a.num_kv_heads = num_kv_heads
    a.head_dim = int(k_pool.shape[3])
    a.block_size = metadata.block_size
    a.status = status.data_ptr()


def _eager_template(per_meta, metadata, k_pool, v_pool, num_kv_heads: int, queries_per_kv: int, chunk_keys: int,
                    stream: int):
    """Filled argument block of one (metadata, K/V pool, stream): everything but Q, O and scale."""
    state = derived_state(metadata, num_kv_heads, queries_per_kv=queries_per_kv, chunk_keys=chunk_keys)
    device = k_pool.device
    workspace = None
    ws_bytes = workspace_bytes(state["workspace_bytes"], state["num_partial_slots"], int(k_pool.shape[3]))
    if ws_bytes:
        # One workspace per plan and stream: launches on one stream run in order, so the
        # per-layer launches of a round reuse it (each merge finishes before the next
        # layer's attention writes its partials).
        ws_key = ("workspace", num_kv_heads, queries_per_kv, chunk_keys, stream, ws_bytes)
        workspace = per_meta.get(ws_key)
        if workspace is None:
            workspace = per_meta[ws_key] = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    a = _lib.TreeAttentionArgs()
    fill_pool_args(a, metadata, k_pool, v_pool, num_kv_heads, queries_per_kv, _device.status_word(device))
    a.ancestor_words = state["ancestor_words"].data_ptr()
    a.ancestor_words_per_row = state["words_per_row"]
    a.items = state["items_dev"].data_ptr()
    a.num_items = state["num_items"]
    a.groups = state["groups_dev"].data_ptr() if state["groups_dev"] is not None else None
    a.num_groups = state["num_groups"]
    a.num_partial_slots = state["num_partial_slots"]
    a.workspace = workspace.data_ptr() if workspace is not None else None
    a.workspace_bytes = ws_bytes
    a.device_counts = None
    # Keep every buffer the block points at alive as long as the block.
    return a, (state["ancestor_words"], state["items_dev"], state["groups_dev"], workspace)


def _capture_id(stream: int) -> int:
    capturing = ctypes.c_int32()
    ident = ctypes.c_uint64()
    lib = _lib.library()
    _lib.check(lib.tv_stream_capture_info(stream, ctypes.byref(capturing), ctypes.byref(ident)),
               "stream_capture_info")
    if capturing.value != 1:
        raise RuntimeError("tree attention: the stream's graph capture is not active")
    return int(ident.value)


def _launch_captured(q, k_pool, v_pool, metadata, scale, out, num_kv_heads: int, queries_per_kv: int,
                     chunk_keys: int, stream: int, exact: bool) -> torch.Tensor:
    """Graph-capturable launch that follows the live device metadata on every replay."""
    from .target_graph import GraphedTreeAttention

    per_meta = _per_metadata(metadata)
    head_dim = int(k_pool.shape[3])
    key = ("graph", num_kv_heads, queries_per_kv, chunk_keys, head_dim)
    graphed = per_meta.get(key)
    if graphed is None:
        graphed = per_meta[key] = GraphedTreeAttention.for_signature(
            metadata, num_kv_heads, queries_per_kv=queries_per_kv, chunk_keys=chunk_keys, head_dim=head_dim)
    capture = _capture_id(stream)
    if graphed.prepared_capture != capture:
        graphed.prepare(metadata)   # recorded once at the head of this graph's sequence
        graphed.prepared_capture = capture
    return graphed(q, k_pool, v_pool, metadata, scale, out, prepared=True, exact=exact)


def _launch(q, k_pool, v_pool, metadata, scale, out, *, chunk_keys: int = 0, exact: bool = False) -> torch.Tensor:
    """Enqueue the attention of `metadata` into `out`.  exact=True keeps every probability
    to ~2^-17 relative in the P.V product (the reference's FP32 entries); otherwise it is
    rounded to the operand type once (the reference's grouped bf16-P kernel).  Batches
    outside the MFMA kernel's geometry run the FP32 kernel (fp32 probabilities)."""
    num_kv_heads = int(k_pool.shape[2])
    queries_per_kv = int(q.shape[1]) // num_kv_heads
    stream = torch.cuda.current_stream(q.device).cuda_stream
    per_meta = _derived.get(id(metadata))
    if per_meta is None:
        per_meta = _per_metadata(metadata)
    key = (num_kv_heads, queries_per_kv, chunk_keys, k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(),
           v_pool.stride(), tuple(k_pool.shape), k_pool.dtype, stream)
    entry = per_meta.get(key)
    if entry is None:
        if not _mfma_geometry(q, k_pool, v_pool, metadata):
            entry = per_meta[key] = (_FP32_ROUTE, _fp32_template(metadata, k_pool, v_pool, queries_per_kv, q.device))
        elif torch.cuda.is_current_stream_capturing():
            entry = None
        else:
            entry = per_meta[key] = _eager_template(per_meta, metadata, k_pool, v_pool, num_kv_heads,
                                                    queries_per_kv, chunk_keys, stream)
    if entry is not None and entry[0] is _FP32_ROUTE:
        return _launch_fp32(entry[1], q, out, scale, stream)
    if q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    if torch.cuda.is_current_stream_capturing():
        return _launch_captured(q, k_pool, v_pool, metadata, scale, out, num_kv_heads, queries_per_kv, chunk_keys,
                                stream, exact)
    a = _lib.TreeAttentionArgs.from_buffer_copy(entry[0])
    a.q = q.data_ptr()
    a.q_stride_row, a.q_stride_head = q.stride(0), q.stride(1)
    a.out = out.data_ptr()
    a.out_stride_row, a.out_stride_head = out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.scale = scale
    a.exact_probabilities = 1 if exact else 0
    _lib.check(_lib.library().tv_tree_attention(ctypes.byref(a), stream), "tree_attention")
    return out


def _launch_new(q, k_pool, v_pool, metadata, scale, dtype, *, exact: bool) -> torch.Tensor:
    """Launch into a new output of `dtype` (the checked entries' allocation, tree_attention.py:36)."""
    return _launch(q, k_pool, v_pool, metadata, scale, torch.empty(q.shape, dtype=dtype, device=q.device),
                   exact=exact)


def packed_tree_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, metadata, scale: float,
                          num_queries_per_kv: int, *, backend: str = "auto",
                          output_dtype: torch.dtype | None = None, chunk_keys: int = 0) -> torch.Tensor:
    """One ragged launch with independent request/ancestor visibility (paged_backend.py:240-306).

    ``backend`` takes the reference's names and dispatches to the same-named entries
    (tree_gqa, tree_attention, tree_prefix modules of this package), as the reference
    does; every entry runs the one HIP kernel.  ``chunk_keys`` (extension, default
    automatic) fixes the prefix split length.
    """
    if backend not in _BACKENDS:
        raise ValueError("tree attention backend must be auto, reference, prefix or gqa")
    if output_dtype not in (None, q.dtype, torch.float32):
        raise ValueError("output dtype must match input or be FP32 for qualification")
    if backend == "gqa":
        from .tree_gqa import packed_tree_attention_gqa
        return packed_tree_attention_gqa(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                         output_dtype=output_dtype)
    if backend == "reference":
        from .tree_attention import packed_tree_attention_reference
        return packed_tree_attention_reference(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                               output_dtype=output_dtype)
    if backend == "prefix":
        from .tree_prefix import packed_tree_attention_prefix_split_exact
        return packed_tree_attention_prefix_split_exact(q, k_pool, v_pool, metadata, scale, num_queries_per_kv,
                                                        output_dtype=output_dtype, num_warps=4)
    dtype = _validate(q, k_pool, v_pool, metadata, num_queries_per_kv, output_dtype)
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    return _launch(q, k_pool, v_pool, metadata, scale, out, chunk_keys=chunk_keys)


def paged_tree_attention(q, k_pool, v_pool, block_table, cu_seqlens_q, seq_lens_k, qq_bias, scale,
                         num_queries_per_kv, block_size, logical_kv_slots=None, logical_kv_starts=None,
                         logical_kv_lens=None):
    """Legacy single-request entry (paged_backend.py:309-415), as the legacy c1 path calls it
    (models/qwen3.py:270-302): one request whose keys are named by a logical slot vector,
    ``logical_kv_slots[0, pos]`` for pos < seq_len (the committed prefix, then the T tree
    nodes), over a pool viewed as ``block_size``-token pages (16 in the c1 path), and a
    request-local ``qq_bias[T, T]``.  A key at position pos is visible to tree row i iff
    pos <= P + i; a tree key's bias is added to its score (paged_backend.py:82-91).

    With a 0 / -inf bias (what the reference's runners build) and the MFMA kernel's
    geometry, the MFMA kernel runs in slot-addressed mode with FP32 probabilities (the
    legacy kernel is the frozen FP32 one, paged_backend.py:20-113); anything else (finite
    bias values, f32 operands, other head sizes or query groups, trees above 1024 nodes beside
    the slot-addressed prefix)
    runs the FP32 kernel.  Like the reference, it reads the sequence length from the
    device (one synchronisation).  Multi-request calls are rejected exactly as in the
    reference; the block-table form without logical slots or bias runs the external
    jetspec kernel in the reference (paged_backend.py:362-363), which is not part of
    this build, and is rejected too.
    """
    num_seqs = int(seq_lens_k.shape[0])
    if num_seqs != 1:
        raise ValueError("multi-request tree verification requires explicit PackedTreeMetadata")
    if logical_kv_slots is None or qq_bias is None:
        raise ValueError("block-table tree attention (the external jetspec kernel) is not part of the MI355X "
                         "build; pass logical_kv_slots and qq_bias, or build PackedTreeMetadata")
    if q.ndim != 3 or k_pool.ndim != 4 or k_pool.shape != v_pool.shape:
        raise ValueError("unsupported packed query/KV head geometry")
    total_q, num_query_heads, head_size = q.shape
    device = _device.require_gpu(q, k_pool, v_pool, logical_kv_slots, qq_bias, seq_lens_k,
                                 what="paged_tree_attention")
    if (q.stride(-1) != 1 or k_pool.shape[3] != head_size or int(k_pool.shape[1]) != int(block_size)
            or isinstance(num_queries_per_kv, bool) or num_queries_per_kv <= 0
            or num_query_heads != k_pool.shape[2] * num_queries_per_kv):
        raise ValueError("unsupported packed query/KV head geometry")
    if (q.dtype not in (torch.bfloat16, torch.float16, torch.float32) or k_pool.dtype != q.dtype
            or v_pool.dtype != q.dtype):
        raise ValueError("packed Q/K/V must use one supported floating dtype")
    if head_size > 512:
        raise ValueError("the MI355X tree-attention kernels take head sizes up to 512")
    if logical_kv_slots.dtype not in (torch.int32, torch.int64):
        raise ValueError("logical KV slots must be int32 or int64")
    if qq_bias.ndim != 2 or qq_bias.shape[0] < total_q or qq_bias.shape[1] < total_q:
        raise ValueError("qq_bias must be a [tree nodes, tree nodes] matrix")
    seq_len = int(seq_lens_k[0].item())
    prefix = seq_len - total_q
    slots = logical_kv_slots.reshape(-1)
    if prefix < 0 or slots.numel() < seq_len or total_q < 1:
        raise ValueError("logical KV slots must cover the prefix and every tree node")
    if not slots.is_contiguous():
        slots = slots.contiguous()
    bias = torch.as_strided(qq_bias, (total_q, total_q), (qq_bias.stride(0), qq_bias.stride(1))).to(
        torch.float32).contiguous().view(-1)
    i32 = dict(dtype=torch.int32, device=device)
    request = _LegacyRequest(
        cu=torch.tensor([0, total_q], **i32), counts=torch.tensor([total_q], **i32),
        rows_local=torch.arange(total_q, **i32), requests=torch.zeros(total_q, **i32),
        bias=bias, bias_offsets=torch.tensor([0, total_q * total_q], dtype=torch.int64, device=device),
        tree_slots=slots[prefix:prefix + total_q].to(torch.int64), prefix_lens=torch.tensor([prefix], **i32),
        table=torch.full((1, 1), -1, **i32), slots=slots, prefix=prefix, total_q=total_q)
    out = torch.empty_like(q)
    # The MFMA kernel reads tree visibility as bits, so a bias other than 0 / -inf (which
    # is added to the score) takes the FP32 kernel.
    mask_bias = bool(((bias == 0) | (bias == float("-inf"))).all())
    geometry = (q.dtype != torch.float32 and mfma_head(head_size, num_queries_per_kv)
                and total_q <= MFMA_MAX_TREE_NODES_SLOTS and k_pool.stride(3) == 1 and v_pool.stride(3) == 1
                and _aligned_rows(k_pool) and _aligned_rows(v_pool)
                and int(k_pool.shape[0]) * int(block_size) < (1 << 31))
    if mask_bias and geometry:
        _legacy_mfma(q, k_pool, v_pool, request, scale, num_queries_per_kv, int(block_size), out, device)
    else:
        _legacy_fp32(q, k_pool, v_pool, request, scale, int(block_size), out, device)
    return out


class _LegacyRequest:
    """Device metadata of the legacy entry's one request (kept alive until the launch returns)."""

    def __init__(self, **fields):
        self.__dict__.update(fields)


def _legacy_fp32(q, k_pool, v_pool, req, scale, block_size: int, out, device) -> None:
    a = _lib.TreeAttentionFp32Args()
    a.q = q.data_ptr()
    a.q_stride_row, a.q_stride_head = q.stride(0), q.stride(1)
    a.k_pool, a.v_pool = k_pool.data_ptr(), v_pool.data_ptr()
    for i in range(4):
        a.k_stride[i] = k_pool.stride(i)
        a.v_stride[i] = v_pool.stride(i)
    a.num_blocks = int(k_pool.shape[0])
    a.in_dtype = _device.dtype_code(q.dtype)
    a.out = out.data_ptr()
    a.out_stride_row, a.out_stride_head = out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.cu_seqlens_q = req.cu.data_ptr()
    a.query_to_request = req.requests.data_ptr()
    a.query_local_row = req.rows_local.data_ptr()
    a.prefix_lens = req.prefix_lens.data_ptr()
    a.node_counts = req.counts.data_ptr()
    a.block_tables = req.table.data_ptr()
    a.block_table_stride = 1
    a.tree_slots = req.tree_slots.data_ptr()
    a.qq_bias = req.bias.data_ptr()
    a.qq_bias_offsets = req.bias_offsets.data_ptr()
    a.prefix_slots = req.slots.data_ptr()
    a.prefix_slots_stride = 0
    a.prefix_slots_is_int64 = 1 if req.slots.dtype == torch.int64 else 0
    a.num_requests = 1
    a.total_queries = req.total_q
    a.num_q_heads = int(q.shape[1])
    a.num_kv_heads = int(k_pool.shape[2])
    a.head_dim = int(q.shape[2])
    a.block_size = block_size
    a.scale = float(scale)
    a.status = _device.status_word(device).data_ptr()
    _lib.check(_lib.library().tv_tree_attention_fp32(ctypes.byref(a), _device.stream_handle(device)),
               "tree_attention_fp32 (slot addressed)")


def _legacy_mfma(q, k_pool, v_pool, req, scale, num_queries_per_kv: int, block_size: int, out, device) -> None:
    lib = _lib.library()
    total_q, prefix = req.total_q, req.prefix
    num_kv_heads = int(k_pool.shape[2])
    stream = _device.stream_handle(device)
    status = _device.status_word(device)
    per_row = (total_q + 63) // 64
    words = torch.empty((total_q, per_row), dtype=torch.int64, device=device)
    _lib.check(lib.tv_pack_ancestor_words(req.bias.data_ptr(), req.bias_offsets.data_ptr(), req.requests.data_ptr(),
                                          req.rows_local.data_ptr(), req.counts.data_ptr(), total_q, 1, per_row,
                                          words.data_ptr(), status.data_ptr(), stream), "pack_ancestor_words")
    info = _lib.PlanInfo()
    prefixes_host = (ctypes.c_int32 * 1)(prefix)
    nodes_host = (ctypes.c_int32 * 1)(total_q)
    cus = _device.compute_units(device.index if device.index is not None else torch.cuda.current_device())
    _lib.check(lib.tv_tree_attention_plan_slots(prefixes_host, nodes_host, 1, num_kv_heads, num_queries_per_kv, cus,
                                                0, None, None, ctypes.byref(info)), "tree_attention_plan_slots")
    items = np.zeros((max(info.num_items, 1), 8), dtype=np.int32)
    groups = np.zeros((max(info.num_groups, 1), 8), dtype=np.int32)
    _lib.check(lib.tv_tree_attention_plan_slots(
        prefixes_host, nodes_host, 1, num_kv_heads, num_queries_per_kv, cus, 0,
        items.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), groups.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
        ctypes.byref(info)), "tree_attention_plan_slots")
    # Pinned and asynchronous, as the packed path's plan: no wait on the stream's queued work.
    staged = _device.upload_fields({"items": items, "groups": groups}, device, pinned=True)
    items_dev, groups_dev = staged["items"], staged["groups"]
    ws_bytes = workspace_bytes(info.workspace_bytes, info.num_partial_slots, int(q.shape[2]))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    if q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    a = _lib.TreeAttentionArgs()
    a.q = q.data_ptr()
    a.q_stride_row, a.q_stride_head = q.stride(0), q.stride(1)
    a.k_pool, a.v_pool = k_pool.data_ptr(), v_pool.data_ptr()
    for i in range(4):
        a.k_stride[i] = k_pool.stride(i)
        a.v_stride[i] = v_pool.stride(i)
    a.num_blocks = int(k_pool.shape[0])
    a.in_dtype = _device.dtype_code(q.dtype)
    a.out = out.data_ptr()
    a.out_stride_row, a.out_stride_head = out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.cu_seqlens_q = req.cu.data_ptr()
    a.prefix_lens = req.prefix_lens.data_ptr()
    a.node_counts = req.counts.data_ptr()
    a.block_tables = req.table.data_ptr()
    a.block_table_stride = 1
    a.tree_slots = req.tree_slots.data_ptr()
    a.ancestor_words = words.data_ptr()
    a.ancestor_words_per_row = per_row
    a.num_requests = 1
    a.total_queries = total_q
    a.num_q_heads = int(q.shape[1])
    a.num_kv_heads = num_kv_heads
    a.head_dim = int(q.shape[2])
    a.block_size = block_size
    a.scale = float(scale)
    a.items = items_dev.data_ptr()
    a.num_items = info.num_items
    a.groups = groups_dev.data_ptr() if info.num_groups else None
    a.num_groups = info.num_groups
    a.num_partial_slots = info.num_partial_slots
    a.workspace = workspace.data_ptr() if ws_bytes else None
    a.workspace_bytes = ws_bytes
    a.status = status.data_ptr()
    a.prefix_slots = req.slots.data_ptr()
    a.prefix_slots_stride = 0
    a.prefix_slots_is_int64 = 1 if req.slots.dtype == torch.int64 else 0
    a.exact_probabilities = 1
    _lib.check(lib.tv_tree_attention(ctypes.byref(a), stream), "tree_attention (slot addressed)")
