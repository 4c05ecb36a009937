"""CPU oracle of the tree-verify hot path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker (or the timed CPU baseline); the product in
nano-vllm-jetspec_amd/ never does.

Contents (each restates the cited reference code):
  tree_attention_f64    paged_backend.py:116-213 (C, double precision)
  store_kvcache         layers/attention.py:15-45 (C, byte copy)
  copy_accepted_kv      speculative/jetspec/state.py:64-86 (C, gather then scatter)
  commit_slots          speculative/jetspec/state.py:54-61 and :757-785 (numpy, per request)
  parent_chain          benchmarks/jetspec_numeric_oracles.py:24-58
  fp64_attention        benchmarks/jetspec_numeric_oracles.py:72-105
  mask_from_parents     benchmarks/jetspec_tree_kernel_qualification.py:102-107
  metadata_arrays       speculative/jetspec/packed_metadata.py:36-126 (host arrays)
  accept_walk           speculative/jetspec/serving_ops.py:55-90
  truncate_accepted     speculative/jetspec/batch_runtime.py:636-655 (per request)
  argmax_flip_witness   benchmarks/jetspec_numeric_oracles.py:171-217
  numerical_metrics     benchmarks/jetspec_numeric_oracles.py:108-168 (max-abs, rel-RMS,
                        the fixed FP32 bound and the bf16-ULP diagnostics)
  rope_scatter_hf       speculative/jetspec/tree_fusion.py:20-82 and the eager HF RoPE
                        + scatter it replaces, models/qwen3.py:241-258 (numpy, exact
                        bf16 round-to-nearest-even on uint16 bit patterns)

Pinning: tests/test_oracle_pins.py checks every function above against the
reference's own known-answer tests (transcribed into tests/golden/reference_kats.json),
closed forms and an independent brute force; see the header of that file.
rope_scatter_hf is pinned against torch's eager CPU bf16/fp32 arithmetic, which is the
expected value of the reference's own test (tests/test_jetspec_tree_fusion.py:21-32),
and against the reference's rounding witness (:117-126).

Parity unpinned: accept_walk's equivalence with the un-vendored jetspec dependency's
gpu_tree_accept (pyproject.toml:27-29) beyond the reference's duplicate-sibling KAT and
the depth-cap closed form; that package is not installed and cannot be fetched here.
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_int32, c_int64, c_void_p
import math
from pathlib import Path
import subprocess
import threading

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"
_lock = threading.Lock()
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def library() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            if not LIBRARY.exists():
                build()
            lib = ctypes.CDLL(str(LIBRARY))
            lib.oracle_store_kvcache.restype = None
            lib.oracle_store_kvcache.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                                 c_void_p, c_int64, c_int64]
            lib.oracle_copy_accepted_kv.restype = c_int64
            lib.oracle_copy_accepted_kv.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                                    c_void_p, c_int64, c_void_p]
            lib.oracle_tree_attention.restype = c_int32
            lib.oracle_tree_attention.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                                  c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                  c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                                  c_double, c_void_p, c_void_p]
            _lib = lib
    return _lib


def _ptr(array: np.ndarray) -> int:
    return array.ctypes.data


def _c(array, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(array), dtype=dtype)


# --------------------------------------------------------------------------- C restatements
def tree_attention_f64(q, k_pool, v_pool, *, cu_seqlens_q, query_to_request, query_local_row, prefix_lens,
                       block_tables, tree_slots, qq_bias, qq_bias_offsets, node_counts, scale,
                       rows=None) -> np.ndarray:
    """Double-precision packed tree attention (paged_backend.py:116-213).

    q [Q, Hq, D], k_pool/v_pool [N, B, Hkv, D] as float32 arrays (bf16 values convert
    exactly); metadata arrays as in PackedTreeMetadata.  `rows` optionally limits
    the rows computed (others are NaN).  Returns float64 [Q, Hq, D].
    """
    q = _c(q, np.float32)
    k = _c(k_pool, np.float32)
    v = _c(v_pool, np.float32)
    total_q, q_heads, head_dim = q.shape
    num_blocks, block_size, kv_heads, _ = k.shape
    tables = _c(block_tables, np.int32)
    if tables.ndim == 1:
        tables = tables.reshape(len(np.asarray(prefix_lens)), -1)
    select = None
    if rows is not None:
        select = np.zeros(total_q, dtype=np.uint8)
        select[np.asarray(list(rows), dtype=np.int64)] = 1
    out = np.full((total_q, q_heads, head_dim), np.nan, dtype=np.float64)
    arrays = [_c(cu_seqlens_q, np.int32), _c(query_to_request, np.int32), _c(query_local_row, np.int32),
              _c(prefix_lens, np.int32), tables, _c(tree_slots, np.int64), _c(qq_bias, np.float32),
              _c(qq_bias_offsets, np.int64), _c(node_counts, np.int32)]
    cu, q2r, local, plen, tables, slots, bias, boff, counts = arrays
    code = library().oracle_tree_attention(
        _ptr(q), _ptr(k), _ptr(v), num_blocks, block_size, q_heads, kv_heads, head_dim, _ptr(cu), _ptr(q2r),
        _ptr(local), _ptr(plen), _ptr(tables), tables.shape[1], _ptr(slots), _ptr(bias), _ptr(boff),
        _ptr(counts), total_q, float(scale), _ptr(select) if select is not None else None, _ptr(out))
    if code != 0:
        raise ValueError("oracle: a page or slot lies outside the pool")
    return out


def metadata_tree_attention_f64(q, k_pool, v_pool, metadata, scale, rows=None) -> np.ndarray:
    """tree_attention_f64 over a PackedTreeMetadata-like object (device tensors are copied)."""
    def host(t):
        return t.detach().float().cpu().numpy() if t.is_floating_point() else t.detach().cpu().numpy()
    return tree_attention_f64(
        host(q), host(k_pool), host(v_pool), cu_seqlens_q=host(metadata.cu_seqlens_q),
        query_to_request=host(metadata.query_to_request), query_local_row=host(metadata.query_local_row),
        prefix_lens=host(metadata.prefix_lens), block_tables=host(metadata.block_tables),
        tree_slots=host(metadata.tree_slots), qq_bias=host(metadata.qq_bias),
        qq_bias_offsets=host(metadata.qq_bias_offsets), node_counts=host(metadata.node_counts), scale=scale,
        rows=rows)


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping) -> None:
    """In-place byte copy of rows into cache slots (layers/attention.py:15-45)."""
    if not (k_cache.flags.c_contiguous and v_cache.flags.c_contiguous):
        raise ValueError("oracle caches must be contiguous")
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    rows = key.shape[0]
    row_bytes = key[0].nbytes if rows else 0
    slots = _c(slot_mapping, np.int64)
    library().oracle_store_kvcache(_ptr(key), row_bytes, _ptr(value), row_bytes, _ptr(k_cache), _ptr(v_cache),
                                   _ptr(slots), rows, row_bytes)


def copy_accepted_kv(pool: np.ndarray, source, destination) -> int:
    """In-place gather-then-scatter on a dense [2, L, N, B, H, D] pool (state.py:64-86)."""
    if not pool.flags.c_contiguous or pool.ndim != 6:
        raise ValueError("oracle pool must be a contiguous [2, L, N, B, H, D] array")
    src = _c(source, np.int64)
    dst = _c(destination, np.int64)
    if src.ndim != 1 or dst.ndim != 1 or src.size != dst.size:
        raise ValueError("slot maps must be equal-length vectors")
    row_bytes = pool.shape[4] * pool.shape[5] * pool.itemsize
    staging = np.empty(max(1, 2 * pool.shape[1] * src.size * row_bytes), dtype=np.uint8)
    return int(library().oracle_copy_accepted_kv(_ptr(pool), pool.shape[1], pool.shape[2], pool.shape[3],
                                                 row_bytes, _ptr(src), _ptr(dst), src.size, _ptr(staging)))


# --------------------------------------------------------------------------- Python restatements
def commit_slots(tree_slots, cu_seqlens, paths, path_offsets, block_tables, cache_lens, block_size: int,
                 num_blocks: int):
    """Commit source/destination slots of a batch, request by request (state.py:757-785).

    A request whose path the reference would reject (empty, not rooted at node 0,
    repeated or out-of-tree nodes, :770-773) or whose destinations leave its table row
    or the pool gets -1 on all of its rows; returns (source, destination, bad) with
    bad[r] True for such a request.
    """
    slots = np.asarray(tree_slots, dtype=np.int64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    path = np.asarray(paths, dtype=np.int64)
    offsets = np.asarray(path_offsets, dtype=np.int64)
    tables = np.asarray(block_tables, dtype=np.int64)
    lens = np.asarray(cache_lens, dtype=np.int64)
    source = np.full(path.size, -1, dtype=np.int64)
    destination = np.full(path.size, -1, dtype=np.int64)
    bad = np.zeros(lens.size, dtype=bool)
    for r in range(lens.size):
        indices = [int(x) for x in path[offsets[r]:offsets[r + 1]]]
        nodes = int(cu[r + 1] - cu[r])
        if (not indices or indices[0] != 0 or len(set(indices)) != len(indices) or min(indices) < 0
                or max(indices) >= nodes or lens[r] < 0):
            bad[r] = True
            continue
        positions = lens[r] + np.arange(len(indices))
        pages = positions // block_size
        if pages.max() >= tables.shape[1]:
            bad[r] = True
            continue
        owned = tables[r, pages]
        if owned.min() < 0 or owned.max() >= num_blocks:
            bad[r] = True
            continue
        source[offsets[r]:offsets[r + 1]] = slots[cu[r] + np.asarray(indices)]
        destination[offsets[r]:offsets[r + 1]] = owned * block_size + positions % block_size
    return source, destination, bad


def parent_chain(parents, chosen: int) -> list[int]:
    """Root-to-node indices by walking parents (jetspec_numeric_oracles.py:24-58)."""
    parents = [int(p) for p in parents]
    if not parents or not 0 <= chosen < len(parents):
        raise ValueError("chosen node is outside the tree")
    if parents[0] != -1:
        raise ValueError("root parent must be -1")
    chain, seen, node = [], set(), chosen
    while True:
        if not 0 <= node < len(parents):
            raise ValueError("parent index is outside the tree")
        if node in seen:
            raise ValueError("cycle in selected parent chain")
        seen.add(node)
        chain.append(node)
        if parents[node] == -1:
            if node != 0:
                raise ValueError("selected chain is disconnected from root 0")
            return chain[::-1]
        node = parents[node]


def fp64_attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float, groups: int) -> np.ndarray:
    """Unmasked attention of one query row over explicit visible keys (jetspec_numeric_oracles.py:72-105).

    q [Hq, D], keys/values [L, Hkv, D]; returns float64 [Hq, D].
    """
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    if q.ndim != 2 or keys.ndim != 3 or keys.shape != values.shape:
        raise ValueError("expected q[Hq,D] and equal K/V[L,Hkv,D]")
    if keys.shape[0] == 0 or keys.shape[1] == 0 or keys.shape[2] != q.shape[1]:
        raise ValueError("visible key sequence and head dimensions must be nonempty and agree")
    if groups < 1 or q.shape[0] != keys.shape[1] * groups:
        raise ValueError("invalid GQA head grouping")
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("attention scale must be finite and positive")
    if not (np.isfinite(q).all() and np.isfinite(keys).all() and np.isfinite(values).all()):
        raise ValueError("nonfinite valid operand")
    out = np.empty_like(q)
    for head in range(q.shape[0]):
        kv = head // groups
        scores = keys[:, kv] @ q[head] * scale
        scores = np.exp(scores - scores.max())
        out[head] = (scores / scores.sum()) @ values[:, kv]
    return out


def mask_from_parents(parents) -> np.ndarray:
    """Row i marks parent_chain(parents, i) (jetspec_tree_kernel_qualification.py:102-107)."""
    n = len(parents)
    mask = np.zeros((n, n), dtype=bool)
    for node in range(n):
        mask[node, parent_chain(parents, node)] = True
    return mask


def metadata_arrays(prefix_lens, block_tables, tree_slots, ancestor_masks, block_size) -> dict:
    """Host arrays of PackedTreeMetadata.build (packed_metadata.py:36-126), validation included."""
    prefixes = [int(p) for p in prefix_lens]
    count = len(prefixes)
    if count < 1 or not (len(block_tables) == len(tree_slots) == len(ancestor_masks) == count):
        raise ValueError("packed metadata requires equally sized nonempty request lists")
    if block_size <= 0 or any(p < 0 for p in prefixes):
        raise ValueError("invalid packed prefix length or page geometry")
    offsets, squares, q2r, local, bias, slots, tables = [0], [0], [], [], [], [], []
    for r, (prefix, table, node_slots, mask) in enumerate(zip(prefixes, block_tables, tree_slots, ancestor_masks)):
        table = [int(p) for p in table]
        if len(table) != -(-prefix // block_size) or len(set(table)) != len(table) or any(p < 0 for p in table):
            raise ValueError("prefix block table must be a tight canonical page table")
        mask = np.asarray(mask, dtype=bool)
        n = len(node_slots)
        if n < 1 or mask.shape != (n, n):
            raise ValueError("ancestor masks must be request-local boolean [nodes,nodes] matrices")
        if not mask.diagonal().all() or np.triu(mask, 1).any():
            raise ValueError("ancestor mask must include self and be causal in local flat order")
        if any(int(s) < 0 for s in node_slots):
            raise ValueError("scratch slot IDs cannot be negative")
        tables.append(table)
        slots.extend(int(s) for s in node_slots)
        offsets.append(offsets[-1] + n)
        squares.append(squares[-1] + n * n)
        q2r.extend([r] * n)
        local.extend(range(n))
        bias.append(np.where(mask, np.float32(0), np.float32(-np.inf)).reshape(-1))
    if len(set(slots)) != len(slots):
        raise ValueError("packed requests have overlapping scratch slot ranges")
    live = {p for table in tables for p in table}
    if any(s // block_size in live for s in slots):
        raise ValueError("scratch pages overlap a live committed prefix")
    width = max(1, max(len(t) for t in tables))
    return {"cu_seqlens_q": np.array(offsets, np.int32), "query_to_request": np.array(q2r, np.int32),
            "query_local_row": np.array(local, np.int32), "prefix_lens": np.array(prefixes, np.int32),
            "block_tables": np.array([t + [-1] * (width - len(t)) for t in tables], np.int32),
            "tree_slots": np.array(slots, np.int64), "qq_bias": np.concatenate(bias).astype(np.float32),
            "qq_bias_offsets": np.array(squares, np.int64), "node_counts": np.array(offsets[1:], np.int32)
            - np.array(offsets[:-1], np.int32)}


def child_maps(tokens, parents) -> list[dict]:
    """token -> child per node, later duplicate siblings win (the rule serving_ops.py:58-59 relies on)."""
    maps = [dict() for _ in tokens]
    for node in range(1, len(tokens)):
        maps[parents[node]][tokens[node]] = node
    return maps


def accept_walk(greedy, tokens, depths, children, max_depth) -> dict:
    """Greedy acceptance of one request (serving_ops.py:78-89)."""
    path = [0]
    while len(path) <= max_depth:
        nxt = children[path[-1]].get(greedy[path[-1]])
        if nxt is None:
            break
        path.append(nxt)
    if [depths[n] for n in path] != list(range(len(path))):
        raise RuntimeError("accepted RoPE positions do not match canonical tail")
    correction = greedy[path[-1]]
    return {"path": path, "accepted_length": len(path) - 1, "correction": correction,
            "outputs": [tokens[n] for n in path[1:]] + [correction]}


def truncate_accepted(values, path, budget: int, ignore_eos: bool, eos_token_ids) -> dict:
    """One request's max_new_tokens / EOS cut (batch_runtime.py:636-655).

    values = the tokens along the accepted path after the root, then the correction;
    budget = max_new_tokens - len(output_ids).  Returns limit, the emitted tokens
    values[:limit] and the cached path path[:limit].
    """
    values, path = [int(x) for x in values], [int(x) for x in path]
    if len(values) != len(path):
        raise ValueError("one value per path node: the draft tokens after the root, then the correction")
    limit = min(len(values), int(budget))
    if not ignore_eos:
        eos = {int(x) for x in eos_token_ids}
        first = next((j for j, token in enumerate(values[:limit]) if token in eos), None)
        if first is not None:
            limit = first + 1
    return {"limit": limit, "emitted": values[:limit], "path": path[:limit]}


def argmax_flip_witness(actual: np.ndarray, reference: np.ndarray) -> dict:
    """Flips allowed only where the reference margin <= 2 * sup error (jetspec_numeric_oracles.py:171-217)."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1, np.shape(actual)[-1])
    b = np.asarray(reference, dtype=np.float64).reshape(-1, np.shape(reference)[-1])
    if a.shape != b.shape or a.shape[-1] < 2:
        raise ValueError("logits must have equal shapes with vocabulary size >=2")
    if not (np.isfinite(a).all() and np.isfinite(b).all()):
        raise ValueError("nonfinite logits")
    flips = violations = 0
    for left, right in zip(a, b):
        wa, wb = int(left.argmax()), int(right.argmax())
        top = np.sort(right)[::-1][:2]
        margin = float(top[0] - top[1])
        delta = float(np.abs(left - right).max())
        gap = float(right[wb] - right[wa])
        flipped = wa != wb
        consistent = margin <= 2 * delta and gap <= 2 * delta
        flips += int(flipped)
        violations += int(flipped and not consistent)
    return {"rows_checked": a.shape[0], "argmax_flips": flips, "large_margin_violations": violations}


FP32_ATTENTION_BOUND = 1e-4   # benchmarks/jetspec_numeric_oracles.py:21


def round_f64_to_bf16(values: np.ndarray) -> np.ndarray:
    """float64 -> bf16 value as float64, the way the reference's ``.to(torch.bfloat16)`` of a
    float64 tensor rounds: to the nearest float32 first, then to the nearest bf16 (ties to
    even at both steps)."""
    with np.errstate(over="ignore"):
        single = np.asarray(values, dtype=np.float64).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(single)).astype(np.float64)


def bf16_ulp(rounded: np.ndarray) -> np.ndarray:
    """The larger spacing between a bf16 value and its two bf16 neighbours: 2^(e-8) for a
    normal value m * 2^e (the spacing below a power of two is the smaller one), and the
    smallest bf16 subnormal 2^-133 at zero."""
    r = np.asarray(rounded, dtype=np.float64)
    _, exponent = np.frexp(r)
    return np.where(r == 0, 2.0 ** -133, np.ldexp(1.0, exponent - 8))


def numerical_metrics(actual, reference, *, bound_scale: float = FP32_ATTENTION_BOUND,
                      bf16_output: bool | None = None) -> dict:
    """The reference's numerical_metrics (jetspec_numeric_oracles.py:108-168) in float64.

    within_fixed_bound = max-abs <= bound_scale * max(1, |reference|_max) and relative RMS
    (RMS of the difference over RMS of the reference) <= bound_scale; the bound applies to
    FP32 output before bf16 rounding.  The bf16 diagnostics measure errors in units of the
    larger neighbour spacing around the reference's nearest bf16 value.
    """
    a_in = np.asarray(actual)
    left = np.asarray(actual, dtype=np.float64)
    right = np.asarray(reference, dtype=np.float64)
    if left.shape != right.shape or left.size == 0:
        raise ValueError("metric tensors must have equal nonempty shapes")
    if not math.isfinite(float(bound_scale)) or float(bound_scale) <= 0:
        raise ValueError("bound scale must be finite and positive")
    quantized = (str(a_in.dtype) == "bfloat16") if bf16_output is None else bool(bf16_output)
    difference = left - right
    max_abs = float(np.abs(difference).max())
    rms_error = float(np.sqrt(np.mean(difference ** 2)))
    reference_rms = float(np.sqrt(np.mean(right ** 2)))
    reference_absmax = float(np.abs(right).max())
    if reference_rms:
        relative_rms = rms_error / reference_rms
    else:
        relative_rms = 0.0 if rms_error == 0.0 else float("inf")
    max_abs_bound = float(bound_scale) * max(1.0, reference_absmax)
    rounded = round_f64_to_bf16(right)
    ulp = bf16_ulp(rounded)
    bf16_difference = round_f64_to_bf16(left) - rounded
    return {
        "elements": int(left.size), "max_abs_error": max_abs, "rms_error": rms_error,
        "relative_rms_error": relative_rms, "reference_absmax": reference_absmax, "reference_rms": reference_rms,
        "max_abs_bound": max_abs_bound, "relative_rms_bound": float(bound_scale),
        "within_fixed_bound": max_abs <= max_abs_bound and relative_rms <= float(bound_scale),
        "fixed_bound_applicable": not quantized,
        "bf16_quantization": {
            "actual_output_is_bf16": quantized,
            "max_error_in_bf16_ulps": float((np.abs(difference) / ulp).max()),
            "max_distance_from_nearest_bf16_in_ulps": float((np.abs(bf16_difference) / ulp).max()),
            "nearest_bf16_unequal_elements": int(np.count_nonzero(bf16_difference)),
            "nearest_rounding_max_abs_error": float(np.abs(rounded - right).max()),
        },
    }


# --------------------------------------------------------------------------- HF-order RoPE + scatter
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; any NaN -> 0x7FC0 (c10 BFloat16 rounding)."""
    x = np.asarray(values, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded)


def _round_bf16(values: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(values))


def rope_hf_order(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, bf16: bool) -> np.ndarray:
    """Eager HF RoPE of float32 values `x` [..., D] with cos/sin [..., D/2] (qwen3.py:241-249).

    bf16: cos/sin are rounded to bf16, every product is rounded to bf16 before the
    add/subtract and the result is rounded to bf16 (tree_fusion.py:21-28); returns bf16
    values as float32.  fp32: separate fp32 products and sums (no fused multiply-add).
    """
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half].astype(np.float32), x[..., half:].astype(np.float32)
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    if bf16:
        with np.errstate(all="ignore"):
            cos, sin = _round_bf16(cos), _round_bf16(sin)
            a, b = _round_bf16(x1 * cos), _round_bf16(x2 * sin)
            c, d = _round_bf16(x2 * cos), _round_bf16(x1 * sin)
            return np.concatenate((_round_bf16(a - b), _round_bf16(c + d)), axis=-1)
    with np.errstate(all="ignore"):
        y1 = (x1 * cos).astype(np.float32) - (x2 * sin).astype(np.float32)
        y2 = (x2 * cos).astype(np.float32) + (x1 * sin).astype(np.float32)
    return np.concatenate((y1, y2), axis=-1).astype(np.float32)


def rope_scatter_hf(q, k, v, positions, cache, k_pool, v_pool, node_slots, bf16: bool):
    """Rotated Q, and K/V pools with the rotated K / raw V rows scattered (tree_fusion.py:42-82).

    q/k/v: float32 values [rows, heads, D] (bf16 operands given as their exact float32
    values); cache: float32 [positions, D] rows [cos | sin] (a bf16 cache as its float32
    values); k_pool/v_pool: [pages, page_size, kv_heads, D] arrays, updated in place;
    node_slots: unique slots.  Returns the rotated Q as float32 values.
    """
    positions = np.asarray(positions, dtype=np.int64)
    slots = np.asarray(node_slots, dtype=np.int64)
    rows = cache[positions]
    half = q.shape[-1] // 2
    cos, sin = rows[:, None, :half], rows[:, None, half:]
    with np.errstate(all="ignore"):
        out_q = rope_hf_order(q, cos, sin, bf16)
        out_k = rope_hf_order(k, cos, sin, bf16)
    page_size = k_pool.shape[1]
    pages, offsets = slots // page_size, slots % page_size
    k_pool[pages, offsets] = out_k
    v_pool[pages, offsets] = v
    return out_q

