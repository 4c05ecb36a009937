"""Helpers for the GPU parity tests: oracle comparisons on selected requests/rows."""
from __future__ import annotations

import numpy as np
import torch

import oracle

MAX_ABS = 2e-2      # north-star gate, bf16 output vs fp64 oracle
MEAN_ABS = 2e-3


def compact_problem(q, k_pool, v_pool, metadata, requests):
    """The selected requests as a self-contained oracle problem on the host.

    Copies only the pages and scratch slots those requests use (pages renumbered),
    so the fp64 oracle runs on a small pool even for multi-GB batches.  Returns the
    oracle's arguments and, per selected request, its packed row range.
    """
    block = metadata.block_size
    tree_slots = metadata.tree_slots.cpu().numpy()
    pages = []
    for r in requests:
        pages.extend(metadata.block_tables_host[r])
        sl = metadata.request_slice(r)
        pages.extend(int(s) // block for s in tree_slots[sl])
    pages = sorted(set(pages))
    remap = {p: i for i, p in enumerate(pages)}
    index = torch.tensor(pages, dtype=torch.long, device=k_pool.device)
    k_sub = k_pool.index_select(0, index).float().cpu().numpy()
    v_sub = v_pool.index_select(0, index).float().cpu().numpy()
    prefixes, tables, slots, masks, q_rows, ranges = [], [], [], [], [], []
    bias = metadata.qq_bias.cpu().numpy()
    boff = metadata.qq_bias_offsets.cpu().numpy()
    for r in requests:
        sl = metadata.request_slice(r)
        n = sl.stop - sl.start
        prefixes.append(metadata.prefix_lengths[r])
        tables.append([remap[p] for p in metadata.block_tables_host[r]])
        slots.append([remap[int(s) // block] * block + int(s) % block for s in tree_slots[sl]])
        masks.append(bias[boff[r]:boff[r] + n * n].reshape(n, n) == 0)
        q_rows.append(np.arange(sl.start, sl.stop))
        ranges.append(sl)
    meta = oracle.metadata_arrays(prefixes, tables, slots, masks, block)
    q_sub = q[torch.as_tensor(np.concatenate(q_rows), device=q.device)].float().cpu().numpy()
    return q_sub, k_sub, v_sub, meta, ranges


def oracle_rows(q, k_pool, v_pool, metadata, scale, requests, rows_per_request=None):
    """fp64 oracle output for the given requests: {request: (packed rows, float64 [rows, Hq, D])}."""
    q_sub, k_sub, v_sub, meta, ranges = compact_problem(q, k_pool, v_pool, metadata, requests)
    select = None
    if rows_per_request is not None:
        select, cursor = [], 0
        for sl in ranges:
            n = sl.stop - sl.start
            picks = sorted({0, n // 2, n - 1} | set(range(0, n, max(1, n // rows_per_request))))
            select.extend(cursor + p for p in picks)
            cursor += n
    out = oracle.tree_attention_f64(q_sub, k_sub, v_sub, scale=scale, rows=select, **meta)
    result, cursor = {}, 0
    for r, sl in zip(requests, ranges):
        n = sl.stop - sl.start
        local = np.arange(n)
        block = out[cursor:cursor + n]
        keep = ~np.isnan(block[:, 0, 0])
        result[r] = (sl.start + local[keep], block[keep])
        cursor += n
    return result


def errors(actual: torch.Tensor, expected: dict) -> tuple[float, float]:
    """(max-abs, mean-abs) of actual packed rows against the oracle rows."""
    got = actual.float().cpu().numpy()
    diffs = [np.abs(got[rows] - ref) for rows, ref in expected.values()]
    flat = np.concatenate([d.reshape(-1) for d in diffs])
    return float(flat.max()), float(flat.mean())


def metrics(actual: torch.Tensor, expected: dict) -> dict:
    """The reference's numerical_metrics (oracle restatement) over the compared rows."""
    got = actual.float().cpu().numpy()
    left = np.concatenate([got[rows].reshape(-1) for rows, _ in expected.values()])
    right = np.concatenate([ref.reshape(-1) for _, ref in expected.values()])
    return oracle.numerical_metrics(left, right, bf16_output=actual.dtype == torch.bfloat16)


def assert_within_gate(actual: torch.Tensor, expected: dict, label: str, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    mx, mean = errors(actual, expected)
    rel = metrics(actual, expected)["relative_rms_error"] if np.isfinite(mx) else float("nan")
    print(f"[{label}] max-abs {mx:.3e} mean-abs {mean:.3e} rel-RMS {100 * rel:.3f}%", flush=True)
    assert np.isfinite(mx), f"{label}: non-finite output"
    assert mx <= max_abs, f"{label}: max-abs {mx} > {max_abs}"
    assert mean <= mean_abs, f"{label}: mean-abs {mean} > {mean_abs}"
    return mx, mean


def torch_fp32_rows(q, k_pool, v_pool, metadata, scale) -> torch.Tensor:
    """Every packed row in float32 on the device: the semantics of paged_backend.py:116-213
    restated with torch (prefix keys through the page table, tree keys through their scratch
    slots and the ancestor bias, one softmax per row and query head).

    An independent floating-point reference for full-size batches, where the fp64 oracle
    can only take sampled rows; the tests pin it to that oracle on the sampled rows."""
    block = metadata.block_size
    kv_heads, dim = int(k_pool.shape[2]), int(k_pool.shape[3])
    groups = int(q.shape[1]) // kv_heads
    k_rows = k_pool.reshape(-1, kv_heads, dim)
    v_rows = v_pool.reshape(-1, kv_heads, dim)
    bias = metadata.qq_bias
    offsets = metadata.qq_bias_offsets.cpu().tolist()
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for r in range(metadata.num_requests):
        sl = metadata.request_slice(r)
        n = sl.stop - sl.start
        prefix = metadata.prefix_lengths[r]
        table = torch.as_tensor(metadata.block_tables_host[r], dtype=torch.long, device=q.device)
        pos = torch.arange(prefix, device=q.device)
        slots = torch.cat([table[pos // block] * block + pos % block, metadata.tree_slots[sl].long()])
        keys = k_rows.index_select(0, slots).float()          # [P + T, Hkv, D]
        values = v_rows.index_select(0, slots).float()
        tree_bias = bias[offsets[r]:offsets[r] + n * n].reshape(n, n).float()
        row_bias = torch.cat([torch.zeros((n, prefix), device=q.device), tree_bias], dim=1)   # [T, P + T]
        row_bias = row_bias.repeat_interleave(groups, dim=0)                                  # [T * G, P + T]
        for h in range(kv_heads):
            query = q[sl, h * groups:(h + 1) * groups, :].float().reshape(n * groups, dim)
            scores = query @ keys[:, h, :].t().contiguous() * scale + row_bias
            probs = torch.softmax(scores, dim=-1)
            result = probs @ values[:, h, :].contiguous()
            out[sl, h * groups:(h + 1) * groups, :] = result.reshape(n, groups, dim)
    return out


def assert_within_gate_dense(actual: torch.Tensor, expected: torch.Tensor, label: str, max_abs=MAX_ABS,
                             mean_abs=MEAN_ABS):
    """The north-star gate over every element of two [rows, heads, dim] tensors on one device."""
    diff = (actual.float() - expected.float()).abs()
    mx, mean = float(diff.max()), float(diff.mean())
    print(f"[{label}] every row: max-abs {mx:.3e} mean-abs {mean:.3e} over {actual.shape[0]} rows", flush=True)
    assert np.isfinite(mx), f"{label}: non-finite output"
    assert mx <= max_abs, f"{label}: max-abs {mx} > {max_abs}"
    assert mean <= mean_abs, f"{label}: mean-abs {mean} > {mean_abs}"
    return mx, mean
