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
