"""One tensor-parallel shard of the verify (GPU): 1 or 2 of the 8 KV heads with their query heads.

A TP split over KV heads gives each GPU `Hkv/TP` heads of every request at the full
context length; the kernel sees only a smaller `num_kv_heads`.  Checked:
  * a shard batch built with 1 or 2 KV heads matches the fp64 oracle on every row
    (the attention tolerance: max-abs 2e-2, mean-abs 2e-3);
  * a shard taken as a strided view of the 8-head pool (key stride of 8 heads, one
    head's columns) gives the same bits as the same heads of a contiguous copy.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import packed_tree_attention, read_and_clear_status, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.mark.parametrize("kv_heads", [1, 2])
def test_shard_matches_oracle(kv_heads):
    batch = workloads.config2(DEV, kv_heads=kv_heads)
    assert batch.q.shape[1] == 4 * kv_heads and batch.k_pool.shape[2] == kv_heads
    out = packed_tree_attention(batch.q, batch.k_pool, batch.v_pool, batch.metadata, batch.scale, batch.groups)
    torch.cuda.synchronize()
    print(f"[shard] kv_heads={kv_heads} rows={batch.total_queries}", flush=True)
    want = oracle.metadata_tree_attention_f64(batch.q, batch.k_pool, batch.v_pool, batch.metadata, batch.scale)
    diff = np.abs(out.float().cpu().numpy() - want)
    assert diff.max() <= MAX_ABS and diff.mean() <= MEAN_ABS, (diff.max(), diff.mean())
    assert read_and_clear_status(DEV) == 0


def test_strided_shard_view_equals_contiguous_shard():
    batch = workloads.config2(DEV)
    h = 5
    k_view, v_view = batch.k_pool[:, :, h:h + 1], batch.v_pool[:, :, h:h + 1]
    q_view = batch.q[:, 4 * h:4 * h + 4]
    a = packed_tree_attention(q_view, k_view, v_view, batch.metadata, batch.scale, 4)
    b = packed_tree_attention(q_view.contiguous(), k_view.contiguous(), v_view.contiguous(), batch.metadata,
                              batch.scale, 4)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert read_and_clear_status(DEV) == 0
