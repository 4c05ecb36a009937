"""Prefill chunks through the packed kernel (GPU): a chunk of C rows at position P, its K/V in
scratch slots and its visibility a chain tree over the P-key prefix, against the reference's
dense-chunk computation (models/qwen3.py:566-618): the context gathered from the pool, then
SDPA under offset_causal_mask (prefill.py:14-26), here in fp32 on the CPU.  Gate: max-abs
2e-2 and mean-abs 2e-3 on the bf16 output.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_helpers import MAX_ABS, MEAN_ABS
from jetspec_amd import (PackedTreeMetadata, chain_tree_masks, offset_causal_mask, packed_tree_attention,
                         read_and_clear_status)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("prefix,chunk", [(0, 64), (300, 64), (2049, 512)])
def test_prefill_chunk_equals_sdpa_under_offset_causal_mask(prefix, chunk):
    print(f"[prefill] P={prefix} C={chunk}", flush=True)
    rng = np.random.default_rng(prefix + chunk)
    block, kv_heads, groups = 256, 8, 4
    prefix_pages = -(-prefix // block)
    scratch_pages = -(-chunk // block)
    order = rng.permutation(prefix_pages + scratch_pages + 2)
    table = [int(x) for x in order[:prefix_pages]]
    scratch = order[prefix_pages:prefix_pages + scratch_pages]
    slots = torch.as_tensor(((scratch[:, None] * block + np.arange(block)).reshape(-1)[:chunk]).astype(np.int64),
                            device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(prefix * 7 + chunk)
    pages = len(order)
    k = torch.randn((pages, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn((pages, block, kv_heads, 128), generator=gen, device=DEV).to(torch.bfloat16)
    q = torch.randn((chunk, kv_heads * groups, 128), generator=gen, device=DEV).to(torch.bfloat16)
    meta = PackedTreeMetadata.build([prefix], [table], [slots], chain_tree_masks([chunk], DEV), block)
    out = packed_tree_attention(q, k, v, meta, 128 ** -0.5, groups)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 0
    # The reference's dense chunk: the context gathered in position order, then SDPA.
    positions = torch.arange(prefix)
    prefix_slots = torch.tensor(table, dtype=torch.int64)[positions // block] * block + positions % block
    context = torch.cat((prefix_slots, slots.cpu()))
    keys = k.view(-1, kv_heads, 128).cpu()[context].float().repeat_interleave(groups, dim=1).transpose(0, 1)
    values = v.view(-1, kv_heads, 128).cpu()[context].float().repeat_interleave(groups, dim=1).transpose(0, 1)
    queries = q.cpu().float().transpose(0, 1)
    mask = offset_causal_mask(prefix, chunk, "cpu")
    expect = F.scaled_dot_product_attention(queries, keys.contiguous(), values.contiguous(), attn_mask=mask,
                                            is_causal=mask is None, scale=128 ** -0.5).transpose(0, 1)
    diff = (out.cpu().float() - expect).abs()
    print(f"[prefill] max-abs {diff.max().item():.3e} mean-abs {diff.mean().item():.3e}", flush=True)
    assert diff.max().item() <= MAX_ABS and diff.mean().item() <= MEAN_ABS
