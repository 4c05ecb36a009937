"""Plans that no longer match the live metadata, and the first call's upload (GPU).

The eager drop-in plans once per metadata object from the object's host copies, as the
reference's frozen dataclass allows; the reference's kernels read the prefix length in every
program (paged_backend.py:138).  Here the kernel checks every work item against the live
device prefix lengths and node counts: a request that grew after planning sets
TV_STATUS_STALE_PLAN, one that shrank below a planned chunk sets TV_STATUS_BAD_REQUEST too and
that chunk is skipped, and a plan made for another query-head grouping is refused item by
item.  Every kernel exits normally, and restoring the metadata restores the bitwise result.
"""
from __future__ import annotations

import ctypes
import gc

import pytest
import torch

from jetspec_amd import _device, _lib, packed_tree_attention, read_and_clear_status, workloads
from jetspec_amd.paged_backend import derived_state, fill_pool_args
from test_attention_gpu import bits_equal, reference_fixture

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5
STALE = _lib.TV_STATUS_STALE_PLAN
BAD_REQUEST = _lib.TV_STATUS_BAD_REQUEST


def attention(q, k, v, meta):
    out = packed_tree_attention(q, k, v, meta, SCALE, 4)
    torch.cuda.synchronize()
    return out, read_and_clear_status(DEV)


@pytest.mark.parametrize("chunk", [0, 32])
def test_grown_prefix_sets_stale_plan(chunk):
    """Request 0's prefix grows from 65 to 85 keys in place (same page) after its plan was made;
    chunk 32 splits every prefix, so the grown request's last chunk is one of several."""
    q, k, v, meta, *_ = reference_fixture()
    print(f"[stale] grown prefix, chunk {chunk}", flush=True)
    run = lambda: (packed_tree_attention(q, k, v, meta, SCALE, 4, chunk_keys=chunk), torch.cuda.synchronize())[0]
    first = run()
    assert read_and_clear_status(DEV) == 0
    rows0 = meta.request_slice(0)
    meta.prefix_lens[0] += 20
    grown = run()
    status = read_and_clear_status(DEV)
    assert status & STALE and not status & ~STALE, status
    # The other requests' rows are untouched by the change; request 0's planned keys are computed.
    assert bits_equal(grown[rows0.stop:], first[rows0.stop:])
    assert torch.isfinite(grown[rows0]).all().item()
    meta.prefix_lens[0] -= 20
    again = run()
    assert read_and_clear_status(DEV) == 0
    assert bits_equal(again, first)


def test_shrunk_prefix_skips_the_chunk_past_it():
    """Request 2's prefix shrinks from 257 to 200 keys: its planned chunk now reaches past the
    prefix, so it is reported (bad request and stale plan) and skipped, never read."""
    q, k, v, meta, *_ = reference_fixture()
    first, status = attention(q, k, v, meta)
    assert status == 0
    meta.prefix_lens[2] -= 57
    out, status = attention(q, k, v, meta)
    assert status == BAD_REQUEST | STALE, status
    rows2 = meta.request_slice(2)
    assert bits_equal(out[:rows2.start], first[:rows2.start])
    meta.prefix_lens[2] += 57
    again, status = attention(q, k, v, meta)
    assert status == 0 and bits_equal(again, first)


def test_grown_node_count_sets_stale_plan():
    """Request 0's tree grows from 63 to 65 nodes in place: its plan's one node block (64 nodes
    of one KV head at 4 query heads per KV head) no longer covers it.  Every address the kernel
    forms stays inside the packed batch (the grown rows are request 1's)."""
    q, k, v, meta, *_ = reference_fixture()
    first, status = attention(q, k, v, meta)
    assert status == 0
    meta.node_counts[0] += 2
    _, status = attention(q, k, v, meta)
    assert status & STALE and not status & ~STALE, status
    meta.node_counts[0] -= 2
    again, status = attention(q, k, v, meta)
    assert status == 0 and bits_equal(again, first)


def test_request_rows_past_the_batch_are_refused():
    """The last request's node count grows past the packed rows: its items would address Q and O
    rows outside the batch, so they are reported and skipped."""
    q, k, v, meta, *_ = reference_fixture()
    first, status = attention(q, k, v, meta)
    assert status == 0
    meta.node_counts[2] += 13
    out, status = attention(q, k, v, meta)
    assert status & BAD_REQUEST, status
    rows2 = meta.request_slice(2)
    assert bits_equal(out[:rows2.start], first[:rows2.start])
    meta.node_counts[2] -= 13
    again, status = attention(q, k, v, meta)
    assert status == 0 and bits_equal(again, first)


def test_plan_for_another_grouping_is_refused():
    """A plan made for 4 query heads per KV head, launched through the C ABI with 8: its items
    lay nodes out for the other grouping, so every item is refused and nothing is written."""
    q, k, v, meta, *_ = reference_fixture()
    kv_heads = int(k.shape[2])
    state = derived_state(meta, kv_heads, queries_per_kv=4)
    q8 = torch.randn((meta.total_queries, 8 * kv_heads, 128), device=DEV).to(q.dtype)
    out = torch.full_like(q8, float("nan"))
    workspace = (torch.empty(state["workspace_bytes"], dtype=torch.uint8, device=DEV)
                 if state["workspace_bytes"] else None)
    a = _lib.TreeAttentionArgs()
    fill_pool_args(a, meta, k, v, kv_heads, 8, _device.status_word(out.device))
    a.q, a.q_stride_row, a.q_stride_head = q8.data_ptr(), q8.stride(0), q8.stride(1)
    a.out, a.out_stride_row, a.out_stride_head = out.data_ptr(), out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.scale = SCALE
    a.ancestor_words = state["ancestor_words"].data_ptr()
    a.ancestor_words_per_row = state["words_per_row"]
    a.items, a.num_items = state["items_dev"].data_ptr(), state["num_items"]
    a.groups = state["groups_dev"].data_ptr() if state["groups_dev"] is not None else None
    a.num_groups, a.num_partial_slots = state["num_groups"], state["num_partial_slots"]
    a.workspace = workspace.data_ptr() if workspace is not None else None
    a.workspace_bytes = workspace.numel() if workspace is not None else 0
    _lib.check(_lib.library().tv_tree_attention(ctypes.byref(a), _device.stream_handle(out.device)), "attention")
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) & BAD_REQUEST
    assert torch.isnan(out).all().item()


def test_first_call_on_new_metadata_queues_behind_a_busy_stream():
    """The first attention call on a new metadata object (plan, pinned upload, argument block)
    returns while the stream is still busy: it enqueues and never waits for queued kernels."""
    warm = workloads.config1(DEV)
    packed_tree_attention(warm.q, warm.k_pool, warm.v_pool, warm.metadata, warm.scale, 4)
    torch.cuda.synchronize()
    fresh = workloads.config1(DEV, seed=11)
    del warm
    gc.collect()
    torch.cuda.synchronize()
    busy_done = torch.cuda.Event()
    torch.cuda._sleep(int(2e8))
    busy_done.record()
    out = packed_tree_attention(fresh.q, fresh.k_pool, fresh.v_pool, fresh.metadata, fresh.scale, 4)
    still_busy = not busy_done.query()
    torch.cuda.synchronize()
    assert still_busy, "the first call on new metadata waited for the stream"
    assert torch.isfinite(out).all().item() and read_and_clear_status(DEV) == 0
