"""The allocation-free attention entry (tv_tree_attention_noalloc) against tv_tree_attention (GPU).

Both are called through the C ABI with the same argument block; the allocation-free one
gets no workspace and keeps split-prefix partials in the library's per-device scratch.
Two calls in a row, the second with a smaller batch (the scratch keeps the first call's
contents), must each equal the existing entry bit for bit and meet the oracle gate; a
plan beyond the scratch is refused before any launch.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_helpers import assert_within_gate, oracle_rows
from jetspec_amd import _device, _lib, read_and_clear_status, workloads
from jetspec_amd.paged_backend import derived_state, fill_pool_args

pytestmark = pytest.mark.gpu
DEV = "cuda"


def argument_block(batch, out, workspace):
    meta = batch.metadata
    kv_heads = int(batch.k_pool.shape[2])
    state = derived_state(meta, kv_heads, queries_per_kv=batch.groups)
    a = _lib.TreeAttentionArgs()
    fill_pool_args(a, meta, batch.k_pool, batch.v_pool, kv_heads, batch.groups, _device.status_word(out.device))
    a.q = batch.q.data_ptr()
    a.q_stride_row, a.q_stride_head = batch.q.stride(0), batch.q.stride(1)
    a.out = out.data_ptr()
    a.out_stride_row, a.out_stride_head = out.stride(0), out.stride(1)
    a.out_dtype = _device.dtype_code(out.dtype)
    a.scale = float(batch.scale)
    a.ancestor_words = state["ancestor_words"].data_ptr()
    a.ancestor_words_per_row = state["words_per_row"]
    a.items = state["items_dev"].data_ptr()
    a.num_items = state["num_items"]
    a.groups = state["groups_dev"].data_ptr() if state["groups_dev"] is not None else None
    a.num_groups = state["num_groups"]
    a.num_partial_slots = state["num_partial_slots"]
    a.workspace = workspace.data_ptr() if workspace is not None else None
    a.workspace_bytes = workspace.numel() if workspace is not None else 0
    return a, state


def test_noalloc_equals_tree_attention_on_two_calls():
    lib = _lib.library()
    stream = _device.stream_handle(torch.device(DEV))
    for name, builder in (("cfg2", workloads.config2), ("cfg1", workloads.config1)):
        batch = builder(DEV)
        meta = batch.metadata
        print(f"[noalloc] {name}: {meta.num_requests} requests, {meta.total_queries} rows", flush=True)
        expect_out = torch.empty_like(batch.q)
        probe, state = argument_block(batch, expect_out, None)
        assert state["num_partial_slots"] > 0, "the case must use the split-K scratch"
        workspace = torch.empty(state["workspace_bytes"], dtype=torch.uint8, device=DEV)
        a, _ = argument_block(batch, expect_out, workspace)
        _lib.check(lib.tv_tree_attention(ctypes.byref(a), stream), "tree_attention")
        got = torch.full_like(batch.q, float("nan"))
        b, _ = argument_block(batch, got, None)
        _lib.check(lib.tv_tree_attention_noalloc(ctypes.byref(b), stream), "tree_attention_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), expect_out.view(torch.int16)), f"{name}: differs from tv_tree_attention"
        expected = oracle_rows(batch.q, batch.k_pool, batch.v_pool, meta, batch.scale,
                               list(range(meta.num_requests)), rows_per_request=8)
        assert_within_gate(got, expected, f"noalloc {name}")
        assert read_and_clear_status(DEV) == 0


def test_noalloc_refuses_plans_beyond_its_scratch():
    lib = _lib.library()
    limit = lib.tv_tree_attention_noalloc_max_workspace()
    assert limit == 64 << 20
    batch = workloads.config1(DEV)
    out = torch.empty_like(batch.q)
    a, _ = argument_block(batch, out, None)
    a.num_partial_slots = 600            # 600 x 130 KiB of partials > 64 MiB
    code = lib.tv_tree_attention_noalloc(ctypes.byref(a), None)
    assert code == _lib.TV_ERR_CAPACITY
    assert b"scratch" in lib.tv_last_error()


_FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys
sys.path[:0] = {paths!r}
import torch
from jetspec_amd import _device, _lib, read_and_clear_status, workloads
from test_zz_no_alloc import argument_block
lib = _lib.library()
batch = workloads.config1("cuda")
expect = torch.empty_like(batch.q)
probe, state = argument_block(batch, expect, None)
workspace = torch.empty(state["workspace_bytes"], dtype=torch.uint8, device="cuda")
a, _ = argument_block(batch, expect, workspace)
_lib.check(lib.tv_tree_attention(ctypes.byref(a), _device.stream_handle(torch.device("cuda"))), "tree_attention")
got = torch.full_like(batch.q, float("nan"))
b, _ = argument_block(batch, got, None)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    code = lib.tv_tree_attention_noalloc(ctypes.byref(b), torch.cuda.current_stream().cuda_stream)
assert code == 0, lib.tv_last_error()
for replay in range(3):
    got.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), expect.view(torch.int16)), f"replay {{replay}} differs"
assert read_and_clear_status("cuda") == 0
print("first call under capture: 3 replays equal tv_tree_attention", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """The process's first tv_tree_attention_noalloc call happens inside a graph capture (the
    scratch address is looked up then); every replay equals tv_tree_attention bit for bit.  Run
    in a fresh process so that no earlier call has resolved the scratch."""
    import subprocess
    import sys
    from pathlib import Path

    tests = Path(__file__).resolve().parent
    paths = [str(tests), str(tests.parent), str(tests.parent / "nano-vllm-jetspec_amd")]
    print("[noalloc] first call under capture (subprocess)", flush=True)
    result = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE.format(paths=paths)],
                            capture_output=True, text=True, timeout=110)
    print(result.stdout[-2000:], result.stderr[-2000:], flush=True)
    assert result.returncode == 0
    assert "3 replays equal" in result.stdout
