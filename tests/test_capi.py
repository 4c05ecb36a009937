"""The C-ABI library: loads, exports every declared symbol, and its host planner (CPU).

No device call is made here (there is no GPU in the CPU suite); the work planner is
pure host code, so its coverage invariants are checked exhaustively on CPU.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
import re

import numpy as np
import pytest

from jetspec_amd import _lib
from jetspec_amd.paged_backend import make_plan

HEADER = Path(__file__).resolve().parents[1] / "include" / "treeverify.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    declared = declared_functions()
    assert declared, "no declarations parsed"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_struct_layout():
    lib = _lib.library()
    assert lib.tv_abi_version() == _lib.ABI_VERSION
    assert lib.tv_sizeof_tree_attention_args() == ctypes.sizeof(_lib.TreeAttentionArgs)
    assert lib.tv_sizeof_tree_attention_fp32_args() == ctypes.sizeof(_lib.TreeAttentionFp32Args)
    assert lib.tv_last_error() is not None


def test_entry_points_reject_bad_arguments_without_a_device():
    lib = _lib.library()
    # A null args pointer and an invalid store are rejected before any launch.
    assert lib.tv_tree_attention(None, None) == _lib.TV_ERR_INVALID
    assert b"null" in lib.tv_last_error()
    assert lib.tv_store_kvcache(None, 0, None, 0, None, None, 0, None, 0, -1, 8, 2, None, None) == _lib.TV_ERR_INVALID
    shape = (ctypes.c_int64 * 6)(3, 1, 1, 16, 1, 8)
    stride = (ctypes.c_int64 * 6)(128, 128, 128, 8, 8, 1)
    assert lib.tv_copy_accepted_kv(None, shape, stride, 2, None, None, 1, None, 0, None, None, None) \
        == _lib.TV_ERR_INVALID
    assert lib.tv_copy_accepted_kv_workspace_bytes(12, 36, 1024, 2) >= 2 * 36 * 12 * 1024 * 2
    # commit_slots: bad sizes and null pointers fail on the host; no requests is a no-op.
    assert lib.tv_commit_slots(None, None, None, None, None, 0, 0, None, 1, 0, 8, None, None, None, None) \
        == _lib.TV_ERR_INVALID
    assert lib.tv_commit_slots(None, None, None, None, None, 2, 4, None, 1, 16, 8, None, None, None, None) \
        == _lib.TV_ERR_INVALID
    assert lib.tv_commit_slots(None, None, None, None, None, 0, 0, None, 0, 16, 8, None, None, None, None) \
        == _lib.TV_OK
    # truncate_accepted: bad counts and null pointers fail on the host; no requests is a no-op.
    assert lib.tv_truncate_accepted(None, 0, None, None, None, 0, None, 1, None, None, None, 0, None, None, None,
                                    None, None, None) == _lib.TV_ERR_INVALID
    assert lib.tv_truncate_accepted(None, 9, None, None, None, 0, None, 1, None, None, None, 0, None, None, None,
                                    None, None, None) == _lib.TV_ERR_INVALID
    assert lib.tv_truncate_accepted(None, 9, None, None, None, 0, None, 0, None, None, None, 0, None, None, None,
                                    None, None, None) == _lib.TV_OK
    with pytest.raises(ValueError, match="block_size"):
        make_plan([10], [4], 8, 48, 256, queries_per_kv=4)
    with pytest.raises(ValueError, match="no tree nodes"):
        make_plan([10], [0], 8, 256, 256, queries_per_kv=4)
    for bad_group in (0, 9, 12, 32):
        with pytest.raises(ValueError, match="query heads per KV head"):
            make_plan([10], [4], 8, 256, 256, queries_per_kv=bad_group)


def test_fp32_attention_rejects_bad_arguments_without_a_device():
    lib = _lib.library()
    assert lib.tv_tree_attention_fp32(None, None) == _lib.TV_ERR_INVALID

    def args(**over):
        a = _lib.TreeAttentionFp32Args()
        a.q = a.k_pool = a.v_pool = a.out = 0x10000
        a.cu_seqlens_q = a.query_to_request = a.query_local_row = a.prefix_lens = a.node_counts = 0x10000
        a.block_tables = a.tree_slots = a.qq_bias = a.qq_bias_offsets = 0x10000
        a.in_dtype = a.out_dtype = _lib.TV_F32
        a.num_requests, a.total_queries = 1, 4
        a.num_q_heads, a.num_kv_heads, a.head_dim, a.block_size = 6, 2, 96, 16
        a.num_blocks = 8
        a.scale = 0.1
        for name, value in over.items():
            setattr(a, name, value)
        return a
    cases = [
        (dict(num_q_heads=5), _lib.TV_ERR_INVALID, b"query heads over"),
        (dict(num_kv_heads=0), _lib.TV_ERR_INVALID, b"query heads over"),
        (dict(head_dim=513), _lib.TV_ERR_UNSUPPORTED, b"head_dim 513"),
        (dict(head_dim=0), _lib.TV_ERR_UNSUPPORTED, b"head_dim 0"),
        (dict(block_size=0), _lib.TV_ERR_INVALID, b"pool geometry"),
        (dict(in_dtype=7), _lib.TV_ERR_INVALID, b"dtypes"),
        (dict(scale=float("nan")), _lib.TV_ERR_INVALID, b"finite"),
        (dict(qq_bias=None), _lib.TV_ERR_INVALID, b"null pointer"),
        (dict(num_requests=0), _lib.TV_ERR_INVALID, b"counts"),
    ]
    for over, code, message in cases:
        assert lib.tv_tree_attention_fp32(ctypes.byref(args(**over)), None) == code, over
        assert message in lib.tv_last_error(), (over, lib.tv_last_error())
    # No rows: nothing to launch (no device needed).
    assert lib.tv_tree_attention_fp32(ctypes.byref(args(total_queries=0)), None) == _lib.TV_OK


def test_attention_rejects_strides_beyond_its_32_bit_offsets_without_a_device():
    """Checked before any launch: the kernel's per-lane tile offsets are 32-bit."""
    lib = _lib.library()

    def args(k_stride):
        a = _lib.TreeAttentionArgs()
        a.q = a.k_pool = a.v_pool = a.out = 0x10000
        a.q_stride_row, a.q_stride_head = 8 * 128, 128
        a.out_stride_row, a.out_stride_head = 8 * 128, 128
        for i in range(4):
            a.k_stride[i] = k_stride[i]
            a.v_stride[i] = (256 * 2 * 128, 2 * 128, 128, 1)[i]
        a.in_dtype = a.out_dtype = _lib.TV_BF16
        a.num_q_heads, a.num_kv_heads, a.head_dim, a.block_size = 8, 2, 128, 256
        a.scale = 128 ** -0.5
        a.ancestor_words_per_row = 1
        return a
    for bad in ((1 << 31, 256, 128, 1),          # page stride of 4 GiB
                (256 * 256, 1 << 25, 128, 1),   # 32 key rows span 2 GiB
                (256 * 256, 256, 1 << 30, 1)):  # next KV head 2 GiB away
        assert lib.tv_tree_attention(ctypes.byref(args(bad)), None) == _lib.TV_ERR_UNSUPPORTED, bad
        assert b"strides out of range" in lib.tv_last_error()
    # Head sizes: 128 for every group, 64 and 256 for the power-of-two groups; others take the
    # FP32 entry.
    for head, q_heads, accepted in ((64, 8, True), (64, 32, True), (64, 6, False), (96, 8, False),
                                    (256, 8, True), (256, 32, True), (256, 6, False), (512, 8, False)):
        a = args((256 * 256, 256, 128, 1))
        a.head_dim, a.num_q_heads, a.num_requests = head, q_heads, 1
        code = lib.tv_tree_attention(ctypes.byref(a), None)
        if accepted:
            assert code == _lib.TV_OK, lib.tv_last_error()   # no items: accepted and nothing launched
        else:
            assert code == _lib.TV_ERR_UNSUPPORTED and b"head_dim" in lib.tv_last_error(), (head, q_heads)
    big = args((256 * 256, 256, 128, 1))
    big.num_blocks, big.num_requests = (1 << 31) // 256, 1
    assert lib.tv_tree_attention(ctypes.byref(big), None) == _lib.TV_ERR_UNSUPPORTED
    assert b"at most 2^31 slots" in lib.tv_last_error()
    # A split plan's partial slots need a workspace; a negative slot count is invalid.
    for slots, workspace, message in ((-1, 0x20000, b"invalid counts"), (4, 0, b"without groups/workspace")):
        a = args((256 * 256, 256, 128, 1))
        a.num_blocks, a.num_requests, a.num_items = 8, 1, 1
        a.cu_seqlens_q = a.prefix_lens = a.node_counts = a.block_tables = a.items = 0x10000
        a.tree_slots = a.ancestor_words = 0x10000
        a.num_partial_slots, a.workspace, a.workspace_bytes = slots, workspace, 1 << 30
        assert lib.tv_tree_attention(ctypes.byref(a), None) == _lib.TV_ERR_INVALID, slots
        assert message in lib.tv_last_error()


def test_split_workspace_follows_the_head_size():
    """A plan's workspace_bytes holds head sizes up to 128; at 256 the partial rows are twice
    as long, and tv_tree_attention refuses the plan's figure (TV_ERR_CAPACITY) until the
    workspace is tv_tree_attention_workspace_bytes(slots, 256)."""
    lib = _lib.library()
    plan = make_plan([3000, 5000, 700], [40, 64, 17], 8, 256, 256, chunk_keys=512, queries_per_kv=4)
    slots, ws = plan["num_partial_slots"], plan["workspace_bytes"]
    assert slots > 0
    for head in (64, 96, 128):
        assert lib.tv_tree_attention_workspace_bytes(slots, head) == ws, head
    rows = slots * 256
    assert ws == -(-rows * 128 * 4 // 256) * 256 + -(-rows * 8 // 256) * 256
    assert lib.tv_tree_attention_workspace_bytes(slots, 256) == -(-rows * 256 * 4 // 256) * 256 + -(-rows * 8 // 256) * 256
    assert lib.tv_tree_attention_workspace_bytes(0, 256) == 0
    a = _lib.TreeAttentionArgs()
    a.q = a.k_pool = a.v_pool = a.out = 0x10000
    a.q_stride_row, a.q_stride_head = 8 * 256, 256
    a.out_stride_row, a.out_stride_head = 8 * 256, 256
    for i in range(4):
        a.k_stride[i] = a.v_stride[i] = (256 * 2 * 256, 2 * 256, 256, 1)[i]
    a.in_dtype = a.out_dtype = _lib.TV_BF16
    a.num_q_heads, a.num_kv_heads, a.head_dim, a.block_size = 8, 2, 256, 256
    a.scale = 256 ** -0.5
    a.ancestor_words_per_row = 1
    a.num_blocks, a.num_requests, a.num_items, a.num_groups = 8, 1, 1, 1
    a.cu_seqlens_q = a.prefix_lens = a.node_counts = a.block_tables = a.items = a.groups = 0x10000
    a.tree_slots = a.ancestor_words = 0x10000
    a.num_partial_slots, a.workspace, a.workspace_bytes = slots, 0x20000, ws
    assert lib.tv_tree_attention(ctypes.byref(a), None) == _lib.TV_ERR_CAPACITY
    assert b"workspace" in lib.tv_last_error()
    # The built-in scratch of the allocation-free entry holds half as many slots at 256.
    scratch = lib.tv_tree_attention_noalloc_max_workspace()
    assert lib.tv_tree_attention_workspace_bytes(504, 128) <= scratch < lib.tv_tree_attention_workspace_bytes(505, 128)
    assert lib.tv_tree_attention_workspace_bytes(254, 256) <= scratch < lib.tv_tree_attention_workspace_bytes(255, 256)
    a.num_partial_slots = 255
    assert lib.tv_tree_attention_noalloc(ctypes.byref(a), None) == _lib.TV_ERR_CAPACITY


def nodes_per_item(hpw, groups):
    """A work item is 8 waves x 32 score rows: (8 / hpw) * (32 / groups) nodes per KV head."""
    return (8 // hpw) * (32 // groups)


def heads_per_group(nodes, kv_heads, groups=4):
    h = 2 if nodes <= nodes_per_item(2, groups) else 1
    while h > 1 and h > kv_heads:
        h //= 2
    return h


def check_plan_covers(prefixes, counts, kv_heads, cus, chunk=0, block=256, groups=4):
    plan = make_plan(prefixes, counts, kv_heads, block, cus, chunk, queries_per_kv=groups)
    items, merges = plan["items"], plan["groups"]
    covered = {}
    slots_seen = set()
    for r, h0, n0, kbeg, kend, flags, slot, hpw in items.tolist():
        assert hpw == heads_per_group(counts[r], kv_heads, groups)
        assert h0 % hpw == 0 and n0 % nodes_per_item(hpw, groups) == 0
        assert 0 <= kbeg <= kend <= prefixes[r] and kbeg % 32 == 0
        key = (r, h0, n0)
        covered.setdefault(key, []).append((kbeg, kend, flags, slot))
        if slot >= 0:
            assert slot not in slots_seen
            slots_seen.add(slot)
    for r, (p, t) in enumerate(zip(prefixes, counts)):
        hpw = heads_per_group(t, kv_heads, groups)
        npw = nodes_per_item(hpw, groups)
        for h0 in range(0, kv_heads, hpw):
            for n0 in range(0, t, npw):
                ranges = sorted(covered.pop((r, h0, n0)))
                # contiguous prefix coverage, tree exactly once, on the last chunk
                assert ranges[0][0] == 0 and ranges[-1][1] == p
                for a, b in zip(ranges, ranges[1:]):
                    assert a[1] == b[0]
                # flags: last chunk (bit 0), last node block (bit 1), the plan's group size (bits 8-15)
                assert [f & 1 for _, _, f, _ in ranges] == [0] * (len(ranges) - 1) + [1]
                assert all(bool(f & 2) == (n0 + npw >= t) for _, _, f, _ in ranges)
                assert all((f >> 8) & 0xFF == groups and not f & ~0xFF03 for _, _, f, _ in ranges)
                if len(ranges) > 1:
                    assert all(s >= 0 for _, _, _, s in ranges)
                else:
                    assert ranges[0][3] == -1
    assert not covered
    assert plan["num_partial_slots"] == len(slots_seen)
    for r, h0, n0, hpw, first, ns, qpk, zero in merges.tolist():
        assert set(range(first, first + ns)) <= slots_seen
        assert qpk == groups and zero == 0
    check_order(items.tolist(), counts)
    return plan


XCD_WINDOW = 64   # 8 XCDs x 8 items: workgroup i runs on XCD i % 8
# Planner cost per key, in quarter key-steps of a one-head item: a two-head item's tile
# takes ~1.25x a one-head tile (measured per workgroup), not 2x.
COST_WEIGHT = {1: 4, 2: 5}


def check_order(items, counts):
    """The dispatch order: longest first, up to the XCD placement of K/V-sharing groups.

    Items of one (request, head group, chunk) stream form a group.  Full 64-item
    windows are column-major (position 8 * (k % 8) + c holds rank k, with column
    c = k / 8, mirrored to 7 - k / 8 in odd windows), so ranks are recovered by
    inverting that.  When every multi-item group has a multiple of 8 items,
    each group must be whole aligned 8-rank blocks, and the rank order may differ from
    longest first only by groups moved ahead of at most 7 longer single items.  Otherwise
    every window must be at least as long as the next (placement only permutes within a
    window) and the partial last window stays longest first.
    """
    n = len(items)
    cost = [(kend - kbeg + (counts[r] if flags & 1 else 0)) * COST_WEIGHT[hpw]
            for r, _, _, kbeg, kend, flags, _, hpw in items]
    stream = [(r, h0, kbeg) for r, h0, _, kbeg, _, _, _, _ in items]
    sizes = {}
    for key in stream:
        sizes[key] = sizes.get(key, 0) + 1
    groups = {k: v for k, v in sizes.items() if v > 1}
    if not groups:
        assert cost == sorted(cost, reverse=True), "items must be ordered longest first"
        return
    full = n // XCD_WINDOW * XCD_WINDOW
    rank_of = list(range(n))
    for pos in range(full):
        w, k = pos - pos % XCD_WINDOW, pos % XCD_WINDOW
        column = 7 - k % 8 if (w // XCD_WINDOW) % 2 else k % 8
        rank_of[pos] = w + 8 * column + k // 8
    by_rank = [None] * n
    for pos in range(n):
        by_rank[rank_of[pos]] = pos
    if all(v % 8 == 0 for v in groups.values()):
        ranks = {}
        for pos in range(n):
            ranks.setdefault(stream[pos], []).append(rank_of[pos])
        for key, rs in ranks.items():
            if key in groups:
                rs = sorted(rs)
                assert rs == list(range(rs[0], rs[0] + len(rs))) and rs[0] % 8 == 0, "group not in whole 8-rank blocks"
        seq = [(cost[pos], stream[pos] in groups, stream[pos]) for pos in by_rank]
        singles = [c for c, g, _ in seq if not g]
        grouped = [c for c, g, _ in seq if g]
        assert singles == sorted(singles, reverse=True) and grouped == sorted(grouped, reverse=True)
        for i, (c, g, key) in enumerate(seq):
            if g and (i == 0 or seq[i - 1][2] != key):
                longer_after = sum(1 for c2, g2, _ in seq[i:] if not g2 and c2 > c)
                assert longer_after <= 7, "a group moved ahead of more than 7 longer items"
        return
    windows = [cost[w:w + XCD_WINDOW] for w in range(0, n, XCD_WINDOW)]
    for a, b in zip(windows, windows[1:]):
        assert min(a) >= max(b), "items must be ordered longest first"
    if n % XCD_WINDOW:
        tail = windows[-1]
        assert tail == sorted(tail, reverse=True), "the partial last window keeps longest-first order"


@pytest.mark.parametrize("prefixes,counts", [
    ([512], [16]),
    ([0, 1, 63, 64, 65, 255, 256, 257], [1, 2, 16, 17, 32, 33, 64, 65]),
    ([4096, 300, 0], [512, 31, 64]),
])
@pytest.mark.parametrize("kv_heads", [1, 2, 8])
@pytest.mark.parametrize("chunk", [0, 32, 256])
def test_plan_covers_every_row_and_key_once(prefixes, counts, kv_heads, chunk):
    check_plan_covers(prefixes, counts, kv_heads, 256, chunk)


@pytest.mark.parametrize("groups", [1, 2, 3, 5, 6, 7, 8, 16])
@pytest.mark.parametrize("kv_heads", [1, 2, 8])
def test_plan_covers_every_row_and_key_once_per_group_size(groups, kv_heads):
    """Items of (8 / hpw) * floor(32 / G) nodes: 256 nodes at G = 1 down to 16 at G = 16
    (48 at G = 5), and the two-head form for trees up to half that."""
    prefixes = [0, 1, 63, 64, 65, 255, 256, 257, 4096, 300, 9000]
    counts = [1, 2, 16, 17, 32, 33, 64, 65, 512, 129, 256]
    for chunk in (0, 64):
        check_plan_covers(prefixes, counts, kv_heads, 256, chunk, groups=groups)


MAX_CHUNK_PAGES = 512   # page numbers one work item caches in LDS


@pytest.mark.parametrize("block", [32, 96, 256])
def test_plan_chunks_fit_the_page_cache(block):
    """However long a prefix and however much work per compute unit, no item's prefix range
    spans more than the 512 page numbers a workgroup caches, wherever the range starts; with
    few compute units the cap is what bounds the chunks."""
    prefixes = [200000, 70000, 511 * block, 511 * block + 1, 5, 0]
    counts = [16, 64, 1, 32, 8, 3]
    for cus in (1, 8, 256):
        plan = check_plan_covers(prefixes, counts, 2, cus, block=block)
        spans = [((kend - 1) // block - kbeg // block + 1) if kend > kbeg else 0
                 for _, _, _, kbeg, kend, _, _, _ in plan["items"].tolist()]
        assert max(spans) <= MAX_CHUNK_PAGES
        if cus == 1:
            assert max(spans) >= MAX_CHUNK_PAGES - 1, "the page cap binds when each unit has long work"


def _slot_plan_items(prefix, nodes, kv_heads, groups, cus):
    lib = _lib.library()
    prefixes, counts, info = (ctypes.c_int32 * 1)(prefix), (ctypes.c_int32 * 1)(nodes), _lib.PlanInfo()
    _lib.check(lib.tv_tree_attention_plan_slots(prefixes, counts, 1, kv_heads, groups, cus, 0, None, None,
                                                ctypes.byref(info)), "plan_slots")
    items = np.zeros((max(info.num_items, 1), 8), dtype=np.int32)
    merges = np.zeros((max(info.num_groups, 1), 8), dtype=np.int32)
    _lib.check(lib.tv_tree_attention_plan_slots(prefixes, counts, 1, kv_heads, groups, cus, 0,
                                                items.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                                merges.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                                ctypes.byref(info)), "plan_slots")
    return items[:info.num_items]


@pytest.mark.parametrize("prefix,nodes,kv_heads,groups,same", [
    (5000, 16, 2, 4, True), (9000, 64, 2, 4, True), (9000, 200, 8, 16, False), (5000, 1024, 8, 8, False)])
def test_slot_plan_caps_prefix_chunks(prefix, nodes, kv_heads, groups, same):
    """The slot-addressed plan (the legacy entry) caches at most 2048 prefix slots per item;
    the page plan's cap is 511 pages.  Where the page plan would give a chunk longer than
    2048 keys (few, long work items: one request with many heads and nodes) the two split the
    prefix differently, so the legacy entry then equals the packed exact entry only within
    rounding, not byte for byte; elsewhere the two plans are the same item for item."""
    slot_items = _slot_plan_items(prefix, nodes, kv_heads, groups, 256)
    assert int((slot_items[:, 4] - slot_items[:, 3]).max()) <= 2048
    page_items = make_plan([prefix], [nodes], kv_heads, 256, 256, queries_per_kv=groups)["items"]
    key = lambda items: sorted(map(tuple, items[:, :5].tolist()))
    assert (key(slot_items) == key(page_items)) == same
    if not same:
        assert int((page_items[:, 4] - page_items[:, 3]).max()) > 2048


@pytest.mark.parametrize("prefixes,counts,kv_heads", [
    ([512, 3000], [2048, 16], 8), ([0], [1500], 2), ([9000, 100], [1025, 2048], 1)])
def test_plan_covers_trees_up_to_2048_nodes(prefixes, counts, kv_heads):
    """Page-table plans take trees of up to 2048 nodes (the kernel caches that many tree slots
    beside 512 page numbers); the slot-addressed plan keeps 1024, its LDS also holding 2048
    prefix slots."""
    check_plan_covers(prefixes, counts, kv_heads, 256)


def test_plan_rejects_trees_beyond_its_slot_caches():
    lib = _lib.library()
    info = _lib.PlanInfo()

    def plan(entry, nodes):
        prefixes, counts = (ctypes.c_int32 * 1)(64), (ctypes.c_int32 * 1)(nodes)
        if entry == "page":
            return lib.tv_tree_attention_plan(prefixes, counts, 1, 8, 4, 256, 256, 0, None, None, ctypes.byref(info))
        return lib.tv_tree_attention_plan_slots(prefixes, counts, 1, 8, 4, 256, 0, None, None, ctypes.byref(info))

    assert plan("page", 2048) == _lib.TV_OK and info.ancestor_words_per_row == 32
    assert plan("page", 2049) == _lib.TV_ERR_UNSUPPORTED and b"2049 tree nodes" in lib.tv_last_error()
    assert plan("slots", 1024) == _lib.TV_OK
    assert plan("slots", 1025) == _lib.TV_ERR_UNSUPPORTED
    assert _capacity(lib, (2048, 7), 8, 256, 256, 0, 20000).ancestor_words_per_row == 32
    with pytest.raises(ValueError):
        _capacity(lib, (2049,), 8, 256, 256, 0, 20000)
    assert _capacity_packed(lib, (2048, 1), 8, 256, 256, 0, 20000).ancestor_words_per_row == 32


def test_plan_at_benchmark_shapes():
    rng = np.random.default_rng(4)
    prefixes = [int(x) for x in rng.integers(8192, 32769, size=64)]
    plan = check_plan_covers(prefixes, [64] * 64, 8, 256)
    assert plan["num_groups"] == 0, "long contexts fill the chip without split-K"
    rng = np.random.default_rng(2)
    prefixes = [int(x) for x in rng.integers(256, 4097, size=8)]
    plan = check_plan_covers(prefixes, [16, 32, 64, 16, 32, 64, 16, 32], 8, 256)
    assert plan["num_items"] >= 128, "short batches are split to occupy the chip"


def test_plan_keeps_blocks_sharing_kv_on_one_xcd():
    """Node blocks that stream the same K/V (same request, head group, prefix chunk) are
    placed on one XCD (workgroup index mod 8) so they share its L2; trees of one block
    keep the plain longest-first order."""
    rng = np.random.default_rng(5)
    prefixes = [int(x) for x in rng.integers(0, 16385, size=16)] + [int(x) for x in rng.integers(2048, 8193, size=32)]
    counts = [512] * 16 + [32] * 32
    plan = check_plan_covers(prefixes, counts, 8, 256)
    streams = {}
    for index, (r, h0, _, kbeg, _, _, _, _) in enumerate(plan["items"].tolist()):
        streams.setdefault((r, h0, kbeg), set()).add(index % 8)
    multi = [xcds for key, xcds in streams.items() if counts[key[0]] > 64]
    assert multi and all(len(x) == 1 for x in multi)
    plain = make_plan([9000 + 37 * i for i in range(64)], [64] * 64, 8, 256, 256, queries_per_kv=4)
    lengths = [kend - kbeg for (_, _, _, kbeg, kend, _, _, _) in plain["items"].tolist()]
    assert lengths == sorted(lengths, reverse=True)



def simulated_makespan(plan, counts, cus=256):
    """Greedy list schedule of the plan's items in order onto `cus` CUs (8 XCDs, item i
    on XCD i % 8), in 32-key tiles: the finish time of the last CU."""
    import heapq
    per_xcd = [[0] * (cus // 8) for _ in range(8)]
    for index, (r, _, _, kbeg, kend, flags, _, hpw) in enumerate(plan["items"].tolist()):
        tiles = (kend - kbeg + 31) // 32 + ((counts[r] + 31) // 32 if flags & 1 else 0)
        heap = per_xcd[index % 8]
        heapq.heapreplace(heap, heap[0] + COST_WEIGHT[hpw] / 4 * tiles)
    return max(max(h) for h in per_xcd)


def test_plan_fills_its_rounds_of_work_items():
    """A one-KV-head shard of the benchmark batch: the first chunking gives 288 items for
    256 CUs, so the chunk target is refitted to fill two whole rounds (<= 512 items); the
    last CU then finishes close to the average load instead of ~1.7x it."""
    rng = np.random.default_rng(4)
    prefixes = [int(x) for x in rng.integers(8192, 32769, size=64)]
    plan = check_plan_covers(prefixes, [64] * 64, 1, 256)
    assert 256 < plan["num_items"] <= 512
    tiles = sum((p + 31) // 32 + 2 for p in prefixes)
    assert simulated_makespan(plan, [64] * 64) < 1.1 * tiles / 256
    # More than 4 rounds of items (or a forced chunk length) is left as first chunked.
    rng = np.random.default_rng(5)
    prefixes = [int(x) for x in rng.integers(0, 16385, size=16)] + [int(x) for x in rng.integers(2048, 8193, size=32)]
    plan = make_plan(prefixes, [512] * 16 + [32] * 32, 8, 256, 256, queries_per_kv=4)
    assert plan["num_items"] == 1152 and plan["num_groups"] == 0


def test_split_prefix_last_chunk_ends_level_with_the_others():
    """The last chunk of a split prefix also walks the tree (two prefix keys' worth per node).
    Within the chunk count the prefix alone gives, the chunks are cut so that the last one,
    with its tree, is at most a 32-key step longer than the others, unless lengthening the
    others by that step would leave the last chunk no prefix keys (the count would change)."""
    rng = np.random.default_rng(12)
    checked = 0
    for _ in range(200):
        count = int(rng.integers(1, 12))
        prefixes = [int(x) for x in rng.integers(0, 6000, size=count)]
        nodes = [int(x) for x in rng.choice([1, 16, 32, 64, 100, 512], size=count)]
        plan = make_plan(prefixes, nodes, 8, 256, 256, queries_per_kv=4)
        for r, (p, t) in enumerate(zip(prefixes, nodes)):
            items = plan["items"][(plan["items"][:, 0] == r) & (plan["items"][:, 1] == 0) & (plan["items"][:, 2] == 0)]
            if len(items) < 2:
                continue
            lengths = sorted({int(e - b) for b, e, f in zip(items[:, 3], items[:, 4], items[:, 5]) if not f & 1})
            last = [int(e - b) for b, e, f in zip(items[:, 3], items[:, 4], items[:, 5]) if f & 1]
            assert len(lengths) == 1 and len(last) == 1, (p, t)
            chunk, nc = lengths[0], len(items)
            assert chunk % 32 == 0 and 1 <= last[0] <= chunk and (nc - 1) * chunk + last[0] == p
            # Equal chunks alone would give ceil(p / nc) rounded up to 32; the tree moves keys off the last.
            assert chunk >= (p + nc - 1) // nc
            assert last[0] + 2 * t <= chunk + 32 or (nc - 1) * (chunk + 32) >= p, (p, t, chunk, last)
            checked += 1
    assert checked > 100


def _capacity(lib, counts, kv_heads, block, cus, chunk, max_prefix, groups=4):
    info = _lib.PlanInfo()
    arr = (ctypes.c_int32 * len(counts))(*counts)
    _lib.check(lib.tv_tree_attention_plan_capacity(arr, len(counts), kv_heads, groups, block, cus, chunk, max_prefix,
                                                   ctypes.byref(info)), "capacity")
    return info


def _capacity_packed(lib, counts, kv_heads, block, cus, chunk, max_prefix, groups=4):
    info = _lib.PlanInfo()
    _lib.check(lib.tv_tree_attention_plan_capacity_packed(sum(counts), len(counts), sum(n * n for n in counts),
                                                          kv_heads, groups, block, cus, chunk, max_prefix,
                                                          ctypes.byref(info)), "capacity_packed")
    return info


def test_signature_capacity_covers_every_node_count_vector():
    """The capture-mode capacity depends only on (requests, rows, sum of squares) and must
    cover the exact capacity of every node-count vector with that signature: checked on
    seeded random vectors and on pairs that share a signature."""
    lib = _lib.library()
    rng = np.random.default_rng(3)
    vectors = [(12, 60, 72), (24, 36, 84), (1, 5, 6), (2, 3, 7), (64,) * 64, (1024,), (1, 1024), (33, 31),
               (2048,), (2048, 1), (1500, 600)]
    for _ in range(3000):
        count = int(rng.integers(1, 9))
        high = int(rng.choice([40, 130, 300, 1024, 2048]))
        vectors.append(tuple(int(x) for x in rng.integers(1, high + 1, size=count)))
    cases = [(8, 0, 4), (1, 0, 4), (2, 0, 4), (8, 2048, 4), (8, 0, 1), (2, 0, 16), (1, 0, 8), (8, 2048, 2),
             (8, 0, 5), (2, 0, 7), (1, 2048, 3)]
    for counts in vectors:
        for kv_heads, chunk, groups in cases:
            where = (counts, kv_heads, chunk, groups)
            try:
                exact = _capacity(lib, counts, kv_heads, 256, 256, chunk, 20000, groups)
            except ValueError:   # beyond the device planner: the signature bound must refuse too
                with pytest.raises(ValueError):
                    _capacity_packed(lib, counts, kv_heads, 256, 256, chunk, 20000, groups)
                continue
            try:
                packed = _capacity_packed(lib, counts, kv_heads, 256, 256, chunk, 20000, groups)
            except ValueError as error:   # the class bound may exceed the planner: a refusal, never a short plan
                assert "exceed" in str(error)
                continue
            assert packed.num_items >= exact.num_items, where
            assert packed.num_groups >= exact.num_groups, where
            assert packed.num_partial_slots >= exact.num_partial_slots, where
            assert packed.ancestor_words_per_row >= exact.ancestor_words_per_row, where
            assert packed.workspace_bytes >= exact.workspace_bytes, where
    # (12, 60, 72) and (24, 36, 84) share a signature; so do (1, 5, 6) and (2, 3, 7).
    a = _capacity_packed(lib, (12, 60, 72), 8, 256, 256, 0, 8192)
    b = _capacity_packed(lib, (24, 36, 84), 8, 256, 256, 0, 8192)
    assert (a.num_items, a.num_groups, a.ancestor_words_per_row) == (b.num_items, b.num_groups,
                                                                      b.ancestor_words_per_row)
    info = _lib.PlanInfo()
    assert lib.tv_tree_attention_plan_capacity_packed(2, 3, 0, 8, 4, 256, 256, 0, 100, ctypes.byref(info)) \
        == _lib.TV_ERR_INVALID   # fewer rows than requests


def test_stream_capture_info_rejects_null_outputs():
    lib = _lib.library()
    assert lib.tv_stream_capture_info(None, None, None) == _lib.TV_ERR_INVALID
