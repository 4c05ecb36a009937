"""Pins the CPU oracle before any kernel is judged against it (CPU only).

Every oracle function is checked against something it does not compute itself:
  * the reference's own known answers (tests/golden/reference_kats.json),
  * closed forms (constant V, zero query, a single visible key),
  * an independent brute force: fp64 attention over keys gathered by walking the
    parent chain, never reading qq_bias or page tables (the reference's own oracle
    design, benchmarks/jetspec_tree_kernel_qualification.py:165-190),
  * planted mistakes: the same checks run on a deliberately wrong oracle input and
    must fail, which shows that a dropped scale, swapped K/V, ignored mask or wrong
    GQA mapping cannot pass unnoticed.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
import pytest

import oracle
from oracle import cpu_path
from jetspec_amd import workloads

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def softmax(x):
    e = np.exp(np.asarray(x, dtype=np.float64) - np.max(x))
    return e / e.sum()


# ----------------------------------------------------------------------------- fp64 attention
def gqa_kat_expected():
    kat = KATS["fp64_attention_gqa"]
    v = np.asarray(kat["v"], dtype=np.float64)
    p0 = softmax([1.0, 0.0])
    p1 = softmax([0.0, 2.0])
    return np.stack((p0[0] * v[0, 0] + p0[1] * v[1, 0],
                     p0[1] * v[0, 0] + p0[0] * v[1, 0],
                     p1[0] * v[0, 1] + p1[1] * v[1, 1],
                     (v[0, 1] + v[1, 1]) / 2))


def test_fp64_attention_matches_hand_computed_gqa_kat():
    kat = KATS["fp64_attention_gqa"]
    out = oracle.fp64_attention(kat["q"], kat["k"], kat["v"], kat["scale"], kat["groups"])
    np.testing.assert_allclose(out, gqa_kat_expected(), rtol=0, atol=kat["tolerance"])


def test_fp64_attention_rejects_bad_geometry_and_nonfinite():
    q = np.ones((2, 4))
    k = np.ones((3, 1, 4))
    for args in ((q, k, k, 1.0, 1), (q, k[:0], k[:0], 1.0, 2), (q, k, k, float("inf"), 2),
                 (q, k * np.nan, k, 1.0, 2)):
        with pytest.raises(ValueError):
            oracle.fp64_attention(*args)


def paged_kat_instance(block_size=16):
    """The GQA KAT as a paged problem: one prefix key in page 3, the root node in page 1."""
    kat = KATS["fp64_attention_gqa"]
    k_src, v_src = np.asarray(kat["k"], np.float32), np.asarray(kat["v"], np.float32)
    k = np.full((4, block_size, 2, 2), np.nan, np.float32)
    v = np.full_like(k, np.nan)
    k[3, 0], v[3, 0] = k_src[0], v_src[0]          # prefix position 0 -> page 3
    k[1, 5], v[1, 5] = k_src[1], v_src[1]          # tree node 0 -> slot 1*16+5
    meta = oracle.metadata_arrays([1], [[3]], [[1 * block_size + 5]], [np.ones((1, 1), bool)], block_size)
    q = np.asarray(kat["q"], np.float32)[None]
    return q, k, v, meta, kat


def test_paged_oracle_reproduces_gqa_kat():
    q, k, v, meta, kat = paged_kat_instance()
    out = oracle.tree_attention_f64(q, k, v, scale=kat["scale"], **meta)
    np.testing.assert_allclose(out[0], gqa_kat_expected(), rtol=0, atol=1e-7)


@pytest.mark.parametrize("mistake", ["scale", "swap_kv", "groups"])
def test_planted_mistakes_fail_the_paged_kat(mistake):
    q, k, v, meta, kat = paged_kat_instance()
    scale = kat["scale"]
    if mistake == "scale":
        scale = scale * 1.01
    if mistake == "swap_kv":
        k, v = v, k
    if mistake == "groups":  # heads mapped to the wrong KV head: interleave instead of block
        q = q[:, [0, 2, 1, 3]]
    out = oracle.tree_attention_f64(q, k, v, scale=scale, **meta)
    assert not np.allclose(out[0], gqa_kat_expected(), rtol=0, atol=1e-7)


def random_case(seed, prefixes, counts, kv_heads=2, groups=4, head_dim=16, block=16):
    rng = np.random.default_rng(seed)
    parents = [workloads.random_parents(n, 4, rng) for n in counts]
    pages_needed = [-(-p // block) for p in prefixes]
    scratch_pages = -(-sum(counts) // block) + 1
    total = sum(pages_needed) + scratch_pages + 2
    order = rng.permutation(total)
    tables, cursor = [], 0
    for n in pages_needed:
        tables.append([int(x) for x in order[cursor:cursor + n]])
        cursor += n
    scratch = order[cursor:cursor + scratch_pages]
    slots_all = (scratch[:, None] * block + np.arange(block)).reshape(-1)
    slots_all = slots_all[rng.permutation(slots_all.size)]
    slots, off = [], 0
    for n in counts:
        slots.append(slots_all[off:off + n].tolist())
        off += n
    masks = [oracle.mask_from_parents(p) for p in parents]
    meta = oracle.metadata_arrays(prefixes, tables, slots, masks, block)
    k = rng.standard_normal((total, block, kv_heads, head_dim)).astype(np.float32)
    v = rng.standard_normal((total, block, kv_heads, head_dim)).astype(np.float32)
    q = rng.standard_normal((sum(counts), kv_heads * groups, head_dim)).astype(np.float32)
    return dict(q=q, k=k, v=v, meta=meta, tables=tables, slots=slots, parents=parents, prefixes=prefixes,
                counts=counts, groups=groups, block=block, scale=head_dim ** -0.5)


def parent_chain_reference(case):
    """Independent brute force: visible keys = prefix positions + parent chain."""
    out = np.zeros(case["q"].shape, np.float64)
    row = 0
    block = case["block"]
    for r, (prefix, count) in enumerate(zip(case["prefixes"], case["counts"])):
        prefix_slots = [case["tables"][r][p // block] * block + p % block for p in range(prefix)]
        for node in range(count):
            chain = oracle.parent_chain(case["parents"][r], node)
            slots = np.asarray(prefix_slots + [case["slots"][r][j] for j in chain], dtype=np.int64)
            kk = case["k"].reshape(-1, *case["k"].shape[2:])[slots]
            vv = case["v"].reshape(-1, *case["v"].shape[2:])[slots]
            out[row] = oracle.fp64_attention(case["q"][row], kk, vv, case["scale"], case["groups"])
            row += 1
    return out


@pytest.mark.parametrize("seed,prefixes,counts", [
    (0, [0], [1]), (1, [1, 0, 2], [3, 2, 3]), (2, [17, 63, 64, 65], [5, 8, 1, 7]),
    (3, [255, 256, 257], [12, 9, 16]), (4, [300, 31], [20, 13]),
])
def test_paged_oracle_equals_parent_chain_brute_force(seed, prefixes, counts):
    case = random_case(seed, prefixes, counts)
    out = oracle.tree_attention_f64(case["q"], case["k"], case["v"], scale=case["scale"], **case["meta"])
    np.testing.assert_allclose(out, parent_chain_reference(case), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("groups,kv_heads", [(1, 3), (2, 2), (5, 2), (8, 2), (16, 1)])
def test_paged_oracle_equals_brute_force_at_every_group_size(groups, kv_heads):
    """Query head h reads KV head h // G (block grouping) for every G the kernel takes."""
    case = random_case(11 + groups, [70, 0, 33], [9, 5, 12], kv_heads=kv_heads, groups=groups)
    out = oracle.tree_attention_f64(case["q"], case["k"], case["v"], scale=case["scale"], **case["meta"])
    np.testing.assert_allclose(out, parent_chain_reference(case), rtol=1e-10, atol=1e-12)


def test_planted_ignored_mask_fails_brute_force():
    case = random_case(5, [40, 9], [12, 10])
    meta = dict(case["meta"])
    meta["qq_bias"] = np.zeros_like(meta["qq_bias"])  # drops the ancestor mask: siblings leak in
    out = oracle.tree_attention_f64(case["q"], case["k"], case["v"], scale=case["scale"], **meta)
    assert not np.allclose(out, parent_chain_reference(case), rtol=1e-6, atol=1e-9)


def test_closed_forms():
    case = random_case(6, [33, 0], [9, 6])
    meta = case["meta"]
    # constant V rows: every convex combination is that constant
    v_const = np.broadcast_to(np.arange(case["v"].shape[-1], dtype=np.float32), case["v"].shape).copy()
    out = oracle.tree_attention_f64(case["q"], case["k"], v_const, scale=case["scale"], **meta)
    np.testing.assert_allclose(out, np.broadcast_to(v_const[0, 0, 0], out.shape), rtol=0, atol=1e-12)
    # zero query: uniform average over the visible keys
    q0 = np.zeros_like(case["q"])
    out = oracle.tree_attention_f64(q0, case["k"], case["v"], scale=case["scale"], **meta)
    ref = parent_chain_reference(dict(case, q=q0))
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    # the root row of a request without prefix sees only itself
    root = meta["cu_seqlens_q"][1]
    slot = case["slots"][1][0]
    v_root = case["v"].reshape(-1, *case["v"].shape[2:])[slot]
    out = oracle.tree_attention_f64(case["q"], case["k"], case["v"], scale=case["scale"], **meta)
    np.testing.assert_allclose(out[root], np.repeat(v_root, case["groups"], axis=0), rtol=0, atol=1e-7)


def test_torch_cpu_path_agrees_with_fp64_oracle():
    import torch
    case = random_case(7, [70, 5], [11, 4], head_dim=32)
    meta = case["meta"]
    q, k, v = (torch.from_numpy(case[x]) for x in ("q", "k", "v"))
    out64 = oracle.tree_attention_f64(case["q"], case["k"], case["v"], scale=case["scale"], **meta)
    row = 0
    for r, (prefix, count) in enumerate(zip(case["prefixes"], case["counts"])):
        got = cpu_path.request_attention(q[row:row + count], k, v, case["tables"][r], prefix,
                                         torch.tensor(case["slots"][r]),
                                         torch.from_numpy(oracle.mask_from_parents(case["parents"][r])),
                                         case["scale"], torch.float32)
        np.testing.assert_allclose(got.numpy(), out64[row:row + count], rtol=0, atol=2e-6)
        row += count


# ----------------------------------------------------------------------------- tree helpers
def test_parent_chain_kats():
    for entry in KATS["parent_chain"]["valid"]:
        assert oracle.parent_chain(entry["parents"], entry["node"]) == entry["chain"]
    for entry in KATS["parent_chain"]["invalid"]:
        with pytest.raises(ValueError):
            oracle.parent_chain(entry["parents"], entry["node"])


def test_mask_from_parents_matches_generator_and_heap_rule():
    heap = [-1] + [(n - 1) // 2 for n in range(1, 63)]
    mask = oracle.mask_from_parents(heap)
    for node in range(63):
        chain, cur = [], node
        while cur >= 0:
            chain.append(cur)
            cur = (cur - 1) // 2 if cur else -1
        assert sorted(np.flatnonzero(mask[node]).tolist()) == sorted(chain)
    rng = np.random.default_rng(3)
    for n in (1, 2, 31, 64):
        parents = workloads.random_parents(n, 8, rng)
        assert np.array_equal(workloads.ancestor_mask(parents), oracle.mask_from_parents(parents))


# ----------------------------------------------------------------------------- store / commit
def test_store_kvcache_oracle_matches_index_assignment_and_skips_minus_one():
    rng = np.random.default_rng(8)
    key = rng.standard_normal((9, 2, 4)).astype(np.float32)
    value = rng.standard_normal((9, 2, 4)).astype(np.float32)
    k_cache = rng.standard_normal((3, 16, 2, 4)).astype(np.float32)
    v_cache = k_cache.copy() + 1
    slots = np.array([5, -1, 17, 40, -1, 0, 47, 33, 2])
    expect_k, expect_v = k_cache.copy(), v_cache.copy()
    keep = slots != -1
    expect_k.reshape(-1, 2, 4)[slots[keep]] = key[keep]
    expect_v.reshape(-1, 2, 4)[slots[keep]] = value[keep]
    oracle.store_kvcache(key, value, k_cache, v_cache, slots)
    assert np.array_equal(k_cache, expect_k) and np.array_equal(v_cache, expect_v)


def test_copy_accepted_kv_oracle_bytes_kats():
    for entry in KATS["kv_copy_bytes"]:
        dtype = {2: np.float16, 4: np.float32}[entry["elem_bytes"]]
        pool = np.zeros((2, entry["layers"], 4, 16, entry["kv_heads"], entry["head_dim"]), dtype)
        n = entry["rows"]
        src = np.arange(n)
        dst = np.arange(32, 32 + n)
        assert oracle.copy_accepted_kv(pool, src, dst) == entry["expected"]


def test_copy_accepted_kv_oracle_is_gather_then_scatter():
    import torch
    rng = np.random.default_rng(9)
    pool = rng.standard_normal((2, 3, 6, 16, 2, 4)).astype(np.float32)
    src = np.array([3, 70, 41, 8, 90])
    dst = np.array([8, 71, 3, 20, 41])        # overlaps: 8, 3 and 41 are both read and written
    expect = torch.from_numpy(pool.copy())
    cpu_path.copy_accepted_kv(expect, torch.from_numpy(src), torch.from_numpy(dst), 16)
    got = pool.copy()
    oracle.copy_accepted_kv(got, src, dst)
    assert np.array_equal(got, expect.numpy())
    # a naive in-order row copy differs on this overlap, so staging is observable
    naive = pool.copy()
    flat = naive.reshape(2, 3, -1, 2, 4)
    for s, d in zip(src, dst):
        flat[:, :, d] = flat[:, :, s]
    assert not np.array_equal(naive, got)


def _enumerated_slots(pages, block_size):
    """Canonical slots by walking the page list one page at a time (no div/mod)."""
    return [page * block_size + offset for page in pages for offset in range(block_size)]


def test_commit_slots_oracle_hand_kat():
    # Pages [7, 3], 4-slot pages, 3 positions cached: the next three positions 3, 4, 5
    # land at 7*4+3, then 3*4+0 and 3*4+1; node slots come from the tree's scratch slots.
    src, dst, bad = oracle.commit_slots([90, 91, 92, 93], [0, 4], [0, 2, 3], [0, 3], [[7, 3]], [3], 4, 8)
    assert dst.tolist() == [31, 12, 13] and src.tolist() == [90, 92, 93] and not bad.any()


def test_commit_slots_oracle_matches_enumeration_and_rejects_reference_errors():
    # state.py:770-773 rejects an empty path, a path not rooted at 0, repeated nodes and
    # nodes outside the tree; the other requests of the batch are unaffected.
    rng = np.random.default_rng(17)
    block, requests = 16, 6
    tables = rng.permutation(64)[:requests * 5].reshape(requests, 5)
    lens = rng.integers(0, 50, size=requests)
    counts = rng.integers(1, 12, size=requests)
    cu = np.concatenate([[0], np.cumsum(counts)])
    tree_slots = rng.permutation(4096)[:cu[-1]] + 2000
    paths, offsets = [], [0]
    for r in range(requests):
        depth = int(rng.integers(1, counts[r] + 1))
        paths += [0] + sorted(rng.permutation(np.arange(1, counts[r]))[:depth - 1].tolist())
        offsets.append(len(paths))
    src, dst, bad = oracle.commit_slots(tree_slots, cu, paths, offsets, tables, lens, block, 64)
    assert not bad.any()
    for r in range(requests):
        rows = slice(offsets[r], offsets[r + 1])
        n = offsets[r + 1] - offsets[r]
        assert dst[rows].tolist() == _enumerated_slots(tables[r], block)[lens[r]:lens[r] + n]
        assert src[rows].tolist() == [tree_slots[cu[r] + x] for x in paths[rows]]
    for broken in ([1, 0], [0, 0], [0, counts[1]], [0, -1]):
        p = list(paths[:offsets[1]]) + broken + list(paths[offsets[2]:])
        o = [0, offsets[1], offsets[1] + len(broken)] + [x - (offsets[2] - offsets[1]) + len(broken)
                                                          for x in offsets[3:]]
        s2, d2, b2 = oracle.commit_slots(tree_slots, cu, p, o, tables, lens, block, 64)
        assert b2.tolist() == [False, True] + [False] * (requests - 2)
        assert (s2[o[1]:o[2]] == -1).all() and (d2[o[1]:o[2]] == -1).all()
        assert np.array_equal(d2[:o[1]], dst[:offsets[1]]) and np.array_equal(d2[o[2]:], dst[offsets[2]:])
    # past the table row, and a page outside the pool
    _, _, b3 = oracle.commit_slots(tree_slots, cu, paths, offsets, tables, [5 * block - 1] + list(lens[1:]), block, 64)
    assert b3[0] == (offsets[1] - offsets[0] > 1) and not b3[1:].any()
    t4 = tables.copy(); t4[2, :] = 64
    _, _, b4 = oracle.commit_slots(tree_slots, cu, paths, offsets, t4, lens, block, 64)
    assert b4.tolist() == [r == 2 for r in range(requests)]


# ----------------------------------------------------------------------------- acceptance / metrics
def test_accept_walk_duplicate_sibling_kat():
    kat = KATS["accept_duplicate_siblings"]
    greedy = [0] * len(kat["tokens"])
    for node, token in kat["forced_argmax"].items():
        greedy[int(node)] = token
    result = oracle.accept_walk(greedy, kat["tokens"], kat["depths"],
                                oracle.child_maps(kat["tokens"], kat["parents"]), kat["max_depth"])
    assert result["path"] == kat["expected_path"]
    assert result["outputs"][:-1] == [kat["tokens"][n] for n in kat["expected_path"][1:]]
    assert result["correction"] == greedy[kat["expected_path"][-1]]


def test_argmax_flip_witness_kats():
    kat = KATS["argmax_flip_witness"]["near_tie"]
    result = oracle.argmax_flip_witness(kat["actual"], kat["reference"])
    assert result["argmax_flips"] == kat["flips"] and result["large_margin_violations"] == kat["violations"]
    ties = KATS["argmax_flip_witness"]["first_index_ties"]
    assert int(np.argmax(ties["actual"])) == ties["actual_argmax"]
    assert int(np.argmax(ties["reference"])) == ties["reference_argmax"]
    result = oracle.argmax_flip_witness([ties["actual"]], [ties["reference"]])
    assert result["argmax_flips"] == 1 and result["large_margin_violations"] == 0


# ----------------------------------------------------------------------------- output truncation
def test_truncate_oracle_reference_kats():
    # tests/test_jetspec_batch_runtime.py:167-172: chain tree from token 9, every node
    # accepted (the fixture's logits predict token + 1), EOS {11}: outputs [10, 11] and
    # two cached rows (cache_len grows by 2, from prompt_length - 1 to prompt_length + 1).
    cut = oracle.truncate_accepted([10, 11, 12], [0, 1, 2], 16, False, {11})
    assert cut == {"limit": 2, "emitted": [10, 11], "path": [0, 1]}
    # tests/test_jetspec_chunked_scheduler.py:310-316: the "ignore" request (max_new_tokens
    # 4, ignore_eos) emits 5 at prefill, then [6, 7, 8] in one round: budget 3 keeps all.
    assert oracle.truncate_accepted([6, 7, 8], [0, 1, 2], 3, True, {5})["emitted"] == [6, 7, 8]
    # The budget cut without EOS, an EOS on the correction, and ignore_eos past an EOS.
    assert oracle.truncate_accepted([6, 7, 8], [0, 1, 2], 2, False, {5}) == {"limit": 2, "emitted": [6, 7],
                                                                             "path": [0, 1]}
    assert oracle.truncate_accepted([1, 2, 63], [0, 4, 9], 16, False, {63})["limit"] == 3
    assert oracle.truncate_accepted([63, 2], [0, 3], 16, True, {63})["limit"] == 2
    assert oracle.truncate_accepted([63, 2], [0, 3], 16, False, {63})["limit"] == 1
    with pytest.raises(ValueError):
        oracle.truncate_accepted([1, 2], [0], 4, False, set())


# ---------------------------------------------------------------- numerical_metrics
def test_numerical_metrics_closed_forms():
    """jetspec_numeric_oracles.py:108-168 restated: identity, a constant offset (every error
    statistic known in closed form), and the fixed bound's conjunction on both sides."""
    rng = np.random.default_rng(11)
    ref = rng.standard_normal((4, 32, 128))
    same = oracle.numerical_metrics(ref.copy(), ref)
    assert same["max_abs_error"] == 0 and same["rms_error"] == 0 and same["relative_rms_error"] == 0
    assert same["within_fixed_bound"] and same["fixed_bound_applicable"]
    ref_rms = float(np.sqrt(np.mean(ref ** 2)))
    for c in (1e-6, 5e-5, 3e-3):
        m = oracle.numerical_metrics(ref + c, ref)
        assert m["max_abs_error"] == pytest.approx(c, rel=1e-9)
        assert m["rms_error"] == pytest.approx(c, rel=1e-9)
        assert m["relative_rms_error"] == pytest.approx(c / ref_rms, rel=1e-9)   # over the REFERENCE's RMS
        bound = 1e-4 * max(1.0, float(np.abs(ref).max()))
        assert m["within_fixed_bound"] == (c <= bound and c / ref_rms <= 1e-4)
    # Scaling the actual alone must not change the denominator.
    m = oracle.numerical_metrics(2 * ref, ref)
    assert m["relative_rms_error"] == pytest.approx(1.0, rel=1e-12)
    assert oracle.numerical_metrics(np.zeros(3), np.zeros(3))["relative_rms_error"] == 0.0
    assert oracle.numerical_metrics(np.ones(3), np.zeros(3))["relative_rms_error"] == float("inf")
    with pytest.raises(ValueError):
        oracle.numerical_metrics(np.zeros(3), np.zeros(4))


def test_numerical_metrics_bf16_ulps_against_torch():
    """The bf16 diagnostics: the nearest bf16 value is torch's own float64 -> bfloat16
    conversion, the ULP is the larger of torch.nextafter's two neighbour spacings, and the
    hand-computed cases 1.0 (ULP 2^-7), 0.75 (2^-8) and 3.0 (2^-6) hold."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal(50000) * np.exp(rng.uniform(-30, 30, 50000))
    t = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(oracle.round_f64_to_bf16(x), t.double().numpy())
    up = torch.nextafter(t, torch.full_like(t, float("inf"))).double() - t.double()
    down = t.double() - torch.nextafter(t, torch.full_like(t, float("-inf"))).double()
    assert np.array_equal(oracle.bf16_ulp(t.double().numpy()), torch.maximum(up, down).numpy())
    ref = np.array([1.0, 0.75, 3.0])
    assert np.array_equal(oracle.bf16_ulp(ref), [2.0 ** -7, 2.0 ** -8, 2.0 ** -6])
    m = oracle.numerical_metrics(ref + np.array([2.0 ** -7, 0, 0]), ref, bf16_output=True)
    q = m["bf16_quantization"]
    assert q["max_error_in_bf16_ulps"] == 1.0 and q["nearest_bf16_unequal_elements"] == 1
    assert q["actual_output_is_bf16"] and not m["fixed_bound_applicable"]
