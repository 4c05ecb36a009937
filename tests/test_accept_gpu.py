"""Device greedy acceptance (tv_argmax_rows + tv_tree_accept) on the GPU.

The argmax must equal torch.argmax index for index (ties to the lower index, NaN
first), at the served shape (4096 tree rows x Qwen3's 151936-token vocabulary, bf16)
and on edge rows.  The walks must equal the oracle's host walk (restating
serving_ops.py:78-89) on random trees with duplicate sibling tokens, the reference's
duplicate-sibling KAT (tests/test_jetspec_serving_ops.py:39-58), depth truncation,
and must raise on a path that leaves the canonical depths.
"""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import (accept_batch, accept_batch_device, commit_slots, greedy_argmax, read_and_clear_status,
                         truncate_accepted, workloads)

pytestmark = pytest.mark.gpu
DEV = "cuda"
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(1, 1), (3, 7), (17, 1000), (64, 4099), (4096, 151936)])
def test_argmax_equals_torch(dtype, rows, vocab):
    print(f"[argmax] dtype={dtype} rows={rows} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + vocab)
    logits = torch.randn(rows, vocab, generator=g, device=DEV).to(dtype)
    got = greedy_argmax(logits)
    assert torch.equal(got, logits.argmax(-1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_edge_rows(dtype):
    vocab = 3001
    logits = torch.randn(18, vocab, device=DEV).to(dtype)
    logits[0] = 1.5                                        # all equal -> 0
    logits[1] = float("-inf")                              # all -inf -> 0
    logits[2, 17] = logits[2, 2000] = 1e4                  # tie -> lower index
    logits[3, 5] = float("nan")                            # NaN wins
    logits[4, 9] = logits[4, 3000] = float("nan")          # first NaN
    logits[4, 100] = float("inf")
    logits[5, 3000] = float("inf")                         # last element, the scalar tail
    logits[6] = 0.0
    logits[6, 2999] = -0.0
    logits[7, 1:] = -1.0
    logits[7, 0] = -0.5                                    # first element
    logits[8, 2048] = 7e3                                  # vector-unit boundary
    logits[9, 2047] = logits[9, 2049] = 7e3
    logits[10] = float("-inf")
    logits[10, 1234] = -3e38 if dtype == torch.float32 else -3.0e38
    logits[11, ::2] = 2.0                                  # many ties
    # The scan keeps one 16-byte unit per thread (8 bf16 or 4 fp32 elements) and resolves
    # the element inside it at the end: NaN and ties inside and across units.
    logits[12, 16], logits[12, 17] = 1e4, float("nan")     # NaN after the max in one unit
    logits[13, 24], logits[13, 25] = float("nan"), 1e4     # NaN before the max in one unit
    logits[14, 40], logits[14, 2500] = 1e4, float("nan")   # a later unit's NaN beats an earlier max
    logits[15] = -1.0
    logits[15, 8], logits[15, 800] = -0.0, 0.0             # -0 then +0: equal, the first wins
    logits[16] = -1.0
    logits[16, 8], logits[16, 800] = 0.0, -0.0             # +0 then -0
    logits[17, 15] = logits[17, 16] = 5e3                  # equal maxima in adjacent units
    got = greedy_argmax(logits)
    assert torch.equal(got, logits.argmax(-1))


def test_argmax_strided_rows():
    backing = torch.randn(40, 5003, device=DEV, dtype=torch.bfloat16)
    view = backing[::3, 1:4998]                            # unaligned start, row stride 3 * 5003
    assert torch.equal(greedy_argmax(view), view.argmax(-1))


def random_batch(rng, sizes, vocab=6, max_depth=8):
    trees, offsets = [], [0]
    for n in sizes:
        parents = workloads.random_parents(n, max_depth, rng)
        tokens = [int(t) for t in rng.integers(0, vocab, size=n)]
        depths = workloads.depths_of(parents)
        trees.append(SimpleNamespace(num_nodes=n, host_token_ids=tokens, host_parents=parents, host_depths=depths,
                                     child_maps=oracle.child_maps(tokens, parents),
                                     token_ids=torch.tensor(tokens, device=DEV),
                                     parent_indices=torch.tensor(parents, device=DEV),
                                     depth=torch.tensor(depths, device=DEV)))
        offsets.append(offsets[-1] + n)
    return trees, offsets


@pytest.mark.parametrize("max_depth", [0, 3, 15])
def test_walks_equal_oracle_walks(max_depth):
    rng = np.random.default_rng(11 + max_depth)
    sizes = [1, 2, 16, 31, 32, 64, 65, 200, 1024]
    trees, offsets = random_batch(rng, sizes)
    vocab = 6
    logits = torch.randn(offsets[-1], vocab, device=DEV)
    # Bias each node's argmax towards one of its children's tokens so walks go deep.
    for tree, lo in zip(trees, offsets):
        for node, children in enumerate(tree.child_maps):
            if children and rng.random() < 0.85:
                logits[lo + node, int(rng.choice(list(children)))] += 6.0
    results = accept_batch(logits, trees, offsets, max_depth)
    greedy = logits.argmax(-1).tolist()
    deepest = 0
    for i, tree in enumerate(trees):
        want = oracle.accept_walk(greedy[offsets[i]:offsets[i + 1]], tree.host_token_ids, tree.host_depths,
                                  tree.child_maps, max_depth)
        assert results[i] == want, f"request {i} ({sizes[i]} nodes)"
        deepest = max(deepest, want["accepted_length"])
    assert deepest >= min(max_depth, 3), "the biased logits should drive some walk deep"


def test_duplicate_sibling_kat_last_child_wins():
    kat = KATS["accept_duplicate_siblings"]
    tree = SimpleNamespace(token_ids=torch.tensor(kat["tokens"], device=DEV),
                           parent_indices=torch.tensor(kat["parents"], device=DEV),
                           depth=torch.tensor(kat["depths"], device=DEV), num_nodes=len(kat["tokens"]))
    logits = torch.randn(len(kat["tokens"]), 80, generator=torch.Generator().manual_seed(99)).to(DEV)
    for node, token in kat["forced_argmax"].items():
        logits[int(node), token] = 100
    result = accept_batch(logits, [tree], [0, len(kat["tokens"])], kat["max_depth"])[0]
    assert result["path"] == kat["expected_path"]
    assert result["accepted_length"] == len(kat["expected_path"]) - 1
    assert result["correction"] == int(logits[kat["expected_path"][-1]].argmax())


def test_device_outputs_without_host_walk():
    rng = np.random.default_rng(3)
    trees, offsets = random_batch(rng, [16, 64, 5])
    logits = torch.randn(offsets[-1], 6, device=DEV, dtype=torch.bfloat16)
    tokens = torch.cat([t.token_ids for t in trees])
    parents = torch.cat([t.parent_indices for t in trees]).to(torch.int32)
    depths = torch.cat([t.depth for t in trees])
    cu = torch.tensor(offsets, dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    greedy, paths, lengths, corrections = accept_batch_device(logits, tokens, parents, depths, cu, 15, status=status)
    assert torch.equal(greedy, logits.argmax(-1))
    host = greedy.tolist()
    for i, tree in enumerate(trees):
        want = oracle.accept_walk(host[offsets[i]:offsets[i + 1]], tree.host_token_ids, tree.host_depths,
                                  tree.child_maps, 15)
        n = want["accepted_length"] + 1
        assert paths[i, :n].tolist() == want["path"] and (paths[i, n:] == -1).all()
        assert int(lengths[i]) == want["accepted_length"] and int(corrections[i]) == want["correction"]
    assert int(status) == 0


def test_noncanonical_depth_raises():
    rng = np.random.default_rng(8)
    trees, offsets = random_batch(rng, [16])
    tree = trees[0]
    child = next(iter(tree.child_maps[0].values()))
    tree.host_depths = list(tree.host_depths)
    tree.host_depths[child] = 5                     # off its canonical depth 1
    logits = torch.full((16, 6), -1.0, device=DEV)
    logits[0, tree.host_token_ids[child]] = 1.0     # the walk takes that child
    with pytest.raises(RuntimeError, match="canonical tail"):
        accept_batch(logits, trees, offsets, 15)


def deep_accept_case(seed, sizes, max_depth=8, vocab=6):
    """Random trees whose logits favour a child's token, run through the device walk."""
    rng = np.random.default_rng(seed)
    trees, offsets = random_batch(rng, sizes, vocab=vocab, max_depth=max_depth)
    logits = torch.randn(offsets[-1], vocab, device=DEV)
    for tree, lo in zip(trees, offsets):
        for node, children in enumerate(tree.child_maps):
            if children and rng.random() < 0.9:
                logits[lo + node, int(rng.choice(list(children)))] += 6.0
    tokens = torch.cat([t.token_ids for t in trees])
    parents = torch.cat([t.parent_indices for t in trees])
    depths = torch.cat([t.depth for t in trees])
    cu = torch.tensor(offsets, dtype=torch.int32, device=DEV)
    _, paths, lengths, corrections = accept_batch_device(logits, tokens, parents, depths, cu, max_depth)
    return rng, trees, offsets, tokens, cu, paths, lengths, corrections


def expected_cuts(trees, paths, lengths, corrections, budgets, ignore, eos):
    cuts = []
    for i, tree in enumerate(trees):
        n = int(lengths[i])
        path = [int(x) for x in paths[i, :n + 1]]
        values = [tree.host_token_ids[x] for x in path[1:]] + [int(corrections[i])]
        cuts.append(oracle.truncate_accepted(values, path, int(budgets[i]), bool(ignore[i]), eos))
    return cuts


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_truncation_matches_oracle(seed):
    sizes = [[1, 5, 16, 32, 64], [3] * 40, [16, 200, 1024, 64, 7, 33] * 5][seed]
    rng, trees, offsets, tokens, cu, paths, lengths, corrections = deep_accept_case(100 + seed, sizes)
    r = len(sizes)
    budgets = torch.tensor(rng.integers(1, 12, size=r), dtype=torch.int32, device=DEV)
    ignore = torch.tensor(rng.random(r) < 0.3, device=DEV)
    eos = {int(x) for x in rng.choice(6, size=2, replace=False)}
    print(f"[truncate] seed={seed} requests={r} eos={sorted(eos)}", flush=True)
    limits, emitted, commit_paths, commit_offsets = truncate_accepted(paths, lengths, corrections, tokens, cu,
                                                                      budgets, ignore, eos)
    torch.cuda.synchronize()
    host = [x.cpu() for x in (paths, lengths, corrections, budgets, ignore)]
    cuts = expected_cuts(trees, *host[:3], host[3].tolist(), host[4].tolist(), eos)
    assert limits.tolist() == [c["limit"] for c in cuts]
    width = paths.shape[1]
    assert emitted.tolist() == [c["emitted"] + [-1] * (width - c["limit"]) for c in cuts]
    offsets_expected = np.concatenate([[0], np.cumsum([c["limit"] for c in cuts])]).tolist()
    assert commit_offsets.tolist() == offsets_expected
    assert commit_paths[:offsets_expected[-1]].tolist() == [x for c in cuts for x in c["path"]]
    full = (host[1] + 1).tolist()
    assert any(c["limit"] < f for c, f in zip(cuts, full)), "some request must be cut"
    assert read_and_clear_status(DEV) == 0


def test_truncation_bad_requests_and_commit_chain():
    """Budget 0 gives limit 0 (status bit, no committed rows); the cut paths feed commit_slots."""
    rng, trees, offsets, tokens, cu, paths, lengths, corrections = deep_accept_case(7, [16, 32, 5, 64])
    budgets = torch.tensor([4, 0, 9, 2], dtype=torch.int32, device=DEV)
    ignore = torch.tensor([False, False, True, False], device=DEV)
    limits, emitted, commit_paths, commit_offsets = truncate_accepted(paths, lengths, corrections, tokens, cu,
                                                                      budgets, ignore, [])
    torch.cuda.synchronize()
    assert limits[1].item() == 0 and (emitted[1] == -1).all().item()
    assert read_and_clear_status(DEV) == 4
    # Chain: the cut paths' commit maps equal the oracle's on the same cut paths.
    n = int(commit_offsets[-1])
    block, pool_pages = 16, 64
    tables = torch.tensor(rng.permutation(pool_pages)[:4 * 4].reshape(4, 4), dtype=torch.int32, device=DEV)
    cache_lens = torch.tensor([3, 17, 0, 40], dtype=torch.int32, device=DEV)
    tree_slots = torch.tensor(rng.permutation(pool_pages * block)[:offsets[-1]], dtype=torch.int64, device=DEV)
    live = [r for r in range(4) if limits[r].item() > 0]
    keep = torch.tensor(live, device=DEV)
    # Requests with limit 0 would be rejected (an empty path): commit the live ones only.
    live_cu = torch.tensor(np.concatenate([[0], np.cumsum([offsets[r + 1] - offsets[r] for r in live])]),
                           dtype=torch.int32, device=DEV)
    live_slots = torch.cat([tree_slots[offsets[r]:offsets[r + 1]] for r in live])
    live_paths = torch.cat([commit_paths[int(commit_offsets[r]):int(commit_offsets[r + 1])] for r in live])
    live_offsets = torch.tensor(np.concatenate([[0], np.cumsum([int(limits[r]) for r in live])]), dtype=torch.int32,
                                device=DEV)
    src, dst = commit_slots(live_slots, live_cu, live_paths, live_offsets, tables[keep], cache_lens[keep], block,
                            pool_pages)
    torch.cuda.synchronize()
    esrc, edst, bad = oracle.commit_slots(live_slots.cpu().numpy(), live_cu.cpu().numpy(), live_paths.cpu().numpy(),
                                          live_offsets.cpu().numpy(), tables[keep].cpu().numpy(),
                                          cache_lens[keep].cpu().numpy(), block, pool_pages)
    assert not bad.any() and live_paths.numel() == n
    assert src.tolist() == esrc.tolist() and dst.tolist() == edst.tolist()
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("max_depth,path_nodes,correction", [(15, 16, 26), (3, 4, 14), (0, 1, 11), (25, 20, 99)])
def test_device_depth_cap_closed_form(max_depth, path_nodes, correction):
    """serving_ops.py:78 on the device: a 20-node chain whose every node's argmax is its child's
    token gives nodes 0..min(max_depth, 19) and the last node's argmax as the correction."""
    nodes, vocab = 20, 128
    tokens = torch.tensor([10 + i for i in range(nodes)], device=DEV)
    parents = torch.tensor([-1] + list(range(nodes - 1)), dtype=torch.int32, device=DEV)
    depths = torch.arange(nodes, device=DEV)
    logits = torch.zeros(nodes, vocab, device=DEV)
    for i in range(nodes - 1):
        logits[i, 10 + i + 1] = 5.0
    logits[nodes - 1, 99] = 5.0
    cu = torch.tensor([0, nodes], dtype=torch.int32, device=DEV)
    _, paths, lengths, corrections = accept_batch_device(logits, tokens, parents, depths, cu, max_depth)
    assert paths[0, :path_nodes].tolist() == list(range(path_nodes))
    assert (paths[0, path_nodes:] == -1).all()
    assert int(lengths[0]) == path_nodes - 1 and int(corrections[0]) == correction
    assert read_and_clear_status(DEV) == 0
