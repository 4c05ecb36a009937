"""Greedy acceptance (host walk): reference KAT and agreement with the oracle walk (CPU)."""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import accept_batch, build_child_maps, workloads

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_duplicate_sibling_kat_last_child_wins():
    kat = KATS["accept_duplicate_siblings"]
    tree = SimpleNamespace(token_ids=torch.tensor(kat["tokens"]), parent_indices=torch.tensor(kat["parents"]),
                           depth=torch.tensor(kat["depths"]), num_nodes=len(kat["tokens"]))
    logits = torch.randn(len(kat["tokens"]), 80, generator=torch.Generator().manual_seed(99))
    for node, token in kat["forced_argmax"].items():
        logits[int(node), token] = 100
    result = accept_batch(logits, [tree], [0, len(kat["tokens"])], kat["max_depth"])[0]
    assert result["path"] == kat["expected_path"]
    assert result["accepted_length"] == len(kat["expected_path"]) - 1
    assert result["correction"] == int(logits[kat["expected_path"][-1]].argmax())
    assert result["outputs"] == [kat["tokens"][n] for n in kat["expected_path"][1:]] + [result["correction"]]


def test_child_maps_match_oracle_rule():
    rng = np.random.default_rng(4)
    for n in (1, 5, 33, 64):
        parents = workloads.random_parents(n, 8, rng)
        tokens = [int(t) for t in rng.integers(0, 6, size=n)]
        assert build_child_maps(tokens, parents) == oracle.child_maps(tokens, parents)


def test_batch_walks_equal_oracle_walks_with_host_topology():
    rng = np.random.default_rng(5)
    trees, offsets = [], [0]
    for n in (1, 16, 31, 64):
        parents = workloads.random_parents(n, 8, rng)
        tokens = [int(t) for t in rng.integers(0, 5, size=n)]
        trees.append(SimpleNamespace(num_nodes=n, host_token_ids=tokens, host_depths=workloads.depths_of(parents),
                                     child_maps=oracle.child_maps(tokens, parents), parents=parents))
        offsets.append(offsets[-1] + n)
    logits = torch.from_numpy(rng.standard_normal((offsets[-1], 5)).astype(np.float32))
    results = accept_batch(logits, trees, offsets, 15)
    greedy = logits.argmax(-1).tolist()
    for i, tree in enumerate(trees):
        expected = oracle.accept_walk(greedy[offsets[i]:offsets[i + 1]], tree.host_token_ids, tree.host_depths,
                                      tree.child_maps, 15)
        assert results[i] == expected


def test_device_operators_reject_cpu_tensors():
    """No operator has a CPU fallback: CPU inputs are refused before any library call
    (the reference's test_cpu_is_not_a_graph_fallback, tests/test_jetspec_target_graph.py:31-33)."""
    from jetspec_amd import commit_slots, truncate_accepted
    from jetspec_amd.target_graph import GraphedTreeAttention, PackedVerifyGraph

    with pytest.raises(ValueError, match="no CPU path"):
        PackedVerifyGraph(torch.empty((2, 1, 1, 256, 8, 128)), torch.empty((16, 128)), 0.1, 4096)
    with pytest.raises(ValueError, match="no CPU path"):
        GraphedTreeAttention([16], 8, 256, max_prefix=512, device="cpu")
    i32 = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="no CPU path"):
        commit_slots(torch.zeros(1, dtype=torch.int64), i32, i32[:1], i32, torch.zeros((1, 1), dtype=torch.int32),
                     i32[:1], 16, 4)
    with pytest.raises(ValueError, match="no CPU path"):
        truncate_accepted(torch.zeros((1, 2), dtype=torch.int32), i32[:1], torch.zeros(1, dtype=torch.int64),
                          i32[:1], i32, i32[:1], torch.zeros(1, dtype=torch.bool), [2])


def _chain_case(nodes: int, vocab: int = 128):
    """A chain whose every node's argmax is its child's token: the walk accepts until the cap."""
    tokens = [10 + i for i in range(nodes)]
    parents = [-1] + list(range(nodes - 1))
    logits = torch.zeros(nodes, vocab)
    for i in range(nodes - 1):
        logits[i, tokens[i + 1]] = 5.0
    logits[nodes - 1, 99] = 5.0
    return tokens, parents, logits


@pytest.mark.parametrize("max_depth,path_nodes,correction", [(15, 16, 26), (3, 4, 14), (0, 1, 11), (25, 20, 99)])
def test_depth_cap_closed_form(max_depth, path_nodes, correction):
    """serving_ops.py:78: the walk keeps at most max_depth + 1 path nodes.  On a 20-node chain
    where every node's argmax names its child, the path is nodes 0..min(max_depth, 19) and the
    correction is the argmax of its last node (token 10 + last + 1, or 99 at the chain's end)."""
    tokens, parents, logits = _chain_case(20)
    tree = SimpleNamespace(num_nodes=20, host_token_ids=tokens, host_depths=list(range(20)),
                           child_maps=oracle.child_maps(tokens, parents), parents=parents)
    result = accept_batch(logits, [tree], [0, 20], max_depth)[0]
    assert result["path"] == list(range(path_nodes))
    assert result["accepted_length"] == path_nodes - 1
    assert result["correction"] == correction
    assert result["outputs"] == tokens[1:path_nodes] + [correction]
