"""PackedTreeMetadata: reference KATs, rejections, and equivalence of both constructors (CPU)."""
from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import PackedTreeMetadata, workloads

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def heap_mask(nodes):
    parents = [-1] + [(n - 1) // 2 for n in range(1, nodes)]
    return torch.from_numpy(oracle.mask_from_parents(parents))


def fixture(counts=(63, 31, 47)):
    kat = KATS["packed_metadata"]
    starts = np.concatenate(([0], np.cumsum(counts)))
    slots = [torch.arange(kat["slot_base"] + starts[i], kat["slot_base"] + starts[i + 1], dtype=torch.int64)
             for i in range(len(counts))]
    prefixes = tuple(kat["prefixes"][:len(counts)])
    pages = [tuple(p) for p in kat["pages"][:len(counts)]]
    masks = [heap_mask(n) for n in counts]
    return PackedTreeMetadata.build(prefixes, pages, slots, masks, kat["block_size"]), slots, masks


def test_exact_ragged_offsets_and_local_masks():
    expect = KATS["packed_metadata"]["expect"]
    meta, _, _ = fixture()
    assert list(meta.query_offsets) == expect["query_offsets"]
    assert meta.request_slice(1) == slice(*expect["request_slice_1"])
    assert list(meta.prefix_lengths) == expect["prefix_lengths"]
    assert list(meta.node_counts_host) == expect["node_counts_host"]
    assert meta.mask_elements == expect["mask_elements"]
    assert meta.mask_elements < meta.total_queries ** 2
    assert meta.block_tables.tolist() == expect["block_tables"]
    assert meta.query_to_request.tolist() == [0] * 63 + [1] * 31 + [2] * 47
    assert meta.query_local_row.tolist() == list(range(63)) + list(range(31)) + list(range(47))
    assert meta.report()["numerical_contract"] == expect["numerical_contract"]
    with pytest.raises(IndexError):
        meta.request_slice(-1)
    with pytest.raises(IndexError):
        meta.request_slice(3)


def test_device_arrays_equal_oracle_restatement():
    meta, slots, masks = fixture()
    kat = KATS["packed_metadata"]
    ref = oracle.metadata_arrays(kat["prefixes"], kat["pages"], [s.tolist() for s in slots],
                                 [m.numpy() for m in masks], kat["block_size"])
    for name, value in ref.items():
        got = getattr(meta, name).numpy()
        assert got.dtype == value.dtype, name
        assert np.array_equal(got, value), name


def test_rejects_overlapping_scratch_and_committed_pages():
    _, slots, masks = fixture()
    with pytest.raises(ValueError, match="overlapping"):
        PackedTreeMetadata.build([65, 0], [[2], []], [slots[0], slots[0][:31]], masks[:2], 256)
    with pytest.raises(ValueError, match="committed"):
        PackedTreeMetadata.build([65], [[6]], [slots[0]], masks[:1], 256)


def test_rejects_noncanonical_tables_and_malformed_ancestors():
    _, slots, masks = fixture()
    with pytest.raises(ValueError, match="canonical"):
        PackedTreeMetadata.build([257], [[2]], slots[:1], masks[:1], 256)
    with pytest.raises(ValueError, match="canonical"):
        PackedTreeMetadata.build([257], [[2, 2]], slots[:1], masks[:1], 256)
    future = masks[0].clone()
    future[0, 1] = True
    with pytest.raises(ValueError, match="causal"):
        PackedTreeMetadata.build([65], [[2]], slots[:1], [future], 256)
    missing_self = masks[0].clone()
    missing_self[1, 1] = False
    with pytest.raises(ValueError, match="self"):
        PackedTreeMetadata.build([65], [[2]], slots[:1], [missing_self], 256)
    with pytest.raises(ValueError, match="negative"):
        PackedTreeMetadata.build([0], [[]], [torch.tensor([-3])], [torch.ones(1, 1, dtype=torch.bool)], 256)
    with pytest.raises(ValueError, match="nonempty"):
        PackedTreeMetadata.build([], [], [], [], 256)


def test_pool_bounds_and_geometry():
    geometry = KATS["packed_metadata"]["pool_geometry"]
    meta, _, _ = fixture()
    meta.validate_pool_geometry(torch.empty(geometry["ok"]))
    with pytest.raises(ValueError, match="geometry"):
        meta.validate_pool_geometry(torch.empty(geometry["bad_page_size"]))
    with pytest.raises(ValueError, match="outside"):
        meta.validate_pool_geometry(torch.empty(geometry["too_few_blocks"]))


def host_trees(counts, seed=17):
    rng = np.random.default_rng(seed)
    trees = []
    for n in counts:
        parents = workloads.random_parents(n, 6, rng)
        mask = torch.from_numpy(workloads.ancestor_mask(parents))
        trees.append(SimpleNamespace(num_nodes=n, host_ancestor=mask, host_parents=parents,
                                     host_depths=workloads.depths_of(parents), ancestor=mask))
    return trees


def test_host_metadata_matches_full_validation_every_field():
    kat = KATS["host_metadata_equivalence"]
    trees = host_trees([1, 31, 47, 63])
    b = kat["block_size"]
    fast = PackedTreeMetadata.from_host_trees(kat["prefixes"], kat["tables"], trees, kat["arena"], b,
                                              device="cpu", request_ids=kat["request_ids"])
    slots, offset = [], 0
    for tree in trees:
        slots.append(torch.arange(kat["arena"][0] * b + offset, kat["arena"][0] * b + offset + tree.num_nodes))
        offset += tree.num_nodes
    full = PackedTreeMetadata.build(kat["prefixes"], kat["tables"], slots, [t.ancestor for t in trees], b,
                                    request_ids=kat["request_ids"])
    for key, value in vars(full).items():
        actual = getattr(fast, key)
        if isinstance(value, torch.Tensor):
            assert torch.equal(value, actual), key
        else:
            assert value == actual, key


def test_host_metadata_rejects_aliases_and_inconsistent_ancestry():
    trees = host_trees([1, 31, 47, 63])
    with pytest.raises(ValueError, match="overlap"):
        PackedTreeMetadata.from_host_trees([1] * 4, [[11]] * 4, trees, [11], 256, device="cpu",
                                           request_ids=list(range(4)))
    trees[1].host_depths[1] = 7
    with pytest.raises(ValueError, match="depth"):
        PackedTreeMetadata.from_host_trees([1] * 4, [[i] for i in range(4)], trees, [11], 256, device="cpu",
                                           request_ids=list(range(4)))
    trees = host_trees([1, 31])
    bad = trees[1].host_ancestor.clone()
    bad[5, 0] = False
    trees[1].host_ancestor = bad
    with pytest.raises(ValueError, match="visibility"):
        PackedTreeMetadata.from_host_trees([0, 0], [[], []], trees, [11], 256, device="cpu", request_ids=[0, 1])
