"""Device-side tree visibility (tv_ancestor_words_from_parents, tv_bias_from_ancestor_words).

The serving constructor PackedTreeMetadata.from_host_trees builds the ancestor bits on
the device from the parent arrays.  Checked against what they must equal:
  * the bits packed from the oracle's ancestor matrix (oracle.mask_from_parents, the
    reference's own fixture rule) for random trees, heap trees, 512- and 1024-node
    causal chains (prefill chunks) and single nodes;
  * every field of the validating constructor build() on the same requests,
    qq_bias bit for bit (packed_metadata.py:36-126 vs :128-199);
  * the attention output through either constructor's metadata, bit for bit;
  * malformed parents are reported, not walked;
  * tv_pack_ancestor_words (the bits read back from a caller's qq_bias, as graph capture
    does) equals the same packed masks, ignores entries above the diagonal, and reports a
    value that bits cannot carry.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import PackedTreeMetadata, _device, _lib, packed_tree_attention, read_and_clear_status, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def packed_words(mask: np.ndarray, per_row: int) -> np.ndarray:
    """uint64 words of a boolean [n, n] ancestor matrix, bit m of word m // 64."""
    n = mask.shape[0]
    padded = np.zeros((n, per_row * 64), dtype=bool)
    padded[:, :n] = mask
    return np.packbits(padded, axis=1, bitorder="little").view(np.uint64)


def host_trees(parent_lists):
    trees = []
    for parents in parent_lists:
        mask = torch.from_numpy(oracle.mask_from_parents(parents))
        trees.append(SimpleNamespace(num_nodes=len(parents), host_ancestor=mask, host_parents=list(parents),
                                     host_depths=workloads.depths_of(parents), ancestor=mask))
    return trees


def cases():
    rng = np.random.default_rng(21)
    return [
        [-1],
        workloads.random_parents(16, 5, rng),
        workloads.random_parents(64, 8, rng),
        [-1] + [(n - 1) // 2 for n in range(1, 63)],
        workloads.chain_parents(512),
        workloads.random_parents(200, 30, rng),
        workloads.chain_parents(1024),
        workloads.random_parents(1000, 1000, rng),
    ]


def test_words_equal_packed_oracle_masks():
    parent_lists = cases()
    trees = host_trees(parent_lists)
    counts = [len(p) for p in parent_lists]
    arena = list(range(100, 100 + (sum(counts) + 255) // 256))
    meta = PackedTreeMetadata.from_host_trees([0] * len(trees), [[]] * len(trees), trees, arena, 256, device=DEV,
                                              request_ids=list(range(len(trees))))
    assert meta.ancestor_words is not None
    per_row = meta.ancestor_words.shape[1]
    got = meta.ancestor_words.cpu().numpy().view(np.uint64)
    for r, parents in enumerate(parent_lists):
        sl = meta.request_slice(r)
        want = packed_words(oracle.mask_from_parents(parents), per_row)
        assert np.array_equal(got[sl], want), f"request {r} ({len(parents)} nodes)"
    assert read_and_clear_status(DEV) == 0


def pack_from_bias(meta, per_row):
    lib = _lib.library()
    words = torch.full((meta.total_queries, per_row), -1, dtype=torch.int64, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.check(lib.tv_pack_ancestor_words(meta.qq_bias.data_ptr(), meta.qq_bias_offsets.data_ptr(),
                                          meta.query_to_request.data_ptr(), meta.query_local_row.data_ptr(),
                                          meta.node_counts.data_ptr(), meta.total_queries, meta.num_requests, per_row,
                                          words.data_ptr(), status.data_ptr(), _device.stream_handle(words.device)),
               "pack_ancestor_words")
    return words.cpu().numpy().view(np.uint64), int(status)


def test_words_packed_from_bias_equal_packed_oracle_masks():
    parent_lists = cases()
    counts = [len(p) for p in parent_lists]
    masks = [torch.from_numpy(oracle.mask_from_parents(p)).to(DEV) for p in parent_lists]
    scratch = list(range(100, 100 + (sum(counts) + 255) // 256))
    slots, offset = [], 0
    for n in counts:
        slots.append(torch.tensor([scratch[(offset + j) // 256] * 256 + (offset + j) % 256 for j in range(n)],
                                  device=DEV))
        offset += n
    meta = PackedTreeMetadata.build([0] * len(counts), [[]] * len(counts), slots, masks, 256)
    for per_row in (16, 17):   # the widest tree's words, and one spare word that must stay zero
        got, status = pack_from_bias(meta, per_row)
        assert status == 0
        for r, parents in enumerate(parent_lists):
            want = packed_words(oracle.mask_from_parents(parents), per_row)
            assert np.array_equal(got[meta.request_slice(r)], want), f"request {r} ({len(parents)} nodes)"
    # An entry above the diagonal carries no bit whatever it holds; one at or below it that is
    # neither 0 nor -inf is reported.
    r = 5   # the 200-node random tree
    base = int(meta.qq_bias_offsets[r])
    n = counts[r]
    meta.qq_bias[base + 3 * n + 150] = 0.0
    got, status = pack_from_bias(meta, 16)
    assert status == 0
    assert np.array_equal(got[meta.request_slice(r)], packed_words(oracle.mask_from_parents(parent_lists[r]), 16))
    meta.qq_bias[base + 150 * n + 100] = 0.5
    _, status = pack_from_bias(meta, 16)
    assert status == _lib.TV_STATUS_BAD_BIAS


def test_serving_constructor_equals_validating_constructor():
    rng = np.random.default_rng(3)
    parent_lists = [workloads.random_parents(n, 8, rng) for n in (1, 31, 47, 63, 64, 65)] + [workloads.chain_parents(512)]
    trees = host_trees(parent_lists)
    counts = [len(p) for p in parent_lists]
    prefixes = [5, 259, 27, 0, 600, 256, 1000]
    tables = [[1], [3, 5], [8], [], [20, 21, 22], [30], [40, 41, 42, 43]]
    arena = [60, 61, 62, 63]
    ids = list(range(len(trees)))
    fast = PackedTreeMetadata.from_host_trees(prefixes, tables, trees, arena, 256, device=DEV, request_ids=ids)
    slots, offset = [], 0
    for n in counts:
        slots.append(torch.tensor([arena[(offset + j) // 256] * 256 + (offset + j) % 256 for j in range(n)],
                                  device=DEV))
        offset += n
    full = PackedTreeMetadata.build(prefixes, tables, slots, [t.ancestor.to(DEV) for t in trees], 256, request_ids=ids)
    for key, value in vars(full).items():
        if key == "ancestor_words":
            continue
        actual = getattr(fast, key)
        if isinstance(value, torch.Tensor):
            assert torch.equal(value.cpu().view(torch.uint8) if value.is_floating_point() else value.cpu(),
                               actual.cpu().view(torch.uint8) if actual.is_floating_point() else actual.cpu()), key
        else:
            assert value == actual, key

    # The attention reads the same visibility through either constructor.
    g = torch.Generator(device=DEV).manual_seed(5)
    pool = torch.randn(2, 64, 256, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(sum(counts), 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    a = packed_tree_attention(q, pool[0], pool[1], fast, 128 ** -0.5, 4)
    b = packed_tree_attention(q, pool[0], pool[1], full, 128 ** -0.5, 4)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert read_and_clear_status(DEV) == 0


def test_malformed_parents_are_reported():
    lib = _lib.library()
    parents = torch.tensor([-1, 0, 5, 1, -1, 0, 2], dtype=torch.int32, device=DEV)   # node 2 -> 5, node 4 -> -1
    cu = torch.tensor([0, 7], dtype=torch.int32, device=DEV)
    words = torch.zeros((7, 1), dtype=torch.int64, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.check(lib.tv_ancestor_words_from_parents(parents.data_ptr(), cu.data_ptr(), 1, 7, 1, words.data_ptr(),
                                                  status.data_ptr(), _device.stream_handle(words.device)), "words")
    assert int(status) & _lib.TV_STATUS_BAD_REQUEST
    got = words.cpu().numpy().view(np.uint64)[:, 0]
    # Malformed nodes are roots: node 2 sees itself, node 6 (child of 2) sees {2, 6}.
    assert got[2] == 1 << 2 and got[4] == 1 << 4 and got[6] == (1 << 2) | (1 << 6)
    with pytest.raises(ValueError):
        lib_code = lib.tv_ancestor_words_from_parents(parents.data_ptr(), cu.data_ptr(), 1, 2048, 32,
                                                      words.data_ptr(), status.data_ptr(), None)
        _lib.check(lib_code, "words")
