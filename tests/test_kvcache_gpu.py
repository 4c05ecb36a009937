"""KV append (store_kvcache) and accepted-only commit (copy_accepted_kv) on the GPU.

Bit-exact against the C oracle at sizes it handles in seconds; at config-3 size
(36 layers, ~52 GB pool) through size-independent properties: destination rows
equal the pre-commit source rows and every other byte of the pool is unchanged.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import commit_slots, copy_accepted_kv, read_and_clear_status, store_kvcache, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def as_bytes(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def test_tree_append_config1_bit_exact():
    batch = workloads.config1(DEV)
    k_pool, v_pool = batch.k_pool.clone(), batch.v_pool.clone()
    k_pool.view(-1, 8, 128)[batch.metadata.tree_slots] = float("nan")
    v_pool.view(-1, 8, 128)[batch.metadata.tree_slots] = float("nan")
    k_ref, v_ref = as_bytes(k_pool).copy(), as_bytes(v_pool).copy()
    store_kvcache(batch.new_k, batch.new_v, k_pool, v_pool, batch.metadata.tree_slots)
    torch.cuda.synchronize()
    oracle.store_kvcache(as_bytes(batch.new_k), as_bytes(batch.new_v), k_ref, v_ref,
                         batch.metadata.tree_slots.cpu().numpy())
    assert np.array_equal(as_bytes(k_pool), k_ref)
    assert np.array_equal(as_bytes(v_pool), v_ref)
    assert read_and_clear_status(DEV) == 0


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_store_with_skips_strided_rows_and_bad_slots(slot_dtype, dtype):
    gen = torch.Generator(device=DEV).manual_seed(5)
    qkv = torch.randn((300, 48, 128), generator=gen, device=DEV).to(dtype)
    key, value = qkv[:, 32:40], qkv[:, 40:48]          # strided views, as after a fused QKV split
    k_cache = torch.randn((7, 256, 8, 128), generator=gen, device=DEV).to(dtype)
    v_cache = torch.randn((7, 256, 8, 128), generator=gen, device=DEV).to(dtype)
    rng = np.random.default_rng(1)
    slots = rng.permutation(7 * 256)[:300].astype(np.int64)
    slots[rng.choice(300, 40, replace=False)] = -1
    slots[7] = 7 * 256 + 3          # outside the cache: skipped and reported
    k_ref, v_ref = as_bytes(k_cache).copy(), as_bytes(v_cache).copy()
    mapping = torch.as_tensor(slots, device=DEV).to(slot_dtype)
    store_kvcache(key, value, k_cache, v_cache, mapping)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 2
    valid = slots.copy()
    valid[7] = -1
    oracle.store_kvcache(as_bytes(key.contiguous()).reshape(300, -1), as_bytes(value.contiguous()).reshape(300, -1),
                         k_ref, v_ref, valid)
    assert np.array_equal(as_bytes(k_cache), k_ref)
    assert np.array_equal(as_bytes(v_cache), v_ref)


def test_store_contract_assertions():
    k_cache = torch.zeros((2, 256, 8, 128), dtype=torch.bfloat16, device=DEV)
    key = torch.zeros((4, 8, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(AssertionError):
        store_kvcache(key, key, k_cache, k_cache, torch.zeros(3, dtype=torch.int64, device=DEV))
    with pytest.raises(AssertionError):
        store_kvcache(key.transpose(1, 2), key.transpose(1, 2), k_cache, k_cache,
                      torch.zeros(4, dtype=torch.int64, device=DEV))


def small_commit_case(seed, overlap=False, layers=4, rows=200, pages=12):
    rng = np.random.default_rng(seed)
    pool = torch.randn((2, layers, pages, 256, 8, 128), generator=torch.Generator(device=DEV).manual_seed(seed),
                       device=DEV).to(torch.bfloat16)
    slots = rng.permutation(pages * 256)
    src, dst = slots[:rows], slots[rows:2 * rows]
    if overlap:
        dst = dst.copy()
        dst[::3] = src[rng.permutation(rows)[:len(dst[::3])]]
    return pool, src.astype(np.int64), dst.astype(np.int64)


# Up to 512 rows take the one-launch commit; 513 and 3000 rows the check + move launches.
@pytest.mark.parametrize("rows,layers,pages", [(200, 4, 12), (512, 2, 12), (513, 2, 12), (3000, 2, 24)])
@pytest.mark.parametrize("overlap", [False, True])
def test_commit_bit_exact_against_oracle(overlap, rows, layers, pages):
    pool, src, dst = small_commit_case(11, overlap, layers=layers, rows=rows, pages=pages)
    print(f"[commit] rows={rows} layers={layers} overlap={overlap}", flush=True)
    expect = as_bytes(pool).copy().view(np.uint16).reshape(pool.shape)
    payload = copy_accepted_kv(pool, torch.as_tensor(src, device=DEV), torch.as_tensor(dst, device=DEV), 256)
    torch.cuda.synchronize()
    assert payload == rows * 2 * layers * 8 * 128 * 2
    assert oracle.copy_accepted_kv(expect, src, dst) == payload
    assert np.array_equal(as_bytes(pool).reshape(-1), expect.view(np.uint8).reshape(-1))
    assert read_and_clear_status(DEV) == 0


def test_commit_contract():
    pool, src, dst = small_commit_case(3)
    s = torch.as_tensor(src, device=DEV)
    with pytest.raises(ValueError, match="one-dimensional"):
        copy_accepted_kv(pool, s.view(2, -1), s.view(2, -1), 256)
    with pytest.raises(ValueError, match="lengths differ"):
        copy_accepted_kv(pool, s, s[:-1], 256)
    assert copy_accepted_kv(pool, s[:0], s[:0], 256) == 0
    bad = torch.as_tensor(dst, device=DEV).clone()
    bad[4] = 12 * 256 + 9
    before = pool.clone()
    copy_accepted_kv(pool, s, bad, 256)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 2
    assert torch.equal(pool.view(torch.int16), before.view(torch.int16)), "an invalid map must not write"
    # The same on the check + move path (more slots than the one-launch commit takes).
    pool, src, dst = small_commit_case(5, rows=3000, layers=2, pages=24)
    bad = torch.as_tensor(dst, device=DEV).clone()
    bad[2999] = -3
    before = pool.clone()
    copy_accepted_kv(pool, torch.as_tensor(src, device=DEV), bad, 256)
    torch.cuda.synchronize()
    assert read_and_clear_status(DEV) == 2
    assert torch.equal(pool.view(torch.int16), before.view(torch.int16)), "an invalid map must not write"


def test_config3_commit_full_size_byte_exact():
    """Config 3 at full size (36 layers, 64 requests): the whole pool after the commit equals,
    byte for byte and one (K/V, layer) plane at a time, a copy of the pool before it to which
    the index-copy closed form of state.py:80-85 (gather the source rows, then scatter them to
    the destinations) was applied."""
    batch = workloads.config3(DEV)
    pool, src, dst = batch.kv_pool, batch.source, batch.destination
    print(f"[cfg3] pool {tuple(pool.shape)} rows {src.numel()} "
          f"payload {2 * pool.shape[1] * src.numel() * 2048 / 1e6:.1f} MB", flush=True)
    block = pool.shape[3]
    expected = pool.clone()
    assert not set(dst.tolist()) & set(src.tolist())
    payload = copy_accepted_kv(pool, src, dst, block)
    torch.cuda.synchronize()
    assert payload == 2 * pool.shape[1] * src.numel() * 8 * 128 * 2
    flat = pool.view(2, pool.shape[1], -1, 8 * 128).view(torch.int16)
    want = expected.view(2, pool.shape[1], -1, 8 * 128).view(torch.int16)
    for kv in range(2):
        for layer in range(pool.shape[1]):
            plane = want[kv, layer]
            rows = plane[src].clone()
            plane[dst] = rows
            assert bool(torch.equal(flat[kv, layer], plane)), f"plane kv={kv} layer={layer} differs"
    del expected
    assert read_and_clear_status(DEV) == 0


def commit_batch_case(seed, requests=24, block=16, width=6, pool_pages=256):
    """A batch of accepted paths over shuffled page tables and scattered tree scratch slots."""
    rng = np.random.default_rng(seed)
    tables = rng.permutation(pool_pages)[:requests * width].reshape(requests, width).astype(np.int32)
    counts = rng.integers(1, 40, size=requests)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    lens = rng.integers(0, (width - 2) * block, size=requests).astype(np.int32)
    tree_slots = rng.permutation(pool_pages * block)[:cu[-1]].astype(np.int64)
    paths, offsets = [], [0]
    for r in range(requests):
        depth = int(rng.integers(1, min(counts[r], block) + 1))
        paths += [0] + rng.permutation(np.arange(1, counts[r]))[:depth - 1].tolist()
        offsets.append(len(paths))
    return tree_slots, cu, np.asarray(paths, np.int32), np.asarray(offsets, np.int32), tables, lens


def run_commit_slots(case, block=16, pool_pages=256):
    tree_slots, cu, paths, offsets, tables, lens = (torch.as_tensor(x, device=DEV) for x in case)
    return commit_slots(tree_slots, cu, paths, offsets, tables, lens, block, pool_pages)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_commit_slots_match_oracle(seed):
    requests = [1, 24, 300][seed]
    pool_pages = max(256, requests * 6)
    case = commit_batch_case(seed, requests=requests, pool_pages=pool_pages)
    print(f"[commit_slots] seed={seed} requests={case[5].size} rows={case[2].size}", flush=True)
    src, dst = run_commit_slots(case, pool_pages=pool_pages)
    torch.cuda.synchronize()
    esrc, edst, bad = oracle.commit_slots(*case, 16, pool_pages)
    assert not bad.any()
    assert np.array_equal(src.cpu().numpy(), esrc) and np.array_equal(dst.cpu().numpy(), edst)
    assert read_and_clear_status(DEV) == 0


def test_commit_slots_reject_like_the_reference():
    tree_slots, cu, paths, offsets, tables, lens = commit_batch_case(4, requests=8)
    paths, lens, tables = paths.copy(), lens.copy(), tables.copy()
    rows = lambda r: slice(offsets[r], offsets[r + 1])
    long_paths = [r for r in range(8) if offsets[r + 1] - offsets[r] >= 2]
    a, b, c = long_paths[:3]
    paths[rows(a)][0] = paths[rows(a)][1]          # not rooted at node 0
    paths[offsets[b] + 1] = 0                      # repeated root
    paths[offsets[c] + 1] = cu[c + 1] - cu[c]      # node outside the tree
    lens[7] = 6 * 16 - 1 if offsets[8] - offsets[7] > 1 else lens[7]
    tables[5, :] = 256                             # page outside the pool
    case = (tree_slots, cu, paths, offsets, tables, lens)
    print(f"[commit_slots] broken requests {a} {b} {c} 5 7", flush=True)
    src, dst = run_commit_slots(case)
    torch.cuda.synchronize()
    esrc, edst, bad = oracle.commit_slots(*case, 16, 256)
    assert bad[[a, b, c, 5]].all()
    assert np.array_equal(src.cpu().numpy(), esrc) and np.array_equal(dst.cpu().numpy(), edst)
    assert read_and_clear_status(DEV) == 2
    with pytest.raises(ValueError, match="request count"):
        commit_slots(*(torch.as_tensor(x, device=DEV) for x in case[:5]), torch.as_tensor(lens[:-1], device=DEV),
                     16, 256)


@pytest.mark.parametrize("broken", [False, True])
def test_commit_slots_then_copy_matches_oracle_commit(broken):
    case = list(commit_batch_case(9, requests=40))
    if broken:
        case[2] = case[2].copy()
        case[2][case[3][3]] = 1                    # request 3's path no longer starts at the root
    rng = np.random.default_rng(9)
    pool = torch.as_tensor(rng.integers(-30000, 30000, size=(2, 3, 256, 16, 2, 64), dtype=np.int16),
                           device=DEV).view(torch.bfloat16)
    expect = pool.cpu().view(torch.int16).numpy().copy()
    print(f"[commit_slots+copy] broken={broken}", flush=True)
    src, dst = run_commit_slots(case)
    copy_accepted_kv(pool, src, dst, 16)
    torch.cuda.synchronize()
    esrc, edst, bad = oracle.commit_slots(*case, 16, 256)
    assert bad.any() == broken
    if not broken:
        oracle.copy_accepted_kv(expect, esrc, edst)
    assert np.array_equal(pool.cpu().view(torch.int16).numpy(), expect)
    assert read_and_clear_status(DEV) == (2 if broken else 0)
