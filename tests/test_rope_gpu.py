"""Fused HF-order RoPE + tree K/V scatter (tv_rope_scatter) on the GPU.

Bit-exact against the numpy oracle (oracle.rope_scatter_hf, itself pinned bitwise to
eager torch on the CPU): the rotated Q and every byte of both pools, including the
slots that must stay untouched.  Covers the reference's fixture (tests/
test_jetspec_tree_fusion.py:40-72: 7 rows, 8/2 heads, dims 32/96/128/256, bf16 and
fp32, contiguous and strided views, rank-2 and rank-3 caches, fp32 and bf16 caches),
its rounding/signed-zero witness (:171-182), replay with changed positions and slots
and request isolation (:158-169), NaN-filled pools (:184-189), rejection before any
store (:191-217), and the served Qwen3 geometry at config-4 size (4096 tree rows).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jetspec_amd import read_and_clear_status, rope_scatter, rope_scatter_prevalidated

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy().view(np.uint32)


def oracle_bits(values: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    if dtype == torch.bfloat16:
        return oracle.f32_to_bf16_bits(values)
    return np.asarray(values, dtype=np.float32).view(np.uint32)


def fixture(dtype=torch.bfloat16, *, dim=128, strided=False, cache_rank=3, cache_dtype=torch.float32,
            rows=7, q_heads=8, kv_heads=2, pages=4, page=256, seed=740319, nan_pools=False):
    g = torch.Generator(device=DEV).manual_seed(seed)

    def values(heads):
        if strided:
            backing = torch.randn(rows * 2, heads * 2, dim * 2, generator=g, device=DEV, dtype=dtype)
            return backing[::2, ::2, ::2]
        return torch.randn(rows, heads, dim, generator=g, device=DEV, dtype=dtype)

    q, k, v = values(q_heads), values(kv_heads), values(kv_heads)
    base_positions = [0, 1, 127, 255, 513, 1023, 2047]
    base_slots = [257, 1, 767, 256, 0, 513, 511]
    if rows <= 7:
        positions = torch.tensor(base_positions[:rows], device=DEV)
        slots = torch.tensor(base_slots[:rows], device=DEV)
    else:
        rng = np.random.default_rng(seed)
        positions = torch.as_tensor(rng.integers(0, 2048, size=rows), device=DEV)
        slots = torch.as_tensor(rng.permutation(pages * page)[:rows], device=DEV)
    if strided:
        pb = torch.zeros(rows * 2, dtype=torch.int64, device=DEV)
        sb = torch.zeros_like(pb)
        pb[::2], sb[::2] = positions, slots
        positions, slots = pb[::2], sb[::2]
    angles = torch.arange(2048, device=DEV, dtype=torch.float32)[:, None] * (
        torch.arange(dim // 2, device=DEV, dtype=torch.float32)[None, :] + 1) * .00317
    cache = torch.cat((angles.cos(), angles.sin()), -1).to(cache_dtype)
    if strided:
        backing = torch.empty(cache.shape[0] * 2, dim * 2, dtype=cache.dtype, device=DEV)
        backing[::2, ::2] = cache
        cache = backing[::2, ::2]
    if cache_rank == 3:
        cache = cache.unsqueeze(1)
    pools = torch.randn(2, pages, page, kv_heads, dim, generator=g, device=DEV, dtype=dtype)
    if nan_pools:
        pools.fill_(float("nan"))
    return [q, k, v, positions, cache, pools[0], pools[1], slots]


def expected(args):
    q, k, v, positions, cache, k_pool, v_pool, slots = args
    k_ref, v_ref = host_f32(k_pool), host_f32(v_pool)
    cache_rows = host_f32(cache).reshape(cache.shape[0], -1)
    out = oracle.rope_scatter_hf(host_f32(q), host_f32(k), host_f32(v), positions.cpu().numpy(), cache_rows,
                                 k_ref, v_ref, slots.cpu().numpy(), q.dtype == torch.bfloat16)
    return out, k_ref, v_ref


def assert_equivalent(args, *, provided_out=False):
    out_ref, k_ref, v_ref = expected(args)
    dtype = args[0].dtype
    out = torch.empty_like(args[0]) if provided_out else None
    actual = rope_scatter(*args, out=out)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(actual), oracle_bits(out_ref, dtype)), "rotated Q differs from the oracle"
    for pool, ref, name in ((args[5], k_ref, "K"), (args[6], v_ref, "V")):
        got = host_bits(pool)
        want = oracle_bits(ref, dtype)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(host_f32(pool)), nan), f"{name} pool NaN positions differ"
        assert np.array_equal(got[~nan], want[~nan]), f"{name} pool differs (written or untouched slots)"
    if provided_out:
        assert actual is out
    assert read_and_clear_status(DEV) == 0
    return actual


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dim", [32, 96, 128, 256])
@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("rank", [2, 3])
def test_reference_fixture_bit_exact(dtype, dim, strided, rank):
    print(f"[rope] dtype={dtype} dim={dim} strided={strided} rank={rank}", flush=True)
    assert_equivalent(fixture(dtype, dim=dim, strided=strided, cache_rank=rank), provided_out=strided)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bf16_cache_and_nan_unallocated_pages_are_untouched(dtype):
    assert_equivalent(fixture(dtype, strided=True, cache_dtype=torch.bfloat16, nan_pools=True))


def test_rounding_witness_and_signed_zero():
    args = fixture(dim=32)
    args[0].fill_(1.0078125)
    args[0][..., 16:] = 1.015625
    args[1].copy_(args[0][:, :2])
    args[4][..., :16] = .70703125
    args[4][..., 16:] = .70703125
    assert_equivalent(args)
    args[0].zero_()
    args[0][..., 16:] = -0.0
    args[1].copy_(args[0][:, :2])
    assert_equivalent(args)


def test_dynamic_positions_slots_replay_and_request_isolation():
    args = fixture(strided=True)
    for _ in range(3):
        assert_equivalent(args)
        args[3].copy_((args[3] + 17) % args[4].shape[0])
        args[7].copy_((args[7] + 43) % (args[5].shape[0] * args[5].shape[1]))
    baseline = assert_equivalent(args).clone()
    args[0][3:].mul_(17)
    args[1][3:].add_(8)
    args[2][3:].sub_(5)
    modified = assert_equivalent(args)
    assert np.array_equal(host_bits(modified[:3]), host_bits(baseline[:3])), "other rows cannot change Q"


def test_served_geometry_at_config4_size():
    """Qwen3-8B attention geometry (32/8 heads x 128, bf16) for 4096 tree rows scattered over a pool."""
    args = fixture(rows=4096, q_heads=32, kv_heads=8, pages=24, page=256, seed=11)
    assert_equivalent(args)


def test_nonfinite_operands_keep_nan_positions():
    args = fixture(dim=64)
    args[0][0, 0, 0] = float("nan")
    args[0][1, 1, 40] = float("inf")
    args[1][2, 0, 5] = float("-inf")
    assert_equivalent(args)


def test_invalid_addresses_duplicates_or_aliases_rejected_before_store():
    for name in ("position", "negative_slot", "too_large_slot", "duplicate"):
        args = fixture()
        k_before, v_before = host_bits(args[5]).copy(), host_bits(args[6]).copy()
        if name == "position":
            args[3][0] = args[4].shape[0]
        elif name == "negative_slot":
            args[7][0] = -1
        elif name == "too_large_slot":
            args[7][0] = args[5].shape[0] * args[5].shape[1]
        else:
            args[7][0] = args[7][1]
        with pytest.raises(ValueError):
            rope_scatter(*args)
        assert np.array_equal(host_bits(args[5]), k_before)
        assert np.array_equal(host_bits(args[6]), v_before)
    args = fixture()
    with pytest.raises(ValueError, match="output must not alias"):
        rope_scatter(*args, out=args[0])
    args = fixture()
    args[6] = args[5]
    with pytest.raises(ValueError, match="pool views must not overlap"):
        rope_scatter(*args)
    args = fixture()
    overlap = torch.empty_like(args[0]).as_strided(args[0].shape, (1, 1, 1))
    with pytest.raises(ValueError, match="overlapping write addresses"):
        rope_scatter(*args, out=overlap)


def test_prevalidated_boundary_refuses_out_of_range_rows_without_writing():
    """The launch-only boundary trusts its caller, but the kernel still writes nothing
    for a row whose position or slot is out of range and reports it in the status word."""
    args = fixture()
    out = torch.zeros_like(args[0])
    good = [0, 1, 3, 5, 6]
    sub = [args[0][good], args[1][good], args[2][good], args[3][good], args[4], args[5].clone(), args[6].clone(),
           args[7][good]]
    out_ref, k_ref, v_ref = expected(sub)
    args[3][2] = args[4].shape[0] + 5                      # row 2: position past the cache
    args[7][4] = args[5].shape[0] * args[5].shape[1]       # row 4: slot past the pool
    read_and_clear_status(DEV)
    rope_scatter_prevalidated(*args, out)
    status = read_and_clear_status(DEV)
    assert status & 8 and status & 2
    got = host_bits(out)
    assert not got[2].any() and not got[4].any()
    assert np.array_equal(got[good], oracle_bits(out_ref, args[0].dtype))
    assert np.array_equal(host_bits(args[5]), oracle_bits(k_ref, args[0].dtype))
    assert np.array_equal(host_bits(args[6]), oracle_bits(v_ref, args[0].dtype))


def test_cpu_tensors_are_rejected():
    args = [t.cpu() for t in fixture()]
    with pytest.raises(ValueError, match="CUDA tensors"):
        rope_scatter(*args)
