"""Pins the HF-order RoPE + scatter oracle (oracle.rope_scatter_hf) on the CPU.

The reference's own GPU test takes its expected values from eager torch bf16/fp32
arithmetic (tests/test_jetspec_tree_fusion.py:21-32, ``eager_rope``), so the oracle is
checked bitwise against that same eager computation here on the CPU, on random
operands and on edge values (signed zeros, infinities, the largest finite bf16,
rounding ties), and against the reference's rounding witness (:117-126).  Planted
mistakes (one cast of an fp32 expression, a swapped sine sign, cos/sin left in fp32)
must fail the same comparison.  NaN payloads are not pinned: the reference's paths
disagree on them (PyTorch CPU kernels and its GPU cast produce different NaN bits),
so the GPU tests compare NaN positions only.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def eager_rope(x: torch.Tensor, positions: torch.Tensor, cache: torch.Tensor) -> torch.Tensor:
    """Eager HF RoPE exactly as models/qwen3.py:241-249 and the reference test write it."""
    selected = cache[positions]
    if selected.ndim == 2:
        selected = selected.unsqueeze(1)
    cos, sin = selected.chunk(2, -1)
    cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    x1, x2 = x.chunk(2, -1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)


def as_f32(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def oracle_rope(x: torch.Tensor, positions: torch.Tensor, cache: torch.Tensor, rope=None) -> np.ndarray:
    rows = as_f32(cache)[positions.numpy()]
    if rows.ndim == 3:
        rows = rows[:, 0]
    half = x.shape[-1] // 2
    fn = rope or oracle.rope_hf_order
    return fn(as_f32(x), rows[:, None, :half], rows[:, None, half:], x.dtype == torch.bfloat16)


def bits(values: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    if dtype == torch.bfloat16:
        return oracle.f32_to_bf16_bits(values)
    return np.asarray(values, dtype=np.float32).view(np.uint32)


def torch_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else \
        t.contiguous().numpy().view(np.uint32)


def fixture(dtype, dim, cache_dtype=torch.float32, rows=7, heads=8, seed=740319):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, heads, dim, generator=g).to(dtype)
    kat = KATS["rope_fixture"]
    positions = torch.tensor(kat["positions"][:rows])
    angles = torch.arange(kat["cache_positions"], dtype=torch.float32)[:, None] * (
        torch.arange(dim // 2, dtype=torch.float32)[None, :] + 1) * kat["angle_step"]
    cache = torch.cat((angles.cos(), angles.sin()), -1).to(cache_dtype).unsqueeze(1)
    return x, positions, cache


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dim", KATS["rope_fixture"]["dims"])
@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
def test_oracle_equals_eager_torch_bitwise(dtype, dim, cache_dtype):
    x, positions, cache = fixture(dtype, dim, cache_dtype)
    expected = eager_rope(x, positions, cache)
    got = oracle_rope(x, positions, cache)
    assert np.array_equal(bits(got, dtype), torch_bits(expected))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_oracle_equals_eager_torch_on_edge_values(dtype):
    edge = [0.0, -0.0, float("inf"), float("-inf"), 3.3895313892515355e38, -3.3895313892515355e38,
            1.0078125, 1.015625, 1e-30, -2.5, 65504.0, 1.00390625]
    rng = np.random.default_rng(3)
    values = rng.choice(edge, size=(16, 4, 64)).astype(np.float32)
    x = torch.from_numpy(values).to(dtype)
    positions = torch.arange(16)
    angles = torch.from_numpy(rng.uniform(-4, 4, size=(16, 32)).astype(np.float32))
    cache = torch.cat((angles.cos(), angles.sin()), -1)
    cache[0, :] = torch.tensor([0.70703125] * 64)
    cache[1, :32], cache[1, 32:] = 1.0, 0.0
    cache[2, :32], cache[2, 32:] = -0.0, -1.0
    expected = eager_rope(x, positions, cache)
    got = oracle_rope(x, positions, cache)
    e, o = torch_bits(expected), bits(got, dtype)
    nan = np.isnan(expected.float().numpy())
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(e[~nan], o[~nan])


def test_reference_rounding_witness():
    kat = KATS["rope_rounding_witness"]
    q = torch.tensor([[kat["q"]]], dtype=torch.bfloat16)
    cache = torch.tensor([[kat["cos"], kat["sin"]]], dtype=torch.float32)
    positions = torch.tensor([0])
    eager = eager_rope(q, positions, cache)
    got = oracle_rope(q, positions, cache)
    assert np.array_equal(bits(got, torch.bfloat16), torch_bits(eager))
    # The reference's point: a single cast of the fp32 expression differs.
    x1, x2 = q.float().chunk(2, -1)
    cos, sin = cache.to(q.dtype).float().unsqueeze(1).chunk(2, -1)
    single = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(q.dtype)
    assert not np.array_equal(torch_bits(single), torch_bits(eager))


def _single_cast(x, cos, sin, bf16):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    cos, sin = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(cos)), oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(sin))
    y = np.concatenate((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)
    return oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(y))


def _swapped_sign(x, cos, sin, bf16):
    return oracle.rope_hf_order(x, cos, -sin, bf16)


def _fp32_cache(x, cos, sin, bf16):
    half = x.shape[-1] // 2
    r = lambda t: oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(t))
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate((r(r(x1 * cos) - r(x2 * sin)), r(r(x2 * cos) + r(x1 * sin))), -1)


@pytest.mark.parametrize("mistake", [_single_cast, _swapped_sign, _fp32_cache])
def test_planted_mistakes_fail(mistake):
    x, positions, cache = fixture(torch.bfloat16, 128)
    expected = torch_bits(eager_rope(x, positions, cache))
    wrong = bits(oracle_rope(x, positions, cache, rope=mistake), torch.bfloat16)
    assert not np.array_equal(wrong, expected)


def test_scatter_writes_only_the_named_slots():
    x, positions, cache = fixture(torch.bfloat16, 64, heads=4, rows=7)
    kat = KATS["rope_fixture"]
    slots = np.asarray(kat["slots"])
    q = as_f32(x)
    k = q[:, :2].copy()
    v = q[:, 1:3].copy() * 3
    k_pool = np.full((4, 256, 2, 64), np.nan, dtype=np.float32)
    v_pool = np.full((4, 256, 2, 64), np.nan, dtype=np.float32)
    out = oracle.rope_scatter_hf(q, k, v, positions.numpy(), as_f32(cache)[:, 0], k_pool, v_pool, slots, True)
    assert np.array_equal(bits(out, torch.bfloat16), torch_bits(eager_rope(x, positions, cache)))
    k_expected = eager_rope(x[:, :2], positions, cache)
    for i, slot in enumerate(slots):
        page, offset = divmod(int(slot), 256)
        assert np.array_equal(bits(k_pool[page, offset], torch.bfloat16), torch_bits(k_expected[i]))
        assert np.array_equal(v_pool[page, offset], v[i])
    touched = np.zeros((4, 256), dtype=bool)
    touched[slots // 256, slots % 256] = True
    assert np.isnan(k_pool[~touched]).all() and np.isnan(v_pool[~touched]).all()
