"""Bit-exact parity of the quantisation kernels against the oracle:
``motif_quantize`` (mx.quantize, affine), ``motif_dequantize`` (the dequant
probe / mx.dequantize) and the single-dispatch 4-slot cache write
``motif_quant_write4`` driven through MotifGroupedQuantizedKVCache.

Shapes follow the reference's tests/test_dequant_probe.py (D in 64/128/256,
gs 32/64/128, bits 4/8, fp16/bf16/fp32) and tests/test_grouped_cache.py
(5-row prefill then 3 decode steps, batched == per-slot), plus the 16000-row
prefill of the 12.7B layer.  Bar: array_equal on packed words, scales and
biases.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits_equal(gpu_t, ref, tag):
    a = torch_to_np(gpu_t)
    if ref.dtype == np.uint32:
        return np.array_equal(a.astype(np.uint32) if a.dtype != np.uint32 else a, ref)
    return np.array_equal(O.round_to(a, tag).astype(np.float64), np.asarray(ref, np.float64))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("tag", ["f16", "bf16", "f32"])
def test_quantize_bit_exact(gpu, rng, bits, gs, D, tag):
    import torch

    from mlx_motif.kernels import quantize

    if D % gs:
        pytest.skip("D not a multiple of group_size")
    x = randn(rng, (2, 5, 7, D), tag)
    d, s, b = quantize(np_to_torch(x, torch_dtype(tag), gpu), group_size=gs, bits=bits)
    rd, rs, rb = O.quantize(x, gs, bits, out_dtype=tag)
    assert d.dtype == torch.uint32 and d.shape == rd.shape
    assert np.array_equal(torch_to_np(d), rd)
    assert _bits_equal(s, rs, tag) and _bits_equal(b, rb, tag)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("tag", ["f16", "bf16", "f32"])
def test_dequant_probe_bit_exact(gpu, rng, bits, gs, D, tag):
    from mlx_motif.kernels import _dequant_probe

    if D % gs:
        pytest.skip("D not a multiple of group_size")
    x = randn(rng, (2, 5, 7, D), tag)
    rd, rs, rb = O.quantize(x, gs, bits, out_dtype=tag)
    dt = torch_dtype(tag)
    y = _dequant_probe(np_to_torch(rd, None, gpu), np_to_torch(rs, dt, gpu),
                       np_to_torch(rb, dt, gpu), group_size=gs, bits=bits)
    assert y.shape == x.shape and y.dtype == dt
    ref = O.dequantize(rd, rs, rb, gs, bits, out_dtype=tag)
    assert np.array_equal(torch_to_np(y), np.asarray(ref, np.float64))


def test_quantize_special_groups(gpu):
    """All-zero, constant, single-outlier and extreme fp16 groups."""
    import torch

    from mlx_motif.kernels import quantize

    rows = [np.zeros(64), np.full(64, 3.0), np.full(64, -2.5),
            np.r_[np.zeros(63), 7.0], np.r_[np.full(63, 1.0), -60000.0],
            np.linspace(-65504, 65504, 64), np.linspace(-1e-7, 1e-7, 64),
            np.r_[np.arange(32), -np.arange(32)] * 0.125]
    x = O.round_to(np.stack(rows), "f16")
    for bits in (4, 8):
        d, s, b = quantize(np_to_torch(x, torch.float16, gpu), group_size=64, bits=bits)
        rd, rs, rb = O.quantize(x, 64, bits)
        assert np.array_equal(torch_to_np(d), rd), bits
        assert np.array_equal(torch_to_np(s), rs.astype(np.float64), equal_nan=True), bits
        assert np.array_equal(torch_to_np(b), rb.astype(np.float64), equal_nan=True), bits


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("unit", [1.0, 0.25])
def test_quantize_exact_ties_half_to_even(gpu, bits, unit):
    """Groups whose codes all land on exact halves (tests/test_quant_ties.py
    builds them and writes the codes out): the GPU kernel resolves every tie
    to even, as the numpy and C oracles and the torch statement do."""
    import torch

    from mlx_motif.kernels import quantize
    from test_quant_ties import tie_groups

    x, even, _ = tie_groups(bits, unit)
    d, s, b = quantize(np_to_torch(x, torch.float16, gpu), group_size=64, bits=bits)
    assert np.array_equal(O.unpack_codes(torch_to_np(d).astype(np.uint32), bits), even)
    rd, rs, rb = O.quantize(x, 64, bits)
    assert np.array_equal(torch_to_np(d), rd)
    assert _bits_equal(s, rs, "f16") and _bits_equal(b, rb, "f16")


def _cache_steps(rng, B, H, D, sizes, tag="f16"):
    return [tuple(randn(rng, (B, H, S, D), tag) for _ in range(4)) for S in sizes]


@pytest.mark.parametrize("bits", [4, 8])
def test_batched_write_matches_per_slot(gpu, rng, bits):
    """5-row prefill + 3 single-row decode steps (tests/test_grouped_cache.py:168)."""
    from mlx_motif.cache import MotifGroupedQuantizedKVCache

    B, H, D, gs = 1, 8, 128, 64
    steps = _cache_steps(rng, B, H, D, [5, 1, 1, 1])
    cache = MotifGroupedQuantizedKVCache(group_size=gs, bits=bits)
    cap = 256
    ref = [(np.zeros((B, H, cap, D * bits // 32), np.uint32), np.zeros((B, H, cap, D // gs)),
            np.zeros((B, H, cap, D // gs))) for _ in range(4)]
    off = 0
    for st in steps:
        live = cache.update_and_fetch_4_quantized(*(np_to_torch(a, torch_dtype("f16"), gpu)
                                                    for a in st))
        O.quant_write4(ref, *st, off, gs, bits)
        off += st[0].shape[2]
    assert cache.offset == off
    for slot_live, slot_ref in zip(live, ref):
        assert slot_live[0].shape[2] == cap
        assert np.array_equal(torch_to_np(slot_live[0]), slot_ref[0])
        assert np.array_equal(torch_to_np(slot_live[1]), slot_ref[1])
        assert np.array_equal(torch_to_np(slot_live[2]), slot_ref[2])


@pytest.mark.parametrize("bits", [4, 8])
def test_write_grows_past_step_and_matches(gpu, rng, bits):
    from mlx_motif.cache import MotifGroupedQuantizedKVCache

    B, H, D, gs = 1, 4, 128, 64
    cache = MotifGroupedQuantizedKVCache(group_size=gs, bits=bits)
    cache.step = 4
    steps = _cache_steps(rng, B, H, D, [3, 1, 1, 2, 1, 5, 1])
    for st in steps:
        live = cache.update_and_fetch_4_quantized(*(np_to_torch(a, torch_dtype("f16"), gpu)
                                                    for a in st))
    o = cache.offset
    allrows = [np.concatenate([st[i] for st in steps], axis=2) for i in range(4)]
    for i, slot in enumerate(live):
        rd, rs, rb = O.quantize(allrows[i], gs, bits)
        assert np.array_equal(torch_to_np(slot[0])[:, :, :o], rd)
        assert np.array_equal(torch_to_np(slot[1])[:, :, :o], rs.astype(np.float64))
        assert np.array_equal(torch_to_np(slot[2])[:, :, :o], rb.astype(np.float64))


@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_16000_rows_then_decode(gpu, rng, bits):
    """12.7B layer: 8 heads, D 128, a 16000-row prefill write then one decode row."""
    from mlx_motif.cache import MotifGroupedQuantizedKVCache

    B, H, D, gs = 1, 8, 128, 64
    cache = MotifGroupedQuantizedKVCache(group_size=gs, bits=bits)
    pre = _cache_steps(rng, B, H, D, [16000])[0]
    dec = _cache_steps(rng, B, H, D, [1])[0]
    cache.update_and_fetch_4_quantized(*(np_to_torch(a, torch_dtype("f16"), gpu) for a in pre))
    live = cache.update_and_fetch_4_quantized(*(np_to_torch(a, torch_dtype("f16"), gpu)
                                                for a in dec))
    assert cache.offset == 16001 and live[0][0].shape[2] == 16128
    for i, slot in enumerate(live):
        rows = np.concatenate([pre[i], dec[i]], axis=2)
        rd, rs, rb = O.quantize(rows, gs, bits)
        assert np.array_equal(torch_to_np(slot[0])[:, :, :16001], rd)
        assert np.array_equal(torch_to_np(slot[1])[:, :, :16001], rs.astype(np.float64))
        assert np.array_equal(torch_to_np(slot[2])[:, :, :16001], rb.astype(np.float64))


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_bridge_fetch(gpu, rng, bits):
    """update_and_fetch_4 returns exact-length dequantised slices (cache.py:448-465)."""
    from mlx_motif.cache import MotifGroupedQuantizedKVCache

    cache = MotifGroupedQuantizedKVCache(group_size=64, bits=bits)
    st = _cache_steps(rng, 1, 8, 128, [5])[0]
    out = cache.update_and_fetch_4(*(np_to_torch(a, torch_dtype("f16"), gpu) for a in st))
    assert all(t.shape == (1, 8, 5, 128) for t in out)
    tol = {4: 0.5, 8: 0.05}[bits]
    for t, src in zip(out, st):
        rd, rs, rb = O.quantize(src, 64, bits)
        assert np.array_equal(torch_to_np(t), O.dequantize(rd, rs, rb, 64, bits, "f16"))
        assert np.max(np.abs(torch_to_np(t) - src.astype(np.float64))) <= tol * 8
