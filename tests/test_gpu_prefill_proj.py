"""Parity of ``motif_gda_prefill_proj``: a GDA layer's prefill chunk from the
projection outputs in one attention launch (RoPE on q and k, the chunk's
k1/k2/v1/v2 rows written into the 4-slot cache, both dual-V passes with the
bottom-right causal mask; model.py:590-629 and 769-797).

Checks:
  - the cache rows equal what ``rope_split4`` writes, bit for bit (same
    fp32 angles and rounding), and rows outside the chunk keep their
    contents (poisoned rows of the chunk are overwritten, never read);
  - the attention outputs against the oracle's float64 attention over the
    same roped q (rope_split4's q1/q2) and the written cache: max-abs
    <= 2e-3 for fp16 (fp32 accumulation, fp16 output), 1e-2 for bf16;
  - end to end against the oracle's composition (float64 RoPE rounded to the
    element type; its fp32-angle drift is part of the rope test's bar) within
    the same 2e-3;
  - against the unfused native path (rope_split4 + two sdpa_dual_v_rows
    calls) within 1e-3: both accumulate in fp32 and differ only in tile
    boundaries at the chunk's first row and in split points.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

BAR = {"f16": 2e-3, "bf16": 1e-2}


def _case(gpu, rng, B, S, qg, gr, kg, offset, cap, tag="f16", origin_first=False, poison=True):
    import torch

    D = 128
    dt = torch_dtype(tag)
    q = randn(rng, (B, S, qg * (gr + 1) * D), tag)
    k = randn(rng, (B, S, 2 * kg * D), tag)
    v = randn(rng, (B, S, 2 * kg * D), tag)
    old = [randn(rng, (B, kg, cap, D), tag) for _ in range(4)]
    if poison:  # the chunk's rows and the rows past it must not be read
        for c in old:
            c[:, :, offset:] = 4096.0  # exact in fp16 and bf16
    T = lambda a: np_to_torch(a, dt, gpu)  # noqa: E731
    return (q, k, v, old), (T(q), T(k), T(v), [T(c) for c in old])


def _fused(args_t, offset, qg, gr, kg, origin_first=False):
    from mlx_motif.kernels import gda_prefill_attention_from_proj

    q, k, v, caches = args_t
    return gda_prefill_attention_from_proj(q, k, v, caches, offset, qg, gr, kg,
                                           1 / np.sqrt(128), origin_first=origin_first)


def _unfused(args_t, offset, qg, gr, kg, origin_first=False):
    from mlx_motif.kernels import rope_split4, sdpa_dual_v_rows

    q, k, v, caches = args_t
    q1, q2, k1, k2, v1, v2 = rope_split4(q, k, v, qg, gr, kg, 1, offset,
                                         origin_first=origin_first, caches=caches)
    S = q.shape[1]
    sc = 1 / np.sqrt(128)
    return (q1, q2, sdpa_dual_v_rows(q1, k1, v1, v2, sc, kv_len=offset + S, causal=True),
            sdpa_dual_v_rows(q2, k2, v1, v2, sc, kv_len=offset + S, causal=True))


def _check(gpu, rng, B, S, qg, gr, kg, offset, cap, tag="f16", origin_first=False,
           end_to_end=False):
    import torch

    print(f"gda_prefill_proj B={B} S={S} qg={qg} gr={gr} kg={kg} offset={offset} cap={cap} "
          f"{tag} origin_first={origin_first}", flush=True)
    np_args, t_fused = _case(gpu, rng, B, S, qg, gr, kg, offset, cap, tag, origin_first)
    t_unf = (t_fused[0], t_fused[1], t_fused[2], [c.clone() for c in t_fused[3]])
    y_o, y_n = _fused(t_fused, offset, qg, gr, kg, origin_first)
    q1, q2, u_o, u_n = _unfused(t_unf, offset, qg, gr, kg, origin_first)
    torch.cuda.synchronize()
    # cache rows: bit for bit what rope_split4 wrote; the rest untouched
    for a, b_, c0 in zip(t_fused[3], t_unf[3], np_args[3]):
        assert torch.equal(a.view(torch.int16), b_.view(torch.int16))
        got = torch_to_np(a)
        np.testing.assert_array_equal(got[:, :, :offset], c0[:, :, :offset])
        np.testing.assert_array_equal(got[:, :, offset + S:], c0[:, :, offset + S:])
    # attention against the oracle over the same roped inputs
    cache = [torch_to_np(c) for c in t_fused[3]]
    sc = 1 / np.sqrt(128)
    kv = offset + S
    ref_o = O.sdpa_dual_v(torch_to_np(q1), cache[0], cache[2], cache[3], sc, kv, causal=True)
    ref_n = O.sdpa_dual_v(torch_to_np(q2), cache[1], cache[2], cache[3], sc, kv, causal=True)
    go, gn = torch_to_np(y_o), torch_to_np(y_n)
    assert np.isfinite(go).all() and np.isfinite(gn).all()
    err_o = float(np.max(np.abs(go - ref_o)))
    err_n = float(np.max(np.abs(gn - ref_n)))
    assert err_o <= BAR[tag] and err_n <= BAR[tag], f"origin {err_o:.3e} noise {err_n:.3e}"
    d_o = float(np.max(np.abs(go - torch_to_np(u_o))))
    d_n = float(np.max(np.abs(gn - torch_to_np(u_n))))
    assert d_o <= BAR[tag] / 2 and d_n <= BAR[tag] / 2, f"vs unfused {d_o:.3e} {d_n:.3e}"
    if end_to_end:
        e_o, e_n, slots = O.gda_prefill_from_proj(*np_args[:3], np_args[3], offset, qg, gr, kg,
                                                  sc, origin_first=origin_first, dtype=tag)
        assert float(np.max(np.abs(go - e_o))) <= BAR[tag]
        assert float(np.max(np.abs(gn - e_n))) <= BAR[tag]
    return err_o, err_n


def test_prefill_chunk_12p7b_layer(gpu, rng):
    """A 512-row chunk of the 12.7B layout (32 origin + 8 noise heads over 8
    KV heads) at offset 3204: rows split, one merge launch for both passes."""
    _check(gpu, rng, 1, 512, 8, 4, 8, 3204, 3840, end_to_end=True)


def test_prefill_first_chunk(gpu, rng):
    """offset 0: every row comes from the projections."""
    _check(gpu, rng, 1, 256, 8, 4, 8, 0, 256)


@pytest.mark.parametrize("B,S,qg,gr,kg,offset,cap,origin_first", [
    (1, 33, 8, 4, 8, 700, 768, False),     # ragged chunk, 4-wave blocks
    (2, 96, 2, 3, 2, 400, 512, True),      # batch 2, origin-first q
    (1, 40, 8, 4, 4, 95, 160, False),      # two q groups per KV head
    (1, 1, 8, 4, 8, 3203, 3328, False),    # a one-row chunk
])
def test_prefill_shapes(gpu, rng, B, S, qg, gr, kg, offset, cap, origin_first):
    _check(gpu, rng, B, S, qg, gr, kg, offset, cap, origin_first=origin_first)


def test_prefill_bf16(gpu, rng):
    _check(gpu, rng, 1, 200, 8, 4, 8, 1000, 1280, tag="bf16")


@pytest.mark.parametrize("rps", [64, 96, 2048])
def test_prefill_forced_splits(gpu, rng, rps):
    """Split points inside the chunk, before it, and a single split."""
    from mlx_motif import _native

    _native.set_tuning("rows_per_split", rps)
    try:
        _check(gpu, rng, 1, 130, 8, 4, 8, 70, 256)
    finally:
        _native.set_tuning("rows_per_split", 0)


def test_prefill_four_and_eight_wave_blocks(gpu, rng):
    from mlx_motif import _native

    for w in (4, 8):
        _native.set_tuning("waves_per_wg", w)
        try:
            _check(gpu, rng, 1, 160, 8, 4, 8, 300, 512)
        finally:
            _native.set_tuning("waves_per_wg", 0)


@pytest.mark.parametrize("ncb", [1, 2])
@pytest.mark.parametrize("S,offset,cap,rps,tag", [
    (160, 300, 512, 0, "f16"),      # 640 origin heads per KV head: one ragged 256-head block
    (130, 70, 256, 64, "f16"),      # many splits, tiles dealt round robin, the chunk's tiles among them
    (200, 1000, 1280, 0, "bf16"),
])
def test_prefill_column_blocks_per_wave(gpu, rng, ncb, S, offset, cap, rps, tag):
    """8-wave blocks with one or two 16-head column blocks per wave."""
    from mlx_motif import _native

    _native.set_tuning("prefill_ncb", ncb)
    _native.set_tuning("rows_per_split", rps)
    try:
        _check(gpu, rng, 1, S, 8, 4, 8, offset, cap, tag=tag)
    finally:
        _native.set_tuning("prefill_ncb", 0)
        _native.set_tuning("rows_per_split", 0)
