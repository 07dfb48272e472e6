"""Packed-cache verify slabs of 17..64 virtual heads per KV head (query rows x
GQA), which run on the slab kernel: each packed tile is dequantised once per
workgroup into LDS, rounded to fp16 as the reference path's mx.dequantize
output is (src/mlx_motif/kernels/attention.py:497-499), then attended on fp16
matrix cores with fp32 accumulation.

Bars: max |gpu - oracle| <= 2e-3 against the oracle at that rounding point
(``dequant_dtype="f16"``) and against exact dequant; the same bar against the
head-chunk / column-block kernels (tuning ``qslab`` 0); the 8-wave kernel
with producer and consumer waves (dequantisation in packed fp16 beside the
attention), the 8-wave kernel whose waves share each step, and the 4-wave
variant.
Shapes: 20 (the 5-row x GQA 4 slab), 17, 32, 36 and 64 virtual heads, group
sizes 32/64/128, q4 and q8, causal and not, batch 2, short and odd kv_len,
poisoned padding rows.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=[(0, 1, 2), (0, 1, 3), (0, 0, 2), (4, 1, 2)],
                ids=["w8_roles", "w8_roles_3sets", "w8", "w4"])
def slab_kernel(request):
    """Every slab on the slab kernel (qslab 2: 4-bit slabs too): 8 waves as
    producers and consumers (default, and with three producer register
    sets), 8 waves sharing every step's work, and 4 waves."""
    from mlx_motif import _native

    waves, roles, sets = request.param
    _native.set_tuning("qslab", 2)
    _native.set_tuning("waves_per_wg", waves)
    _native.set_tuning("qslab_ws", roles)
    _native.set_tuning("qslab_sets", sets)
    yield
    _native.set_tuning("qslab", 2)
    _native.set_tuning("waves_per_wg", 0)
    _native.set_tuning("qslab_ws", 1)
    _native.set_tuning("qslab_sets", 2)

_CASES = [
    # B, Hq, Hkv, S, cap, kv_len, causal, bits, gs
    (1, 32, 8, 5, 1024, 1000, True, 8, 64),
    (1, 32, 8, 5, 640, 37, True, 4, 64),
    (2, 16, 4, 5, 512, 300, True, 4, 32),
    (1, 32, 8, 8, 2048, 2048, True, 8, 128),
    (1, 32, 8, 9, 1024, 777, True, 4, 64),
    (1, 64, 8, 8, 512, 500, False, 8, 64),
    (1, 8, 8, 17, 320, 290, True, 8, 64),
    (1, 32, 8, 5, 4096, 4001, False, 4, 128),
]


def _slab(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal, bits, gs):
    from mlx_motif.kernels import sdpa_dual_v_q4_rows

    q = randn(rng, (B, Hq, S, 128), "f16")
    raw = [randn(rng, (B, Hkv, cap, 128), "f16") for _ in range(3)]
    for t in raw:
        t[:, :, kv_len:] = 1e3  # padding rows: must not be seen
    trips = [O.quantize(t, gs, bits) for t in raw]
    G = lambda t: (np_to_torch(t[0], None, gpu), np_to_torch(t[1], torch_dtype("f16"), gpu),  # noqa: E731
                   np_to_torch(t[2], torch_dtype("f16"), gpu))
    gt = [G(t) for t in trips]
    qt = np_to_torch(q, torch_dtype("f16"), gpu)
    call = lambda: torch_to_np(sdpa_dual_v_q4_rows(qt, *gt, 1 / np.sqrt(128), group_size=gs,  # noqa: E731
                                                   bits=bits, kv_len=kv_len, causal=causal))
    return q, trips, call


@pytest.mark.parametrize("B,Hq,Hkv,S,cap,kv_len,causal,bits,gs", _CASES)
def test_slab_matches_oracle_and_previous_kernels(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal,
                                                  bits, gs):
    from mlx_motif import _native

    print(f"slab B={B} Hq={Hq} Hkv={Hkv} S={S} kv_len={kv_len} causal={causal} bits={bits} "
          f"gs={gs}", flush=True)
    q, trips, call = _slab(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal, bits, gs)
    y = call()
    assert np.isfinite(y).all()
    scale = 1 / np.sqrt(128)
    ref16 = O.sdpa_dual_v_q(q, *trips, scale, gs, bits, kv_len, causal=causal,
                            dequant_dtype="f16")
    exact = O.sdpa_dual_v_q(q, *trips, scale, gs, bits, kv_len, causal=causal)
    err16 = float(np.max(np.abs(y - ref16)))
    err = float(np.max(np.abs(y - exact)))
    assert err16 <= 2e-3 and err <= 2e-3, (err16, err)
    _native.set_tuning("qslab", 0)
    try:
        print("  previous kernels (qslab 0)", flush=True)
        y0 = call()
    finally:
        _native.set_tuning("qslab", 2)
    assert float(np.max(np.abs(y - y0))) <= 2e-3


def test_slab_split_count_forced(gpu, rng):
    """Forced small splits (many partials for the merge launch) and a single
    split give the same output within the bar."""
    from mlx_motif import _native

    q, trips, call = _slab(gpu, rng, 1, 32, 8, 5, 2048, 1999, True, 8, 64)
    ys = []
    for rps in (0, 64, 4096):
        _native.set_tuning("rows_per_split", rps)
        try:
            print(f"slab rows_per_split={rps}", flush=True)
            ys.append(call())
        finally:
            _native.set_tuning("rows_per_split", 0)
    ref16 = O.sdpa_dual_v_q(q, *trips, 1 / np.sqrt(128), 64, 8, 1999, causal=True,
                            dequant_dtype="f16")
    for y in ys:
        assert float(np.max(np.abs(y - ref16))) <= 2e-3
