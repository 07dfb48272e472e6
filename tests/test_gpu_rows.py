"""Parity of the multi-row dual-V path (speculative verify / chunked prefill):
``motif_sdpa_dual_v_rows`` and ``motif_sdpa_dual_v_q_rows`` against the
oracle's bottom-right causal attention (the FALLBACK composition of
model.py:769-807 with mask "causal").

Includes the verify slab of the 12.7B layer: K+1 = 5 query rows per head, 32
q-heads over 8 KV heads, head_dim 128, over a q8 cache of 32768 rows.
Tolerance: fp16 max |gpu - oracle| <= 2e-3.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,Hq,Hkv,S,cap,kv_len,d,causal", [
    (1, 32, 8, 5, 512, 300, 128, True),
    (1, 32, 8, 5, 512, 5, 128, True),
    (2, 8, 8, 3, 256, 200, 64, True),
    (1, 40, 8, 4, 1024, 1000, 128, False),
    (1, 16, 4, 7, 256, 256, 128, True),
])
def test_rows_fp16(gpu, rng, B, Hq, Hkv, S, cap, kv_len, d, causal):
    from mlx_motif.kernels import sdpa_dual_v_rows

    q = randn(rng, (B, Hq, S, d), "f16")
    k, v1, v2 = (randn(rng, (B, Hkv, cap, d), "f16") for _ in range(3))
    for t in (k, v1, v2):
        t[:, :, kv_len:] = 1e4
    T = lambda a: np_to_torch(a, torch_dtype("f16"), gpu)  # noqa: E731
    y = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(d), kv_len=kv_len, causal=causal)
    assert y.shape == (B, Hq, S, 2 * d)
    ref = O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(d), kv_len, causal=causal)
    assert np.max(np.abs(torch_to_np(y) - ref)) <= 2e-3


@pytest.mark.parametrize("tag,S,Hq,cap,kv_len,min_heads", [
    ("f16", 4, 32, 1024, 1000, 0),      # 16 virtual heads per KV head: one 16-column chunk
    ("f16", 5, 32, 32768, 32768, 64),   # the 5-row verify slab at 32k rows: chunks of 16 + 4
    ("f16", 5, 32, 32768, 32768, 0),    # the same on the shared-tile kernel (the default)
    ("bf16", 5, 32, 512, 300, 0),       # bf16 matrix cores, 16 + 4
    ("bf16", 5, 32, 4096, 4001, 0),     # bf16, shared tiles (20 heads over 2048+ rows)
    ("bf16", 3, 40, 640, 600, 0),       # GQA 5 x 3 rows = 15 columns
])
def test_rows_sixteen_column_chunks(gpu, rng, tag, S, Hq, cap, kv_len, min_heads):
    """fp16/bf16 slabs at head_dim 128: the matrix-core decode kernel with up
    to 16 virtual heads per workgroup, or, from 17 heads over 2048+ rows,
    the shared-tile kernel (min_heads 64 keeps the decode kernel)."""
    from mlx_motif import _native
    from mlx_motif.kernels import sdpa_dual_v_rows

    q = randn(rng, (1, Hq, S, 128), tag)
    k, v1, v2 = (randn(rng, (1, 8, cap, 128), tag) for _ in range(3))
    T = lambda a: np_to_torch(a, torch_dtype(tag), gpu)  # noqa: E731
    print(f"rows {tag} S={S} Hq={Hq} kv_len={kv_len} min_heads={min_heads}", flush=True)
    _native.set_tuning("prefill_min_heads", min_heads)
    try:
        y = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(128), kv_len=kv_len,
                             causal=True)
        torch_y = torch_to_np(y)
    finally:
        _native.set_tuning("prefill_min_heads", 0)
    ref = O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(128), kv_len, causal=True)
    err = float(np.max(np.abs(torch_y - ref)))
    assert err <= (2e-3 if tag == "f16" else 1e-2), f"{tag} S={S}: {err:.3e}"


def test_rows_single_row_equals_decode(gpu, rng):
    """S_q = 1 with the causal mask is the decode kernel's computation."""
    from mlx_motif.kernels import sdpa_dual_v, sdpa_dual_v_rows

    q = randn(rng, (1, 32, 1, 128), "f16")
    k, v1, v2 = (randn(rng, (1, 8, 700, 128), "f16") for _ in range(3))
    T = lambda a: np_to_torch(a, torch_dtype("f16"), gpu)  # noqa: E731
    a = torch_to_np(sdpa_dual_v(T(q), T(k), T(v1), T(v2), 0.088, kv_len=650))
    b = torch_to_np(sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 0.088, kv_len=650, causal=True))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("S,cap,kv_len", [(5, 512, 400), (3, 256, 3), (4, 512, 300)])
def test_rows_packed(gpu, rng, bits, S, cap, kv_len):
    """S x GQA 4 virtual heads: 12 and 16 take the two-column-block kernel
    (one workgroup per KV head and split), 20 the slab kernel for q8 (tiles
    dequantised into LDS once per workgroup) and three head chunks for q4."""
    from mlx_motif.kernels import sdpa_dual_v_q4_rows

    q = randn(rng, (1, 32, S, 128), "f16")
    trips = [O.quantize(randn(rng, (1, 8, cap, 128), "f16"), 64, bits) for _ in range(3)]
    G = lambda t: (np_to_torch(t[0], None, gpu), np_to_torch(t[1], torch_dtype("f16"), gpu),  # noqa: E731
                   np_to_torch(t[2], torch_dtype("f16"), gpu))
    y = sdpa_dual_v_q4_rows(np_to_torch(q, torch_dtype("f16"), gpu), *(G(t) for t in trips),
                            1 / np.sqrt(128), group_size=64, bits=bits, kv_len=kv_len)
    ref = O.sdpa_dual_v_q(q, *trips, 1 / np.sqrt(128), 64, bits, kv_len, causal=True)
    assert np.max(np.abs(torch_to_np(y) - ref)) <= 2e-3


def test_verify_slab_q8_32k(gpu, rng):
    """5 query rows, q8 cache of 32768 rows (all live, the 5 new rows included)."""
    from mlx_motif.kernels import sdpa_dual_v_q4_rows

    S, cap = 5, 32768
    q = randn(rng, (1, 32, S, 128), "f16")
    trips = [O.quantize(randn(rng, (1, 8, cap, 128), "f16"), 64, 8) for _ in range(3)]
    G = lambda t: (np_to_torch(t[0], None, gpu), np_to_torch(t[1], torch_dtype("f16"), gpu),  # noqa: E731
                   np_to_torch(t[2], torch_dtype("f16"), gpu))
    y = sdpa_dual_v_q4_rows(np_to_torch(q, torch_dtype("f16"), gpu), *(G(t) for t in trips),
                            1 / np.sqrt(128), group_size=64, bits=8, kv_len=cap)
    y = torch_to_np(y)
    ref = O.sdpa_dual_v_q(q, *trips, 1 / np.sqrt(128), 64, 8, cap, causal=True)
    assert np.max(np.abs(y - ref)) <= 2e-3
    # The reference path dequantises to fp16 first (cache.py:448-465 then
    # mx.fast SDPA, model.py:769-807): within the same bar of that too.
    ref16 = O.sdpa_dual_v_q(q, *trips, 1 / np.sqrt(128), 64, 8, cap, causal=True,
                            dequant_dtype="f16")
    assert np.max(np.abs(y - ref16)) <= 2e-3


@pytest.mark.parametrize("bits", [4, 8])
def test_two_column_blocks_decode_group_size_32(gpu, rng, bits):
    """GQA 6 at group size 32: 6 heads x 4 scale groups need two column
    blocks of 4 heads in one workgroup."""
    from mlx_motif.kernels import sdpa_dual_v_q4

    q = randn(rng, (1, 48, 1, 128), "f16")
    trips = [O.quantize(randn(rng, (1, 8, 512, 128), "f16"), 32, bits) for _ in range(3)]
    G = lambda t: (np_to_torch(t[0], None, gpu), np_to_torch(t[1], torch_dtype("f16"), gpu),  # noqa: E731
                   np_to_torch(t[2], torch_dtype("f16"), gpu))
    y = sdpa_dual_v_q4(np_to_torch(q, torch_dtype("f16"), gpu), *(G(t) for t in trips),
                       1 / np.sqrt(128), group_size=32, bits=bits, kv_len=437)
    ref = O.sdpa_dual_v_q(q, *trips, 1 / np.sqrt(128), 32, bits, 437)
    assert np.max(np.abs(torch_to_np(y) - ref)) <= 2e-3
