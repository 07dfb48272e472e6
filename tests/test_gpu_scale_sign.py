"""Attention with a zero or negative softmax scale.

The reference's kernels take any float ``scale`` (attention.py:190-260,
510-645): q is scaled first, then the running maximum is taken over the
scaled scores.  The build's tile-softmax kernels (shared-tile prefill/slab,
packed slab, paired-tile decode, fused prefill chunk) take the maximum
over unscaled scores, which is only right for a positive scale; calls with
any other scale are routed to the per-tile kernels.  These tests run the
shapes that take each of those routes with scale -1/sqrt(128) and 0 and
hold the outputs to the oracle (fp16 max-abs 2e-3, bf16 1e-2).  Scale 0 gives every
visible key the same weight: y is the mean of the visible V rows.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3
SCALES = [-1.0 / np.sqrt(128.0), 0.0]


def _t(x, gpu):
    import torch

    return np_to_torch(x, torch.float16, gpu)


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("S_q,G,kv_len", [(16, 4, 600), (1, 32, 2304), (5, 4, 3000)])
def test_fp16_rows(gpu, rng, scale, S_q, G, kv_len):
    """fp16 cache: 64 virtual heads per KV head (the shared-tile route for a
    positive scale), 32 heads over 2304 rows (a decode call on that route),
    and a 5-row slab."""
    from mlx_motif.kernels import sdpa_dual_v_rows

    B, Hkv, D, cap = 1, 2, 128, kv_len + 37
    q = randn(rng, (B, Hkv * G, S_q, D), "f16")
    k, v1, v2 = (randn(rng, (B, Hkv, cap, D), "f16") for _ in range(3))
    y = sdpa_dual_v_rows(_t(q, gpu), _t(k, gpu), _t(v1, gpu), _t(v2, gpu), scale,
                         kv_len=kv_len, causal=True)
    ref = O.sdpa_dual_v(q, k, v1, v2, scale, kv_len=kv_len, causal=True)
    err = float(np.max(np.abs(torch_to_np(y) - ref)))
    assert np.all(np.isfinite(torch_to_np(y))) and err <= TOL, err


def _packed(rng, B, Hkv, cap, D, bits, tag="f16"):
    return [O.quantize(randn(rng, (B, Hkv, cap, D), tag), 64, bits, out_dtype=tag)
            for _ in range(3)]


def _gpu_trip(trip, gpu, tag="f16"):
    import torch

    dt = torch.float16 if tag == "f16" else torch.bfloat16
    d, s, b = trip
    return (np_to_torch(d, None, gpu), np_to_torch(s, dt, gpu), np_to_torch(b, dt, gpu))


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("tag", ["f16", "bf16"])
def test_packed_decode(gpu, rng, scale, bits, tag):
    """q4/q8 decode at group size 64 over 5000 rows, 32 heads over 8:
    fp16 (per-tile kernel) and bf16 (q4: the paired-tile route for a
    positive scale; q8: per-tile)."""
    import torch

    from mlx_motif.kernels import sdpa_dual_v_q4

    B, Hq, Hkv, D, kv_len, cap = 1, 32, 8, 128, 5000, 5120
    dt = torch.float16 if tag == "f16" else torch.bfloat16
    q = randn(rng, (B, Hq, 1, D), tag)
    kq, v1q, v2q = _packed(rng, B, Hkv, cap, D, bits, tag)
    y = sdpa_dual_v_q4(np_to_torch(q, dt, gpu), _gpu_trip(kq, gpu, tag), _gpu_trip(v1q, gpu, tag),
                       _gpu_trip(v2q, gpu, tag), scale, group_size=64, bits=bits, kv_len=kv_len)
    ref = O.sdpa_dual_v_q(q, kq, v1q, v2q, scale, 64, bits, kv_len)
    err = float(np.max(np.abs(torch_to_np(y) - ref)))
    assert np.all(np.isfinite(torch_to_np(y))) and err <= (TOL if tag == "f16" else 1e-2), err


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("bits", [4, 8])
def test_packed_slab(gpu, rng, scale, bits):
    """A 5-row verify slab of 20 virtual heads per KV head over a packed
    cache (the packed slab route for a positive scale), causal."""
    from mlx_motif.kernels import sdpa_dual_v_q4_rows

    B, Hq, Hkv, D, S_q, kv_len, cap = 1, 8, 2, 128, 5, 3000, 3072
    q = randn(rng, (B, Hq, S_q, D), "f16")
    kq, v1q, v2q = _packed(rng, B, Hkv, cap, D, bits)
    y = sdpa_dual_v_q4_rows(_t(q, gpu), _gpu_trip(kq, gpu), _gpu_trip(v1q, gpu),
                            _gpu_trip(v2q, gpu), scale, group_size=64, bits=bits,
                            kv_len=kv_len, causal=True)
    ref = O.sdpa_dual_v_q(q, kq, v1q, v2q, scale, 64, bits, kv_len, causal=True)
    err = float(np.max(np.abs(torch_to_np(y) - ref)))
    assert np.all(np.isfinite(torch_to_np(y))) and err <= TOL, err


@pytest.mark.parametrize("scale", SCALES)
def test_prefill_chunk_from_proj(gpu, rng, scale):
    """A layer's 64-row prefill chunk from the projections: the fused entry
    refuses the scale and the wrapper composes rope_split4 + two multi-row
    calls; the outputs match the oracle over the roped q and written cache."""
    from mlx_motif.kernels import gda_prefill_attention_from_proj, rope_split4

    B, S, qg, gr, kg, D, offset, cap = 1, 64, 8, 4, 4, 128, 700, 1024
    q = randn(rng, (B, S, qg * (gr + 1) * D), "f16")
    k = randn(rng, (B, S, 2 * kg * D), "f16")
    v = randn(rng, (B, S, 2 * kg * D), "f16")
    old = [randn(rng, (B, kg, cap, D), "f16") for _ in range(4)]
    caches = [_t(c, gpu) for c in old]
    yo, yn = gda_prefill_attention_from_proj(_t(q, gpu), _t(k, gpu), _t(v, gpu), caches, offset,
                                             qg, gr, kg, scale)
    # the roped queries, as the composed path computes them (fresh caches)
    scratch = [_t(c, gpu) for c in old]
    q1, q2, *_ = rope_split4(_t(q, gpu), _t(k, gpu), _t(v, gpu), qg, gr, kg, 1, offset, 10000.0,
                             False, caches=scratch)
    k1, k2, v1, v2 = (torch_to_np(c) for c in caches)
    kv_len = offset + S
    ref_o = O.sdpa_dual_v(torch_to_np(q1), k1, v1, v2, scale, kv_len=kv_len, causal=True)
    ref_n = O.sdpa_dual_v(torch_to_np(q2), k2, v1, v2, scale, kv_len=kv_len, causal=True)
    for y, ref in ((yo, ref_o), (yn, ref_n)):
        err = float(np.max(np.abs(torch_to_np(y) - ref)))
        assert np.all(np.isfinite(torch_to_np(y))) and err <= TOL, err
