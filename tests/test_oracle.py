"""Pins of the CPU oracle (oracle/oracle.py) — each check is independent of
the formula it tests: a library routine, a brute-force loop, a closed form,
an invariant of the format, the reference's own golden vector, or the second
(C) restatement.  CPU only.
"""

from __future__ import annotations

import json
import math
import pathlib

import numpy as np
import pytest

from oracle import c_oracle
from oracle import oracle as O

GOLDEN = pathlib.Path(__file__).parent / "golden"


def _f16(rng, shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float16)


# ---------------------------------------------------------------- sdpa ---

def test_sdpa_matches_torch_sdpa_float64(rng):
    """An independent library routine: torch's scaled_dot_product_attention."""
    import torch

    B, Hq, Hkv, S, D, kv = 2, 8, 2, 1, 64, 77
    q, k, v1, v2 = _f16(rng, (B, Hq, S, D)), *(_f16(rng, (B, Hkv, kv, D)) for _ in range(3))
    y = O.sdpa_dual_v(q, k, v1, v2, 0.125)
    G = Hq // Hkv
    t = lambda a: torch.from_numpy(np.repeat(a.astype(np.float64), G, axis=1))  # noqa: E731
    tq = torch.from_numpy(q.astype(np.float64))
    a1 = torch.nn.functional.scaled_dot_product_attention(tq, t(k), t(v1), scale=0.125)
    a2 = torch.nn.functional.scaled_dot_product_attention(tq, t(k), t(v2), scale=0.125)
    np.testing.assert_allclose(y, torch.cat([a1, a2], -1).numpy(), rtol=1e-12, atol=1e-12)


def test_causal_rows_match_torch_masked_sdpa(rng):
    import torch

    B, H, S, D, kv = 1, 4, 5, 32, 40
    q, k, v1, v2 = _f16(rng, (B, H, S, D)), *(_f16(rng, (B, H, kv, D)) for _ in range(3))
    y = O.sdpa_dual_v(q, k, v1, v2, 0.3, causal=True)
    mask = torch.ones(S, kv, dtype=torch.bool).tril(diagonal=kv - S)  # bottom-right aligned
    t = lambda a: torch.from_numpy(a.astype(np.float64))  # noqa: E731
    a1 = torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v1), attn_mask=mask,
                                                          scale=0.3)
    np.testing.assert_allclose(y[..., :D], a1.numpy(), rtol=1e-12, atol=1e-12)


def test_sdpa_brute_force_scalar_loop(rng):
    q, k, v1, v2 = _f16(rng, (1, 2, 1, 8)), *(_f16(rng, (1, 1, 5, 8)) for _ in range(3))
    y = O.sdpa_dual_v(q, k, v1, v2, 0.5, kv_len=4)
    for h in range(2):
        s = [0.5 * sum(float(q[0, h, 0, d]) * float(k[0, 0, j, d]) for d in range(8))
             for j in range(4)]
        w = [math.exp(x - max(s)) for x in s]
        for d in range(8):
            e1 = sum(w[j] * float(v1[0, 0, j, d]) for j in range(4)) / sum(w)
            e2 = sum(w[j] * float(v2[0, 0, j, d]) for j in range(4)) / sum(w)
            assert abs(y[0, h, 0, d] - e1) < 1e-12 and abs(y[0, h, 0, 8 + d] - e2) < 1e-12


def test_sdpa_closed_forms(rng):
    q, k, v1, v2 = _f16(rng, (1, 4, 1, 32)), *(_f16(rng, (1, 4, 9, 32)) for _ in range(3))
    # one live key -> that key's value rows
    y = O.sdpa_dual_v(q, k, v1, v2, 0.2, kv_len=1)
    np.testing.assert_array_equal(y[..., :32], np.broadcast_to(v1[:, :, :1], y[..., :32].shape))
    np.testing.assert_array_equal(y[..., 32:], np.broadcast_to(v2[:, :, :1], y[..., 32:].shape))
    # equal keys -> uniform weights -> mean of the values
    kk = np.broadcast_to(k[:, :, :1], k.shape).copy()
    y = O.sdpa_dual_v(q, kk, v1, v2, 0.2)
    np.testing.assert_allclose(y[..., :32], v1.astype(np.float64).mean(axis=2, keepdims=True),
                               rtol=1e-12, atol=1e-12)
    # kv_len = 0 -> zeros (the kernel's o = 0 when l = 0)
    assert not O.sdpa_dual_v(q, k, v1, v2, 0.2, kv_len=0).any()


def test_sdpa_invariants(rng):
    q = _f16(rng, (1, 8, 1, 64))
    k, v = _f16(rng, (1, 2, 50, 64)), _f16(rng, (1, 2, 50, 64))
    y = O.sdpa_dual_v(q, k, v, v, 0.1)
    np.testing.assert_array_equal(y[..., :64], y[..., 64:])  # V1 = V2 -> equal halves
    # GQA broadcast == explicitly repeated K/V (repeat-interleave of heads)
    rep = lambda a: np.repeat(a, 4, axis=1)  # noqa: E731
    np.testing.assert_allclose(y, O.sdpa_dual_v(q, rep(k), rep(v), rep(v), 0.1), atol=0, rtol=0)
    # rows past kv_len never matter
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 30:] = 1e4
    v2[:, :, 30:] = -1e4
    np.testing.assert_array_equal(O.sdpa_dual_v(q, k, v, v, 0.1, kv_len=30),
                                  O.sdpa_dual_v(q, k2, v2, v2, 0.1, kv_len=30))


def test_c_port_matches_numpy(rng):
    q, k, v1, v2 = _f16(rng, (1, 16, 1, 128)), *(_f16(rng, (1, 4, 300, 128)) for _ in range(3))
    y = c_oracle.sdpa_dual_v_f16(q, k, v1, v2, 1 / np.sqrt(128), kv_len=257)
    np.testing.assert_allclose(y, O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(128), 257), atol=2e-6)
    q5 = _f16(rng, (1, 16, 5, 128))
    y = c_oracle.sdpa_dual_v_f16(q5, k, v1, v2, 0.09, kv_len=200, causal=True)
    np.testing.assert_allclose(y, O.sdpa_dual_v(q5, k, v1, v2, 0.09, 200, causal=True),
                               atol=2e-6)
    kq, vq1, vq2 = (O.quantize(t, 64, 4) for t in (k, v1, v2))
    y = c_oracle.sdpa_dual_v_q_f16(q, kq, vq1, vq2, 0.09, 64, 4, kv_len=299)
    np.testing.assert_allclose(y, O.sdpa_dual_v_q(q, kq, vq1, vq2, 0.09, 64, 4, 299), atol=2e-6)


# ------------------------------------------------------------ quantizer ---

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantizer_format_invariants(rng, bits, gs):
    x = _f16(rng, (3, 5, 256), 2.0)
    data, scales, biases = O.quantize(x, gs, bits)
    codes = O.unpack_codes(data, bits).reshape(3, 5, 256 // gs, gs)
    n_bins = 2 ** bits - 1
    assert codes.min() >= 0 and codes.max() <= n_bins
    xg = x.astype(np.float32).reshape(3, 5, 256 // gs, gs)
    edge_is_min = np.abs(xg.min(-1)) > np.abs(xg.max(-1))
    edge = np.where(edge_is_min, xg.min(-1), xg.max(-1))
    # the edge element gets code 0 and the bias is the edge (rounded to fp16)
    at_edge = np.take_along_axis(codes, np.argmax(xg == edge[..., None], -1)[..., None], -1)
    assert (at_edge == 0).all()
    np.testing.assert_array_equal(biases.astype(np.float32),
                                  edge.astype(np.float16).astype(np.float32))
    # reconstruction in the format's fp32 arithmetic: codes strictly inside
    # (0, n_bins) are within half a step of the input; refitting the scale to
    # make the edge exact can shrink the far end of the range, where codes
    # clamp at n_bins, by at most one more step.
    d32, s32, b32 = O.quantize(x, gs, bits, out_dtype="f32")
    c32 = O.unpack_codes(d32, bits).reshape(xg.shape)
    recon = (s32.astype(np.float64)[..., None] * c32 + b32.astype(np.float64)[..., None])
    step = np.abs(s32.astype(np.float64))[..., None]
    err = np.abs(recon - xg)
    inner = (c32 > 0) & (c32 < n_bins)
    # (w - bias) / scale is rounded to fp32 before rint, and exact ties do occur
    # with fp16 inputs, so allow that rounding on top of half a step
    slack = 2.0 ** -22 * np.abs(xg - b32.astype(np.float64)[..., None])
    assert (err[inner] <= (0.5 * step + slack)[inner]).all()
    assert (err <= 1.5 * step + slack).all()


def test_quantizer_zero_reconstructs_when_the_group_straddles_it():
    """With bias = edge and scale = edge / q0, code -q0 decodes to exactly 0 in
    the fp32 arithmetic of the format."""
    w = np.linspace(-3.0, 1.5, 64).astype(np.float16)
    w[10] = 0.0
    data, s32, b32 = O.quantize(w[None], 64, 4, out_dtype="f32")
    code = O.unpack_codes(data, 4)[0, 10]
    assert np.float32(s32[0, 0]) * np.float32(code) + np.float32(b32[0, 0]) == 0.0


def test_quantizer_special_groups():
    zeros = O.quantize(np.zeros((1, 64), np.float16), 64, 4)
    assert not zeros[0].any() and zeros[2][0, 0] == 0
    # all-zero group: scale is -1e-7 (max side, eps floor), rounded to fp16
    assert zeros[1][0, 0] == np.float16(-1e-7)
    const = O.quantize(np.full((1, 64), 3.0, np.float16), 64, 8)
    assert np.all(O.dequantize(*const, 64, 8) == 3.0)


def test_quantizer_hand_worked_group():
    """w = 0..31 (gs 32, 4 bits): max side, scale = 31/-15, bias = 31,
    code(w) = rint((w - 31) / scale) = rint((31 - w) * 15 / 31)."""
    w = np.arange(32, dtype=np.float16)[None]
    data, s, b = O.quantize(w, 32, 4, out_dtype="f32")
    assert b[0, 0] == np.float32(31.0)
    assert s[0, 0] == np.float32(31.0) / np.float32(-15.0)
    codes = O.unpack_codes(data, 4)[0]
    assert codes[0] == 15 and codes[31] == 0 and codes[16] == 7 and codes[15] == 8


@pytest.mark.parametrize("bits", [4, 8])
def test_quantizer_batched_equals_per_slot(rng, bits):
    """Head-axis concat + one quantisation == per-slot quantisation
    (the invariant of reference tests/test_grouped_cache.py:168)."""
    slots = [_f16(rng, (1, 8, 5, 128)) for _ in range(4)]
    d, s, b = O.quantize(np.concatenate(slots, axis=1), 64, bits)
    for i, x in enumerate(slots):
        di, si, bi = O.quantize(x, 64, bits)
        np.testing.assert_array_equal(d[:, 8 * i:8 * (i + 1)], di)
        np.testing.assert_array_equal(s[:, 8 * i:8 * (i + 1)], si)
        np.testing.assert_array_equal(b[:, 8 * i:8 * (i + 1)], bi)


@pytest.mark.parametrize("bits,tol", [(4, 0.5), (8, 0.05)])
def test_quantizer_roundtrip_tolerance(rng, bits, tol):
    """Reference tests/test_grouped_cache.py:112-129 (N(0, 0.1), atol=rtol=tol)."""
    x = _f16(rng, (1, 8, 5, 128), 0.1)
    np.testing.assert_allclose(O.dequantize(*O.quantize(x, 64, bits), 64, bits),
                               x.astype(np.float64), atol=tol, rtol=tol)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantizer_c_restatement_bit_identical(rng, bits, gs):
    x = _f16(rng, (4, 7, 256), 3.0)
    for a, b in zip(O.quantize(x, gs, bits), c_oracle.quantize_f16(x, gs, bits)):
        np.testing.assert_array_equal(np.asarray(a).view(np.uint16) if a.dtype == np.float16
                                      else a, np.asarray(b).view(np.uint16)
                                      if b.dtype == np.float16 else b)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_bit_extract_loop(rng, bits):
    """Little-endian code order and s*u+b (probe contract, mlp.py:165-198),
    checked by a scalar loop over words and bit positions."""
    x = _f16(rng, (2, 64))
    data, s, b = O.quantize(x, 32, bits)
    y = O.dequantize(data, s, b, 32, bits, out_dtype="f16")
    el = 32 // bits
    for r in range(2):
        for i in range(64):
            word = int(data[r, i // el])
            u = (word >> ((i % el) * bits)) & ((1 << bits) - 1)
            ref = np.float16(np.float32(s[r, i // 32]) * np.float32(u) + np.float32(b[r, i // 32]))
            assert y[r, i] == ref


def test_round_to_bf16():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.14159, 65504.0, 1e-40], np.float32)
    r = O.round_to(x, "bf16")
    assert r[0] == 1.0 and r[1] == 1.0  # tie -> even
    assert r[2] == np.float32(1.0078125)
    np.testing.assert_allclose(r[:5], x[:5], rtol=2 ** -8)
    assert abs(r[5] - x[5]) <= 2.0 ** -133  # subnormal: half of bf16's subnormal spacing


# ------------------------------------------------------------ epilogues ---

def test_polynorm_reference_golden_vector():
    case = json.loads((GOLDEN / "polynorm_reference_2x3.json").read_text())
    y = O.polynorm(np.array(case["input"]), case["weight"], case["bias"], case["eps"])
    np.testing.assert_allclose(y, np.array(case["expected"]), rtol=1e-13, atol=1e-13)


def test_gda_closed_forms(rng):
    o = rng.standard_normal((1, 8, 3, 64))
    n = rng.standard_normal((1, 2, 3, 64))
    w = np.full(64, 1.7)
    y = O.gda_post_split(o, n, w, 0.3, 0.6, 4, 0.0)
    # constant weight: each row's RMS is |w * (1 - lambda_init)|
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.7 * 0.4, rtol=1e-12)
    # lambda = 0: RMSNorm of o
    y0 = O.gda_post_split(o, n, np.ones(64), 0.0, 0.0, 4, 0.0)
    np.testing.assert_allclose(y0, o / np.sqrt((o * o).mean(-1, keepdims=True)), rtol=1e-12)
    # gr broadcast == explicit repeat with gr = 1
    np.testing.assert_allclose(y, O.gda_post_split(o, np.repeat(n, 4, axis=1), w, 0.3, 0.6, 1,
                                                   0.0), rtol=0, atol=0)
    # merged layout == split layout
    m = np.concatenate([o, n], axis=1)
    np.testing.assert_array_equal(O.gda_post(m, w, 0.3, 0.6, 2, 4, 0.0), y)


def test_gda_decode_attention_per_head_loop(rng):
    """The decode-step composition against an explicit per-head loop over
    the reference's three calls (model.py:749-768): torch's float64 SDPA for
    each origin head h (k1 of KV head h // gr) and noise head (k2), outputs
    rounded to fp16, then a scalar RMS-norm epilogue."""
    import torch

    B, Hkv, gr, D, kv, cap = 2, 2, 3, 32, 9, 12
    q1 = _f16(rng, (B, Hkv * gr, 1, D))
    q2 = _f16(rng, (B, Hkv, 1, D))
    k1, k2, v1, v2 = (_f16(rng, (B, Hkv, cap, D)) for _ in range(4))
    w = _f16(rng, (2 * D,))
    lam, lam_init, eps, scale = 0.37, 0.55, 1e-5, 0.2
    y = O.gda_decode_attention(q1, q2, k1, k2, v1, v2, scale, w, lam, lam_init, gr, eps,
                               kv_len=kv)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    t = lambda a: torch.from_numpy(a.astype(np.float64))  # noqa: E731

    def att(q, k, j, b):
        qs = t(q)[None, None]
        ks = t(k[b, j, :kv])[None, None]
        a1 = sdpa(qs, ks, t(v1[b, j, :kv])[None, None], scale=scale)
        a2 = sdpa(qs, ks, t(v2[b, j, :kv])[None, None], scale=scale)
        o = torch.cat([a1, a2], -1).numpy().reshape(-1)
        return o.astype(np.float32).astype(np.float16).astype(np.float64)

    lam32 = float(np.float32(lam))
    for b in range(B):
        for h in range(Hkv * gr):
            j = h // gr
            o = att(q1[b, h, 0], k1, j, b)
            n = att(q2[b, j, 0], k2, j, b)
            d = o - lam32 * n
            ref = d / math.sqrt(float(np.mean(d * d)) + eps) * w.astype(np.float64) * (1 - lam_init)
            np.testing.assert_allclose(y[b, h, 0], ref, rtol=1e-10, atol=1e-12)


def test_lambda_formulas():
    assert abs(O.lambda_init(1) - 0.2) < 1e-15
    assert abs(O.lambda_init(1000) - 0.8) < 1e-12
    lq1, lk1, lq2, lk2 = (np.full(4, 0.1), np.full(4, 0.2), np.zeros(4), np.zeros(4))
    assert abs(O.lambda_full(lq1, lk1, lq2, lk2, 0.2) - (math.exp(0.08) - 1 + 0.2)) < 1e-15


# ----------------------------------------------------------------- RoPE ---
def test_rope_closed_form_on_two_channels(rng):
    """D = 2: one pair rotated by angle = position (theta^0 = 1)."""
    x = rng.standard_normal((1, 5, 3, 2))
    y = O.rope(x, 7, 10000.0)
    ang = 7 + np.arange(5)
    c, s = np.cos(ang)[None, :, None], np.sin(ang)[None, :, None]
    np.testing.assert_allclose(y[..., 0], x[..., 0] * c - x[..., 1] * s, atol=1e-12)
    np.testing.assert_allclose(y[..., 1], x[..., 1] * c + x[..., 0] * s, atol=1e-12)


def test_rope_identity_norms_and_relative_position(rng):
    D = 128
    x = rng.standard_normal((2, 1, 4, D))
    np.testing.assert_array_equal(O.rope(x, 0), x)  # position 0: identity
    y = O.rope(x, 1234)
    half = D // 2
    n_x = x[..., :half] ** 2 + x[..., half:] ** 2
    n_y = y[..., :half] ** 2 + y[..., half:] ** 2
    np.testing.assert_allclose(n_y, n_x, rtol=1e-12)  # each pair keeps its norm
    q, k = rng.standard_normal((1, 1, 1, D)), rng.standard_normal((1, 1, 1, D))
    d1 = np.sum(O.rope(q, 500) * O.rope(k, 480))
    d2 = np.sum(O.rope(q, 9020) * O.rope(k, 9000))
    assert abs(d1 - d2) < 1e-9 * (1 + abs(d1))  # depends on m - n only
    # the frequency of pair i is theta^(-2i/D): pair 1 at position 1
    e = np.zeros((1, 1, 1, D))
    e[..., 1] = 1.0
    r = O.rope(e, 1)
    w = 10000.0 ** (-2.0 / D)
    np.testing.assert_allclose([r[0, 0, 0, 1], r[0, 0, 0, half + 1]], [np.cos(w), np.sin(w)])


def test_rope_split4_head_mapping_explicit_loop(rng):
    """The split against a per-head index loop (model.py:620-629, 669-679)."""
    B, S, qg, gr, kg, kr, D = 2, 3, 2, 3, 2, 1, 32
    q = rng.standard_normal((B, S, qg * (gr + 1) * D))
    k = rng.standard_normal((B, S, kg * (kr + 1) * D))
    v = rng.standard_normal((B, S, 2 * kg * D))
    q1, q2, k1, k2, v1, v2 = O.rope_split4(q, k, v, qg, gr, kg, kr, 5)
    qr = O.rope(q.reshape(B, S, -1, D), 5)
    kr_ = O.rope(k.reshape(B, S, -1, D), 5)
    vv = v.reshape(B, S, -1, D)
    for b in range(B):
        for s in range(S):
            for g in range(qg):
                for j in range(gr):
                    np.testing.assert_array_equal(q1[b, g * gr + j, s], qr[b, s, g * (gr + 1) + j])
                np.testing.assert_array_equal(q2[b, g, s], qr[b, s, g * (gr + 1) + gr])
            for g in range(kg):
                np.testing.assert_array_equal(k1[b, g, s], kr_[b, s, 2 * g])
                np.testing.assert_array_equal(k2[b, g, s], kr_[b, s, 2 * g + 1])
                np.testing.assert_array_equal(v1[b, g, s], vv[b, s, 2 * g])
                np.testing.assert_array_equal(v2[b, g, s], vv[b, s, 2 * g + 1])
    o1, o2, *_ = O.rope_split4(q, k, v, qg, gr, kg, kr, 5, origin_first=True)
    np.testing.assert_array_equal(o1, qr.transpose(0, 2, 1, 3)[:, : qg * gr])
    np.testing.assert_array_equal(o2, qr.transpose(0, 2, 1, 3)[:, qg * gr:])


def test_gda_prefill_from_proj_per_head_loop(rng):
    """The prefill-chunk composition against an explicit loop over the
    reference's steps (model.py:590-629 rope + 4-slot write, 769-797 four
    causal SDPA calls): for each origin head h (KV head of q1 head h under
    the GQA broadcast) and noise head, torch's float64 SDPA over the cache
    with the chunk written, query row s seeing rows [0, offset + s]."""
    import torch

    B, S, qg, gr, kg, D, offset, cap = 2, 3, 4, 2, 2, 32, 5, 12
    f16 = lambda x: O.round_to(x, "f16").astype(np.float64)  # noqa: E731
    q = f16(rng.standard_normal((B, S, qg * (gr + 1) * D)))
    k = f16(rng.standard_normal((B, S, 2 * kg * D)))
    v = f16(rng.standard_normal((B, S, 2 * kg * D)))
    caches = [f16(rng.standard_normal((B, kg, cap, D))) for _ in range(4)]
    scale = 0.17
    y_o, y_n, slots = O.gda_prefill_from_proj(q, k, v, caches, offset, qg, gr, kg, scale)
    qr = f16(O.rope(q.reshape(B, S, -1, D), offset))
    kr_ = f16(O.rope(k.reshape(B, S, -1, D), offset))
    vv = v.reshape(B, S, -1, D)
    cache = [c.copy() for c in caches]
    for b in range(B):
        for s in range(S):
            for g in range(kg):
                cache[0][b, g, offset + s] = kr_[b, s, 2 * g]
                cache[1][b, g, offset + s] = kr_[b, s, 2 * g + 1]
                cache[2][b, g, offset + s] = vv[b, s, 2 * g]
                cache[3][b, g, offset + s] = vv[b, s, 2 * g + 1]
    for a, c in zip(slots, cache):
        np.testing.assert_array_equal(a, c)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    t = torch.from_numpy
    kv = offset + S
    mask = t(np.arange(kv)[None, :] <= offset + np.arange(S)[:, None])

    def att(qrows, kslot, j, b):
        qs = t(qrows)[None, None]
        ks = t(cache[kslot][b, j, :kv])[None, None]
        a1 = sdpa(qs, ks, t(cache[2][b, j, :kv])[None, None], attn_mask=mask, scale=scale)
        a2 = sdpa(qs, ks, t(cache[3][b, j, :kv])[None, None], attn_mask=mask, scale=scale)
        return torch.cat([a1, a2], -1).numpy()[0, 0]

    G_o, G_n = qg * gr // kg, qg // kg
    for b in range(B):
        for h in range(qg * gr):  # q1 head h = group h // gr, slot h % gr
            qrows = qr[b, :, (h // gr) * (gr + 1) + h % gr]
            np.testing.assert_allclose(y_o[b, h], att(qrows, 0, h // G_o, b), rtol=1e-12,
                                       atol=1e-12)
        for h in range(qg):
            qrows = qr[b, :, h * (gr + 1) + gr]
            np.testing.assert_allclose(y_n[b, h], att(qrows, 1, h // G_n, b), rtol=1e-12,
                                       atol=1e-12)


def test_vectorised_c_port_matches_scalar_build():
    """The -O3 -ffast-math build of the C port (timed by bench.py's CPU
    baseline only) computes what the scalar checker build computes, to
    fp32 reassociation error."""
    from oracle import c_oracle

    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 8, 1, 128)).astype(np.float16)
    k, v1, v2 = (rng.standard_normal((1, 2, 700, 128)).astype(np.float16) for _ in range(3))
    a = c_oracle.sdpa_dual_v_f16(q, k, v1, v2, 128 ** -0.5, 650)
    b = c_oracle.sdpa_dual_v_f16(q, k, v1, v2, 128 ** -0.5, 650, fast=True)
    assert np.max(np.abs(a - b)) <= 1e-5
    trips = [c_oracle.quantize_f16(t, 64, 4) for t in (k, v1, v2)]
    a = c_oracle.sdpa_dual_v_q_f16(q, *trips, 128 ** -0.5, 64, 4, 650)
    b = c_oracle.sdpa_dual_v_q_f16(q, *trips, 128 ** -0.5, 64, 4, 650, fast=True)
    assert np.max(np.abs(a - b)) <= 1e-5


def test_rope_linear_scaling_pins():
    """The oracle's RoPE position scale (a "linear" scaling config of factor f
    ropes position p at p / f): at scale 1/2 position 2p equals position p
    unscaled, scale 1 is the unscaled RoPE, and scale 2 (the inverse, a
    plausible mistake) differs."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 1, 3, 64))
    for p in (0, 7, 1601):
        np.testing.assert_allclose(O.rope(x, 2 * p, scale=0.5), O.rope(x, p), rtol=0, atol=1e-12)
        np.testing.assert_array_equal(O.rope(x, p, scale=1.0), O.rope(x, p))
    assert np.max(np.abs(O.rope(x, 10, scale=2.0) - O.rope(x, 5))) > 1e-3
