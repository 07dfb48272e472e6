"""CPU oracle of the Motif decode-attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for ``cpu_baseline``, as the timed CPU restatement).  The product
(``mlx-motif_amd/``) never imports or calls it.

Each function restates what the reference computes for one row of the hot
path, in numpy, citing the reference file:line it follows (paths relative to
the junhoyeo/mlx-motif tree).  Floating-point work is done in float64 so the
oracle sits well inside every tolerance; the quantizer and dequantizer are
done in float32, step by step, because their outputs are compared bit for
bit.

Element types: numpy has no bfloat16, so bf16 data travels as float32 arrays
holding bf16-representable values; ``round_to(x, "bf16")`` rounds to the
nearest bf16 (ties to even) in that representation.

How each function is pinned (tests/test_oracle.py):
  sdpa_dual_v        torch.nn.functional.scaled_dot_product_attention in
                     float64 (an independent library routine), brute-force
                     scalar loops on tiny inputs, closed forms (one key ->
                     its value row; equal keys -> mean of values), V1=V2
                     halves, GQA == pre-repeated K/V.
  sdpa_dual_v_q      sdpa_dual_v on dequantize()'d inputs + the above.
  quantize           invariants that fix the affine format: codes in
                     [0, 2^bits-1], the edge element's code is 0 and
                     reconstructs exactly in fp32, zero reconstructs exactly
                     when the group straddles it, per-element error <=
                     |scale|/2, batched == per-slot (reference
                     tests/test_grouped_cache.py:168), round-trip tolerance
                     (tests/test_grouped_cache.py:112).  The exact rounding of
                     MLX 0.31.2's mx.quantize (not in this tree, not
                     importable here) is PARITY UNPINNED: the restatement
                     follows MLX's published CPU quantizer.
  dequantize         bit layout pinned by the probe contract
                     (src/mlx_motif/kernels/mlp.py:165-198: little-endian
                     codes, no zero point) and a scalar bit-extract loop.
  gda_post_split     closed form: rows of the output have RMS equal to
                     |w*(1-lambda_init)| when w is constant; lambda=0 reduces
                     to RMSNorm; gr broadcasting == explicit repeat.
  gda_decode_attention
                     a composition of the two functions above (pinned as
                     stated), in the order and with the rounding points of
                     model.py:749-768; checked against an explicit per-head
                     loop over the reference's three calls on a tiny shape.
  polynorm           the reference's only numeric golden vector
                     (tests/fixtures/motif_parity_cases.json,
                     component_checks[0]).
  gda_prefill_from_proj
                     a composition of rope_split4 and sdpa_dual_v (pinned as
                     stated), in the order of model.py:590-629 and 769-797;
                     checked against an explicit per-head loop over the
                     reference's four causal SDPA calls (torch float64) on a
                     tiny shape.
  rope / rope_split4 the rotation's closed form on D = 2 (angle = position),
                     position 0 is the identity, every channel pair keeps
                     its norm, and q(m).k(n) depends on m - n only; the split
                     is checked against an explicit per-head index loop.
                     The exact cos/sin and angle rounding of mlx_lm's
                     initialize_rope / mx.fast.rope (not in this tree, not
                     importable here) are PARITY UNPINNED: the restatement
                     is the textbook non-traditional RoPE in float64.
"""

from __future__ import annotations

import numpy as np

# ------------------------------------------------------------ elements ---


def round_to(x, dtype: str) -> np.ndarray:
    """Round float values to fp16 / bf16 / fp32 (returned as float32 arrays,
    or float16 for "f16")."""
    x = np.asarray(x)
    if dtype == "f16":
        return x.astype(np.float32).astype(np.float16)
    if dtype == "f32":
        return x.astype(np.float32)
    if dtype == "bf16":
        u = np.ascontiguousarray(x.astype(np.float32)).view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        r = np.where(nan, (u >> 16) | 0x40, r)
        return (r.astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dtype)


# ------------------------------------------------------------ quantizer ---


def _round_ties(t: np.ndarray, ties: str) -> np.ndarray:
    """Round float32 t to integers: ``"even"`` is round-half-even (rint);
    ``"away"`` sends exact halves away from zero (C ``round``).  Only exact
    halves differ; they are found as t - trunc(t) == +-0.5, which is exact in
    float32."""
    r = np.rint(t).astype(np.float32)
    if ties == "even":
        return r
    assert ties == "away", ties
    f = np.trunc(t).astype(np.float32)
    half = np.abs(t - f) == np.float32(0.5)
    return np.where(half, f + np.sign(t), r).astype(np.float32)


def quantize(w, group_size: int = 64, bits: int = 4, out_dtype: str = "f16", ties: str = "even"):
    """MLX affine quantisation of the last axis (what ``mx.quantize`` computes
    for cache.py:498 and cache.py:399-402), in float32 step by step:

        n_bins = 2^bits - 1
        scale  = max((max - min) / n_bins, 1e-7)
        side   = |min| > |max|;  scale = side ? scale : -scale
        edge   = side ? min : max;  q0 = rint(edge / scale)
        if q0 != 0: scale = edge / q0; bias = edge   else bias = 0
        code   = clamp(rint((w - bias) / scale), 0, n_bins)

    ``ties`` picks the rounding of exact halves in both rint steps: "even"
    (the default, MLX's CPU quantizer) or "away" (C ``round``), so tests can
    bound what an unknown tie rule would change.

    Returns (data uint32 (..., D*bits/32), scales, biases (..., D/gs)) with
    scales/biases rounded to ``out_dtype``.  Codes are packed little-endian:
    value i of a row at bits [(i % (32/bits))*bits, +bits) of word
    i // (32/bits) (src/mlx_motif/kernels/mlp.py:165-168).
    """
    w = np.asarray(w)
    *lead, D = w.shape
    assert bits in (4, 8) and D % group_size == 0
    el = 32 // bits
    x = w.astype(np.float32).reshape(-1, D // group_size, group_size)
    n_bins = np.float32((1 << bits) - 1)
    w_max = x.max(axis=-1)
    w_min = x.min(axis=-1)
    scale = np.maximum((w_max - w_min) / n_bins, np.float32(1e-7)).astype(np.float32)
    side = np.abs(w_min) > np.abs(w_max)
    scale = np.where(side, scale, -scale).astype(np.float32)
    edge = np.where(side, w_min, w_max).astype(np.float32)
    q0 = _round_ties((edge / scale).astype(np.float32), ties)
    nz = q0 != 0
    safe_q0 = np.where(nz, q0, np.float32(1)).astype(np.float32)
    scale = np.where(nz, edge / safe_q0, scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
    codes = _round_ties(((x - bias[..., None]) / scale[..., None]).astype(np.float32), ties)
    codes = np.clip(codes, np.float32(0), n_bins).astype(np.uint32)
    codes = codes.reshape(-1, D // el, el)
    words = np.zeros(codes.shape[:-1], dtype=np.uint32)
    for i in range(el):
        words |= codes[..., i] << np.uint32(bits * i)
    g = D // group_size
    return (
        words.reshape(*lead, D // el),
        round_to(scale, out_dtype).reshape(*lead, g),
        round_to(bias, out_dtype).reshape(*lead, g),
    )


def unpack_codes(data, bits: int) -> np.ndarray:
    """Unsigned codes (..., D) from packed words (..., D*bits/32)."""
    data = np.asarray(data, dtype=np.uint32)
    el = 32 // bits
    shifts = (np.arange(el, dtype=np.uint32) * np.uint32(bits)).astype(np.uint32)
    codes = (data[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(*data.shape[:-1], data.shape[-1] * el)


def dequantize(data, scales, biases, group_size: int = 64, bits: int = 4, out_dtype=None):
    """``float32(scale) * code + float32(bias)`` in float32 (the dequant probe
    formula, src/mlx_motif/kernels/mlp.py:196), rounded to ``out_dtype`` when
    given ("f16" / "bf16" / "f32"), else returned as float64 exact values."""
    codes = unpack_codes(data, bits)
    *lead, D = codes.shape
    g = D // group_size
    c = codes.reshape(*lead, g, group_size)
    if out_dtype is None:
        s = np.asarray(scales, dtype=np.float64)[..., None]
        b = np.asarray(biases, dtype=np.float64)[..., None]
        return (s * c + b).reshape(*lead, D)
    s = np.asarray(scales, dtype=np.float32)[..., None]
    b = np.asarray(biases, dtype=np.float32)[..., None]
    y = (s * c.astype(np.float32)).astype(np.float32) + b
    return round_to(y.astype(np.float32).reshape(*lead, D), out_dtype)


def quant_write4(slots, k1, k2, v1, v2, offset: int, group_size: int, bits: int,
                 out_dtype: str = "f16"):
    """Per-slot quantisation of the new rows into four cache triples at rows
    [offset, offset+S): the pre-batching write the reference test keeps as
    its oracle (tests/test_grouped_cache.py:131-163).  ``slots`` is a list of
    4 (data, scales, biases) numpy arrays updated in place."""
    S = np.asarray(k1).shape[2]
    for new, (d, s, b) in zip((k1, k2, v1, v2), slots):
        qd, qs, qb = quantize(new, group_size, bits, out_dtype)
        d[:, :, offset:offset + S] = qd
        s[:, :, offset:offset + S] = qs
        b[:, :, offset:offset + S] = qb


# ------------------------------------------------------------- attention ---


def sdpa_dual_v(q, k, v1, v2, scale: float, kv_len=None, causal: bool = False) -> np.ndarray:
    """Shared-QK dual-V attention in float64.

    Follows the reference path of sdpa_dual_v (attention.py:217-229 and
    181-187): slice K/V1/V2 to the live rows, repeat each KV head
    H_q/H_kv times (repeat-interleave), y = cat(softmax(scale q K^T) V1,
    softmax(scale q K^T) V2).  With ``causal`` and S_q query rows, row i sees
    keys [0, kv_len - S_q + i] (bottom-right alignment of the "causal" mask
    the multi-row fallback uses, model.py:769-807).  Rows that see no key
    come out zero, as the decode kernel returns o = 0 when l == 0
    (attention.py:149).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v1 = np.asarray(v1, dtype=np.float64)
    v2 = np.asarray(v2, dtype=np.float64)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if kv_len is None:
        kv_len = k.shape[2]
    k, v1, v2 = k[:, :, :kv_len], v1[:, :, :kv_len], v2[:, :, :kv_len]
    G = Hq // Hkv
    k, v1, v2 = (np.repeat(t, G, axis=1) for t in (k, v1, v2))
    y = np.zeros((B, Hq, S, 2 * D))
    if kv_len == 0:
        return y
    s = np.einsum("bhsd,bhkd->bhsk", q * scale, k)
    if causal:
        rows = np.arange(S)[:, None]
        cols = np.arange(kv_len)[None, :]
        visible = cols <= kv_len - S + rows
    else:
        visible = np.ones((S, kv_len), dtype=bool)
    s = np.where(visible, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.where(visible, np.exp(s - m), 0.0)
    l = p.sum(axis=-1, keepdims=True)
    o1 = np.einsum("bhsk,bhkd->bhsd", p, v1)
    o2 = np.einsum("bhsk,bhkd->bhsd", p, v2)
    lz = np.where(l == 0, 1.0, l)
    y[..., :D] = o1 / lz
    y[..., D:] = o2 / lz
    return y


def sdpa_dual_v_q(q, k_q, v1_q, v2_q, scale: float, group_size: int = 64, bits: int = 4,
                  kv_len=None, causal: bool = False, dequant_dtype=None) -> np.ndarray:
    """sdpa_dual_v on dequantised K, V1, V2: the reference path of
    sdpa_dual_v_q4 (attention.py:473-507).  ``dequant_dtype`` rounds the
    dequantised values like ``mx.dequantize`` does; None keeps them exact
    (what an fp32-accumulating kernel consumes)."""
    if kv_len is None:
        kv_len = np.asarray(k_q[0]).shape[2]
    sl = lambda t: tuple(np.asarray(x)[:, :, :kv_len] for x in t)  # noqa: E731
    k = dequantize(*sl(k_q), group_size=group_size, bits=bits, out_dtype=dequant_dtype)
    v1 = dequantize(*sl(v1_q), group_size=group_size, bits=bits, out_dtype=dequant_dtype)
    v2 = dequantize(*sl(v2_q), group_size=group_size, bits=bits, out_dtype=dequant_dtype)
    return sdpa_dual_v(q, k, v1, v2, scale, kv_len, causal)


# ------------------------------------------------------------ epilogues ---


def gda_post_split(attn_o, attn_n, subln_w, lambda_full: float, lambda_init: float, gr: int,
                   eps: float) -> np.ndarray:
    """Float64 GDA epilogue (gda.py:207-220):
    d = o - lambda * repeat(n, gr); y = d * rsqrt(mean(d^2) + eps) * w * (1 - lambda_init).
    ``subln_w`` is expected already rounded to the activation dtype (the
    wrapper casts it, gda.py:263); ``lambda_full`` is an fp32 value."""
    o = np.asarray(attn_o, dtype=np.float64)
    n = np.repeat(np.asarray(attn_n, dtype=np.float64), gr, axis=1)
    lam = float(np.float32(lambda_full))
    d = o - lam * n
    rms_inv = 1.0 / np.sqrt((d * d).mean(axis=-1, keepdims=True) + eps)
    return d * rms_inv * np.asarray(subln_w, dtype=np.float64) * (1.0 - lambda_init)


def gda_post(merged, subln_w, lambda_full: float, lambda_init: float, q_groups: int, gr: int,
             eps: float) -> np.ndarray:
    """Merged-layout epilogue (gda.py:108-124): origin heads first, then noise."""
    m = np.asarray(merged)
    q_origin = q_groups * gr
    return gda_post_split(m[:, :q_origin], m[:, q_origin:], subln_w, lambda_full, lambda_init,
                          gr, eps)


def gda_decode_attention(q1, q2, k1, k2, v1, v2, scale: float, subln_w, lambda_full: float,
                         lambda_init: float, gr: int, eps: float, kv_len=None,
                         dtype: str = "f16") -> np.ndarray:
    """One GDA decode-attention step, the DUAL_V path of model.py:749-768:
    attn_origin = sdpa_dual_v(q1, k1, v1, v2), attn_noise = sdpa_dual_v(q2,
    k2, v1, v2), both returned in the activation dtype by the reference's
    kernels (so rounded to ``dtype`` here), then gda_post_split with gr
    origin heads per noise head.  Returns float64 (round once to compare)."""
    o = round_to(sdpa_dual_v(q1, k1, v1, v2, scale, kv_len), dtype)
    n = round_to(sdpa_dual_v(q2, k2, v1, v2, scale, kv_len), dtype)
    return gda_post_split(o, n, subln_w, lambda_full, lambda_init, gr, eps)


def polynorm(x, weight, bias, eps: float) -> np.ndarray:
    """Float64 PolyNorm (mlp.py:108-116):
    y = w0*rms(x^3) + w1*rms(x^2) + w2*rms(x) + b, rms(z) = z/sqrt(mean(z^2)+eps)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64).reshape(-1)
    b = float(np.asarray(bias, dtype=np.float64).reshape(-1)[0])

    def rms(z):
        return z / np.sqrt((z * z).mean(axis=-1, keepdims=True) + eps)

    return w[0] * rms(x ** 3) + w[1] * rms(x ** 2) + w[2] * rms(x) + b


# ----------------------------------------------------- model constants ---


def lambda_init(layer_idx: int) -> float:
    """model.py:389: lambda_init = 0.8 - 0.6 * exp(-0.3 * (layer_idx - 1))."""
    return 0.8 - 0.6 * float(np.exp(-0.3 * (layer_idx - 1)))


def lambda_full(lq1, lk1, lq2, lk2, lam_init: float) -> float:
    """model.py:462-470 in float64: exp(sum(lq1*lk1)) - exp(sum(lq2*lk2)) + lambda_init."""
    l1 = np.exp(np.sum(np.asarray(lq1, np.float64) * np.asarray(lk1, np.float64)))
    l2 = np.exp(np.sum(np.asarray(lq2, np.float64) * np.asarray(lk2, np.float64)))
    return float(l1 - l2 + lam_init)


# ----------------------------------------------------------------- RoPE ---


def rope(x, pos0: int, theta: float = 10000.0, scale: float = 1.0) -> np.ndarray:
    """Non-traditional RoPE (model.py:413-419: initialize_rope(head_dim,
    traditional=False, scaling_config=rope_scaling); applied at
    model.py:590-594) on x (B, S, H, D) in float64: channel pairs (i, i + D/2)
    rotated by (scale * (pos0 + s)) * theta^(-2i/D).  scale is 1 unscaled and
    1 / factor for a "linear" scaling config (mlx-lm's initialize_rope builds
    nn.RoPE(..., scale=1 / factor) for it)."""
    x = np.asarray(x, np.float64)
    B, S, H, D = x.shape
    half = D // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / D)
    pos = (pos0 + np.arange(S, dtype=np.float64)) * float(scale)
    ang = pos[:, None] * inv[None, :]  # (S, half)
    c = np.cos(ang)[None, :, None, :]
    s_ = np.sin(ang)[None, :, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s_, x2 * c + x1 * s_], axis=-1)


def rope_split4(q, k, v, q_groups: int, gr: int, k_groups: int, kr: int, pos0: int,
                theta: float = 10000.0, origin_first: bool = False, scale: float = 1.0):
    """model.py:580-594 (reshape to heads, rope q and k), 620-629 (k1/k2 and
    v1/v2 split of the 4-slot cache write) and 669-679 (q1/q2 split).  q (B,
    S, HQ*D), k (B, S, HK*D), v (B, S, 2*k_groups*D).  Returns float64
    (q1, q2, k1, k2, v1, v2), each (B, H, S, D)."""
    q = np.asarray(q, np.float64)
    B, S, _ = q.shape
    HQ = q_groups * (gr + 1)
    HK = k_groups * (kr + 1)
    D = q.shape[-1] // HQ
    qr = rope(q.reshape(B, S, HQ, D), pos0, theta, scale).transpose(0, 2, 1, 3)  # (B, HQ, S, D)
    kr_ = rope(np.asarray(k, np.float64).reshape(B, S, HK, D), pos0, theta,
               scale).transpose(0, 2, 1, 3)
    vv = np.asarray(v, np.float64).reshape(B, S, 2 * k_groups, D).transpose(0, 2, 1, 3)
    if origin_first:
        q1, q2 = qr[:, : q_groups * gr], qr[:, q_groups * gr:]
    else:
        q_ = qr.reshape(B, q_groups, gr + 1, S, D)
        q1 = q_[:, :, :gr].reshape(B, q_groups * gr, S, D)
        q2 = q_[:, :, gr:].reshape(B, q_groups, S, D)
    k_ = kr_.reshape(B, k_groups, kr + 1, S, D)
    k1 = k_[:, :, :kr].reshape(B, k_groups * kr, S, D)
    k2 = k_[:, :, kr:].reshape(B, k_groups, S, D)
    v_ = vv.reshape(B, k_groups, 2, S, D)
    return q1, q2, k1, k2, v_[:, :, 0], v_[:, :, 1]


def gda_prefill_from_proj(q, k, v, caches, offset: int, q_groups: int, gr: int, k_groups: int,
                          scale: float, theta: float = 10000.0, origin_first: bool = False,
                          dtype: str = "f16", position_scale: float = 1.0):
    """A GDA layer's prefill chunk on the k_ratio-1 fallback path: rope q and k
    at positions offset + s (model.py:590-594), split and write the 4-slot
    cache rows offset .. offset + S - 1 (model.py:620-629, update_and_fetch_4),
    split q1/q2 (model.py:669-679), then the four causal SDPA calls, concatenated
    per pass (model.py:769-797): origin = [q1 over (k1, V1) || q1 over (k1, V2)],
    noise = the same for q2 over k2 (positions scaled by ``position_scale``
    for a linear RoPE scaling config).  The roped q/k are rounded to ``dtype``
    (the reference's rope output has the activation dtype).  ``caches`` is
    (k1, k2, v1, v2), each (B, k_groups, cap, D).  Returns float64 (y_origin,
    y_noise, the four written cache slots)."""
    q1, q2, k1n, k2n, v1n, v2n = rope_split4(q, k, v, q_groups, gr, k_groups, 1, offset, theta,
                                             origin_first, position_scale)

    def rnd(x):
        return round_to(x, dtype).astype(np.float64)

    S = q1.shape[2]
    slots = [np.array(c, dtype=np.float64, copy=True) for c in caches]
    for c, new in zip(slots, (k1n, k2n, v1n, v2n)):
        c[:, :, offset:offset + S] = rnd(new)
    kv_len = offset + S
    y_o = sdpa_dual_v(rnd(q1), slots[0], slots[2], slots[3], scale, kv_len, causal=True)
    y_n = sdpa_dual_v(rnd(q2), slots[1], slots[2], slots[3], scale, kv_len, causal=True)
    return y_o, y_n, slots
