"""Parity of the fused GDA decode step (``motif_gda_decode``) against the
oracle composition of the reference's three calls (model.py:749-768:
sdpa_dual_v for the origin heads, sdpa_dual_v for the noise heads, both
returned in the activation dtype, then gda_post_split), and against the
separately validated native calls.

The fused path runs for fp16 and bf16 at head_dim 128 (columns G + 1 = 2 ..
16 per KV head, both the 8-wave and the 4-wave variants); fp32, other head
dims and mfma=0 take the composed path inside the library.

Bar: the attention outputs carry the dual-V kernels' own bar (max |o -
o_exact| <= 2e-3 for fp16, 1e-2 bf16, 1e-5 fp32; tests/test_gpu_sdpa.py),
and the epilogue normalises d = o - lambda*n to unit RMS, so an error e in o
moves y by about rsqrt(mean d^2) * |w| * (1 - lambda_init) * e.  Per
element, |gpu - ref| <= rms_inv |w| s (E + lambda E) + 2 ulp(y) + 1e-5 with
E that attention bar; on top, the mean error must stay below a tenth of the
mean bar (no systematic offset).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ULP = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7, "f32": 2.0 ** -23}
ATT = {"f16": 2e-3, "bf16": 1e-2, "f32": 1e-5}  # dual-V attention bars


def _ulp(x, tag):
    mag = np.maximum(np.abs(x), 2.0 ** -14)
    return ULP[tag] * 2.0 ** np.floor(np.log2(mag))


def _case(rng, B, Hkv, gr, cap, D, tag, poison_from=None):
    q1 = randn(rng, (B, Hkv * gr, 1, D), tag)
    q2 = randn(rng, (B, Hkv, 1, D), tag)
    ks = [randn(rng, (B, Hkv, cap, D), tag) for _ in range(4)]
    if poison_from is not None:
        for t in ks:
            t[:, :, poison_from:] = 1e4
    w = randn(rng, (2 * D,), tag)
    return q1, q2, ks, w


def _bar(q1, q2, k1, k2, v1, v2, w, scale, lam, lam_init, gr, eps, kv_len, tag):
    """Oracle y and the per-element bar of the module docstring."""
    o = O.sdpa_dual_v(q1, k1, v1, v2, scale, kv_len)
    n = O.sdpa_dual_v(q2, k2, v1, v2, scale, kv_len)
    orr, nr = O.round_to(o, tag), O.round_to(n, tag)
    y = O.gda_post_split(orr, nr, w, lam, lam_init, gr, eps)
    d = np.asarray(orr, np.float64) - float(np.float32(lam)) * np.repeat(
        np.asarray(nr, np.float64), gr, axis=1)
    rms_inv = 1.0 / np.sqrt((d * d).mean(axis=-1, keepdims=True) + eps)
    tol = (rms_inv * np.abs(np.asarray(w, np.float64)) * (1 - lam_init) * (1 + lam) * ATT[tag]
           + 2 * _ulp(y, tag) + 1e-5)
    return y, tol


def _run(gpu, rng, B, Hkv, gr, cap, kv_len, D, tag, poison=False):
    import torch

    from mlx_motif.kernels import gda_decode_attention

    q1, q2, (k1, k2, v1, v2), w = _case(rng, B, Hkv, gr, cap, D, tag,
                                        kv_len if poison else None)
    dt = torch_dtype(tag)
    T = [np_to_torch(a, dt, gpu) for a in (q1, q2, k1, k2, v1, v2, w)]
    scale, lam, lam_init, eps = 1.0 / np.sqrt(D), 0.4321, 0.2, 1e-5
    lam_t = torch.tensor([lam], dtype=torch.float32, device=gpu)
    print(f"gda_decode B={B} Hkv={Hkv} gr={gr} cap={cap} kv_len={kv_len} D={D} {tag}", flush=True)
    y = gda_decode_attention(*T[:6], scale, T[6], lam_t, lam_init, gr, eps, kv_len=kv_len)
    torch.cuda.synchronize()
    assert y.shape == (B, Hkv * gr, 1, 2 * D) and y.dtype == dt
    ref, tol = _bar(q1, q2, k1, k2, v1, v2, w, scale, lam, lam_init, gr, eps, kv_len, tag)
    got = torch_to_np(y)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert float(err.mean()) <= 0.1 * float(tol.mean()) + 1e-6, (err.mean(), tol.mean())
    excess = float(np.max(err - tol))
    return excess, y, T, (scale, lam_t, lam_init, eps)


@pytest.mark.parametrize("kv_len", [1, 17, 300, 1024, 3204])
def test_fused_decode_12p7b_heads(gpu, rng, kv_len):
    """32 origin heads over 8 KV heads (gr 4) + 8 noise heads, head_dim 128."""
    cap = (kv_len + 255) // 256 * 256
    excess, *_ = _run(gpu, rng, 1, 8, 4, cap, kv_len, 128, "f16")
    assert excess <= 0, f"kv_len={kv_len}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("B,Hkv,gr", [(1, 4, 1), (2, 2, 2), (1, 2, 3), (1, 3, 7), (1, 2, 15)])
def test_fused_decode_column_counts(gpu, rng, B, Hkv, gr):
    """G + 1 columns of 2, 3 (-> 4), 4, 8 and 16 (the 4-wave variant)."""
    excess, *_ = _run(gpu, rng, B, Hkv, gr, 256, 200, 128, "f16")
    assert excess <= 0, f"B={B} Hkv={Hkv} gr={gr}: exceeds the bar by {excess:.3e}"


def test_fused_decode_ignores_poisoned_padding(gpu, rng):
    excess, *_ = _run(gpu, rng, 1, 8, 4, 512, 385, 128, "f16", poison=True)
    assert excess <= 0


def test_fused_decode_kv_len_zero(gpu, rng):
    """No live rows: both attention outputs are zero, so d = 0 and y = 0."""
    _, y, _, _ = _run(gpu, rng, 1, 8, 4, 256, 0, 128, "f16")
    assert not torch_to_np(y).any()


@pytest.mark.parametrize("kv_len,gr", [(1, 4), (300, 4), (3204, 4), (200, 15), (200, 1)])
def test_fused_decode_bf16(gpu, rng, kv_len, gr):
    """The bf16 cache on the bf16 matrix-core kernel (p rounded to bf16)."""
    cap = (kv_len + 255) // 256 * 256
    excess, *_ = _run(gpu, rng, 1, 8 if gr == 4 else 2, gr, cap, kv_len, 128, "bf16")
    assert excess <= 0, f"bf16 kv_len={kv_len} gr={gr}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("D,tag", [(64, "f16"), (64, "bf16"), (128, "f32"), (256, "f16")])
def test_composed_path_other_shapes(gpu, rng, D, tag):
    excess, *_ = _run(gpu, rng, 1, 4, 4, 256, 150, D, tag)
    assert excess <= 0, f"D={D} {tag}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("kv_len", [3204, 16000])
def test_fused_equals_separate_native_calls(gpu, rng, kv_len):
    """Full-size property: the fused step and the reference's three calls run
    through the separately validated native kernels agree to the bar's
    scale (one rounding of the attention outputs)."""
    import torch

    from mlx_motif.kernels import gda_decode_attention, gda_post_split, sdpa_dual_v

    cap = (kv_len + 127) // 128 * 128
    B, Hkv, gr, D = 1, 8, 4, 128
    dt = torch.float16
    g = torch.Generator(device=gpu)
    g.manual_seed(7)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).to(dt)  # noqa: E731
    q1, q2 = mk(B, Hkv * gr, 1, D), mk(B, Hkv, 1, D)
    k1, k2, v1, v2 = (mk(B, Hkv, cap, D) for _ in range(4))
    w = mk(2 * D)
    lam_t = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode fused vs separate kv_len={kv_len}", flush=True)
    y = gda_decode_attention(q1, q2, k1, k2, v1, v2, scale, w, lam_t, lam_init, gr, eps,
                             kv_len=kv_len)
    o = sdpa_dual_v(q1, k1, v1, v2, scale, kv_len=kv_len)
    n = sdpa_dual_v(q2, k2, v1, v2, scale, kv_len=kv_len)
    y2 = gda_post_split(o, n, w, lam_t, lam_init, gr, eps)
    torch.cuda.synchronize()
    a, b = torch_to_np(y), torch_to_np(y2)
    on, nn = torch_to_np(o), torch_to_np(n)
    d = on - 0.4321 * np.repeat(nn, gr, axis=1)
    rms_inv = 1.0 / np.sqrt((d * d).mean(axis=-1, keepdims=True) + eps)
    tol = (rms_inv * np.abs(torch_to_np(w)) * (1 - lam_init) * 1.4321 * ATT["f16"]
           + 2 * _ulp(b, "f16") + 1e-5)
    assert float(np.max(np.abs(a - b) - tol)) <= 0
    # Most elements are bit-identical: the two paths differ only where a
    # rescale decision moved an fp16 rounding of p.
    assert np.mean(a == b) > 0.5


def test_mfma_off_takes_composed_path(gpu, rng):
    from mlx_motif import _native

    _native.set_tuning("mfma", 0)
    try:
        excess, *_ = _run(gpu, rng, 1, 8, 4, 256, 200, 128, "f16")
    finally:
        _native.set_tuning("mfma", 1)
    assert excess <= 0


def test_disable_toggle_reference_matches_oracle(gpu, rng):
    """The *_reference twin (what MLX_MOTIF_DISABLE_KERNELS routes to)."""
    import torch

    from mlx_motif.kernels import gda_decode_attention_reference

    q1, q2, (k1, k2, v1, v2), w = _case(rng, 1, 2, 4, 64, 64, "f32")
    T = [torch.from_numpy(np.asarray(a, np.float32)).to(gpu) for a in (q1, q2, k1, k2, v1, v2, w)]
    lam_t = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    y = gda_decode_attention_reference(*T[:6], 0.125, T[6], lam_t, 0.2, 4, 1e-5, kv_len=50)
    ref = O.gda_decode_attention(q1, q2, k1, k2, v1, v2, 0.125, w, 0.4321, 0.2, 4, 1e-5, 50,
                                 dtype="f32")
    np.testing.assert_allclose(torch_to_np(y), ref, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------ packed cache ---
def _run_q(gpu, rng, B, Hkv, gr, cap, kv_len, D, bits, gs, tag, poison=False):
    import torch

    from mlx_motif.kernels import gda_decode_attention_q4

    q1, q2, ks, w = _case(rng, B, Hkv, gr, cap, D, tag)
    if poison:
        for t in ks:
            t[:, :, kv_len:] = 1e3
    trips = [O.quantize(t, gs, bits, out_dtype=tag) for t in ks]
    dt = torch_dtype(tag)
    gt = [(np_to_torch(d, None, gpu), np_to_torch(s, dt, gpu), np_to_torch(b, dt, gpu))
          for d, s, b in trips]
    scale, lam, lam_init, eps = 1.0 / np.sqrt(D), 0.4321, 0.2, 1e-5
    lam_t = torch.tensor([lam], dtype=torch.float32, device=gpu)
    print(f"gda_decode_q B={B} Hkv={Hkv} gr={gr} cap={cap} kv_len={kv_len} bits={bits} gs={gs} "
          f"{tag}", flush=True)
    y = gda_decode_attention_q4(np_to_torch(q1, dt, gpu), np_to_torch(q2, dt, gpu), *gt, scale,
                                np_to_torch(w, dt, gpu), lam_t, lam_init, gr, gs, bits, eps,
                                kv_len=kv_len)
    torch.cuda.synchronize()
    assert y.shape == (B, Hkv * gr, 1, 2 * D) and y.dtype == dt
    deq = [O.dequantize(*t, group_size=gs, bits=bits) for t in trips]
    ref, tol = _bar(q1, q2, *deq, w, scale, lam, lam_init, gr, eps, kv_len, tag)
    got = torch_to_np(y)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert float(err.mean()) <= 0.1 * float(tol.mean()) + 1e-6, (err.mean(), tol.mean())
    return float(np.max(err - tol))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("kv_len", [1, 64, 300, 3204])
def test_fused_decode_q_12p7b_heads(gpu, rng, bits, kv_len):
    cap = (kv_len + 255) // 256 * 256
    excess = _run_q(gpu, rng, 1, 8, 4, cap, kv_len, 128, bits, 64, "f16")
    assert excess <= 0, f"bits={bits} kv_len={kv_len}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("gr,gs", [(1, 32), (3, 32), (4, 128), (7, 64), (15, 128), (4, 32)])
def test_fused_decode_q_groups_and_columns(gpu, rng, gr, gs):
    """Fused for (gr+1 -> 2/4/8/16 columns) x (128/gs groups) <= 16; gr 4 at
    gs 32 needs 32 columns and takes the composed path."""
    excess = _run_q(gpu, rng, 1, 2, gr, 256, 200, 128, 4, gs, "f16")
    assert excess <= 0, f"gr={gr} gs={gs}: exceeds the bar by {excess:.3e}"


def test_fused_decode_q_poisoned_padding_and_bf16(gpu, rng):
    assert _run_q(gpu, rng, 1, 8, 4, 512, 385, 128, 4, 64, "f16", poison=True) <= 0
    assert _run_q(gpu, rng, 1, 4, 4, 256, 150, 128, 8, 64, "bf16") <= 0


@pytest.mark.parametrize("bits,gs,gr,kv_len", [
    (4, 64, 4, 1), (4, 64, 4, 300), (8, 64, 4, 3204), (4, 128, 4, 3204),
    (4, 32, 3, 300),    # 4 columns x 4 groups
    (8, 128, 15, 385),  # 16 columns x 1 group
])
def test_fused_decode_q_bf16(gpu, rng, bits, gs, gr, kv_len):
    """bf16 activations, scales and biases on the fused packed step: q
    scaled per head by a power of two into fp16 for the products, the K
    scale and bias terms in fp32 (one wave per SIMD)."""
    cap = (kv_len + 255) // 256 * 256
    Hkv = 8 if gr <= 4 else 2
    print(f"gda_decode_q bf16 bits={bits} gs={gs} gr={gr} kv_len={kv_len}", flush=True)
    excess = _run_q(gpu, rng, 1, Hkv, gr, cap, kv_len, 128, bits, gs, "bf16")
    assert excess <= 0, f"bits={bits} gs={gs} gr={gr} kv_len={kv_len}: exceeds the bar by {excess:.3e}"


# ---------------------------------------------------------- append (write) ---
def _append_inputs(gpu, B, Hkv, gr, cap, D, dt, seed):
    import torch

    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).to(dt)  # noqa: E731
    q1, q2 = mk(B, Hkv * gr, 1, D), mk(B, Hkv, 1, D)
    caches = [mk(B, Hkv, cap, D) for _ in range(4)]
    rows = [mk(B, Hkv, 1, D) for _ in range(4)]
    w = mk(2 * D)
    lam_t = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    return q1, q2, caches, rows, w, lam_t


@pytest.mark.parametrize("B,Hkv,gr,cap,kv_len,D,tag", [
    (1, 8, 4, 256, 1, 128, "f16"),       # the first token
    (1, 8, 4, 256, 16, 128, "f16"),      # last row of the first 16-row block
    (1, 8, 4, 256, 17, 128, "f16"),      # first row of the second block
    (1, 8, 4, 3328, 3204, 128, "f16"),
    (1, 8, 4, 16000, 16000, 128, "f16"),  # the last row of the capacity
    (2, 3, 1, 301, 301, 128, "f16"),     # 2 columns, capacity not a multiple of 16
    (1, 2, 15, 512, 385, 128, "f16"),    # 16 columns: the 4-wave kernel
    (1, 4, 4, 256, 150, 64, "f16"),      # composed: head_dim 64
    (1, 4, 4, 256, 150, 128, "bf16"),    # bf16 kernel
    (1, 4, 4, 256, 150, 128, "f32"),     # composed: fp32
])
def test_append_writes_row_then_attends(gpu, B, Hkv, gr, cap, kv_len, D, tag):
    """``new_kv`` stores the token's rows at row kv_len - 1 of each slot
    (bit-exact, nothing else touched) and the output is bit-identical to
    writing the rows first and running the step without append."""
    import torch

    from mlx_motif.kernels import gda_decode_attention

    dt = torch_dtype(tag)
    q1, q2, caches, rows, w, lam_t = _append_inputs(gpu, B, Hkv, gr, cap, D, dt, kv_len)
    for c in caches:
        c[:, :, kv_len - 1] = 1e4  # stale contents of the row being written
    expect = [c.clone() for c in caches]
    for c, r in zip(expect, rows):
        c[:, :, kv_len - 1:kv_len] = r
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode append B={B} Hkv={Hkv} gr={gr} cap={cap} kv_len={kv_len} D={D} {tag}",
          flush=True)
    y = gda_decode_attention(q1, q2, *caches, scale, w, lam_t, lam_init, gr, eps, kv_len=kv_len,
                             new_kv=rows)
    y_ref = gda_decode_attention(q1, q2, *expect, scale, w, lam_t, lam_init, gr, eps,
                                 kv_len=kv_len)
    torch.cuda.synchronize()
    for c, e in zip(caches, expect):
        assert torch.equal(c.view(torch.int16), e.view(torch.int16))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


def test_append_matches_oracle_step(gpu, rng):
    """Oracle check of an append step: the oracle's step over the cache with
    the new rows in place."""
    import torch

    from mlx_motif.kernels import gda_decode_attention

    B, Hkv, gr, cap, kv_len, D, tag = 1, 8, 4, 512, 300, 128, "f16"
    q1, q2, ks, w = _case(rng, B, Hkv, gr, cap, D, tag)
    rows = [randn(rng, (B, Hkv, 1, D), tag) for _ in range(4)]
    dt = torch_dtype(tag)
    T = [np_to_torch(a, dt, gpu) for a in (q1, q2, *ks, w)]
    R = [np_to_torch(a, dt, gpu) for a in rows]
    scale, lam, lam_init, eps = 1.0 / np.sqrt(D), 0.4321, 0.2, 1e-5
    lam_t = torch.tensor([lam], dtype=torch.float32, device=gpu)
    y = gda_decode_attention(*T[:6], scale, T[6], lam_t, lam_init, gr, eps, kv_len=kv_len,
                             new_kv=R)
    torch.cuda.synchronize()
    for k, r in zip(ks, rows):
        k[:, :, kv_len - 1:kv_len] = r
    ref, tol = _bar(q1, q2, *ks, w, scale, lam, lam_init, gr, eps, kv_len, tag)
    assert float(np.max(np.abs(torch_to_np(y) - ref) - tol)) <= 0


@pytest.mark.parametrize("bits,gs,gr,cap,kv_len,tag", [
    (4, 64, 4, 256, 1, "f16"),
    (4, 64, 4, 256, 17, "f16"),
    (4, 64, 4, 3328, 3204, "f16"),
    (8, 64, 4, 16000, 16000, "f16"),
    (4, 32, 3, 300, 300, "f16"),      # 4 columns x 4 groups
    (8, 128, 15, 512, 385, "f16"),    # 16 columns x 1 group
    (4, 32, 4, 256, 200, "f16"),      # 32 columns: composed (quant_write4 first)
    (8, 64, 4, 256, 150, "bf16"),     # bf16 on the fused kernel
    (4, 64, 4, 3328, 3204, "bf16"),
])
def test_append_q_quantises_row_then_attends(gpu, bits, gs, gr, cap, kv_len, tag):
    """Packed cache: the token's rows are quantised into row kv_len - 1
    bit-exactly as the oracle quantizer does (data words, scales, biases;
    nothing else touched) and the output is bit-identical to the step without
    append over that cache."""
    import torch

    from mlx_motif.kernels import gda_decode_attention_q4, quantize

    B, Hkv, D = 1, 8 if gr <= 4 else 2, 128
    dt = torch_dtype(tag)
    q1, q2, caches, rows, w, lam_t = _append_inputs(gpu, B, Hkv, gr, cap, D, dt, kv_len + bits)
    trips = []
    for c in caches:  # the cache's other rows: any packed contents will do
        c[:, :, kv_len - 1] = 1e3
        trips.append(quantize(c, gs, bits))
    expect = [tuple(x.clone() for x in t) for t in trips]
    for t, r in zip(expect, rows):
        for dst, src in zip(t, O.quantize(torch_to_np(r), gs, bits, out_dtype=tag)):
            dst[:, :, kv_len - 1:kv_len] = np_to_torch(src, dst.dtype if dst.dtype != torch.uint32
                                                       else None, gpu)
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode_q append bits={bits} gs={gs} gr={gr} cap={cap} kv_len={kv_len} {tag}",
          flush=True)
    y = gda_decode_attention_q4(q1, q2, *trips, scale, w, lam_t, lam_init, gr, gs, bits, eps,
                                kv_len=kv_len, new_kv=rows)
    y_ref = gda_decode_attention_q4(q1, q2, *expect, scale, w, lam_t, lam_init, gr, gs, bits,
                                    eps, kv_len=kv_len)
    torch.cuda.synchronize()
    for t, e in zip(trips, expect):
        assert torch.equal(t[0].view(torch.int32), e[0].view(torch.int32))
        assert torch.equal(t[1].view(torch.int16), e[1].view(torch.int16))
        assert torch.equal(t[2].view(torch.int16), e[2].view(torch.int16))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


def test_append_rejects_kv_len_zero_and_strided_cache(gpu):
    import torch

    from mlx_motif.kernels import gda_decode_attention

    q1, q2, caches, rows, w, lam_t = _append_inputs(gpu, 1, 2, 2, 64, 128, torch.float16, 0)
    with pytest.raises(ValueError, match="appended row"):
        gda_decode_attention(q1, q2, *caches, 0.1, w, lam_t, 0.2, 2, kv_len=0, new_kv=rows)
    strided = caches[0].transpose(2, 3).contiguous().transpose(2, 3)
    with pytest.raises(ValueError, match="contiguous"):
        gda_decode_attention(q1, q2, strided, *caches[1:], 0.1, w, lam_t, 0.2, 2, kv_len=5,
                             new_kv=rows)
