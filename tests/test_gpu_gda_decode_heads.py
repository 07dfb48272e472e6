"""The GDA decode step for any noise-head count (``motif_gda_decode_heads``,
``motif_gda_decode_q_heads``): q2 with G2 noise heads per KV head, origin
head h paired with noise head h // gr (gr = Hq1 / Hq2), as the reference's
two GQA ``sdpa_dual_v`` calls and ``gda_post_split`` compute it
(model.py:749-768; gda.py:248).  The small step of 8 origin and 8 noise
heads over 4 KV heads at 1024 rows (gr 1) is the reference's CPU-runnable
decode step.

Checks, against the oracle composition with the bar of
tests/test_gpu_gda_decode.py (attention within its kernels' bar, then the
epilogue's amplification):
  - the small step at 1..3204 rows, fp16 and bf16, on the fused launch
    (G1 + G2 = 4 columns per KV head);
  - 6, 8, 9 and 16 columns (the 8-, 16-column variants; 16 runs 4 waves);
  - the composed path (fp32, head_dim 64, matrix cores off);
  - one noise head per KV head through this entry point is bit-identical
    to ``motif_gda_decode`` (the same kernels and plan);
  - the token's rows written inside the launch (cache rows bit-exact, y
    bit-identical to writing first);
  - the packed q4/q8 cache, fused (<= 16 columns x groups) and composed;
  - the fused step against the separately validated native calls.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O
from test_gpu_gda_decode import _bar, _ulp, ATT

pytestmark = pytest.mark.gpu


def _case(rng, B, Hkv, G1, G2, cap, D, tag, poison_from=None):
    q1 = randn(rng, (B, Hkv * G1, 1, D), tag)
    q2 = randn(rng, (B, Hkv * G2, 1, D), tag)
    ks = [randn(rng, (B, Hkv, cap, D), tag) for _ in range(4)]
    if poison_from is not None:
        for t in ks:
            t[:, :, poison_from:] = 1e4
    w = randn(rng, (2 * D,), tag)
    return q1, q2, ks, w


def _check(got, ref, tol):
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert float(err.mean()) <= 0.1 * float(tol.mean()) + 1e-6, (err.mean(), tol.mean())
    return float(np.max(err - tol))


def _run(gpu, rng, B, Hkv, G1, G2, cap, kv_len, D, tag, poison=False):
    import torch

    from mlx_motif.kernels import gda_decode_attention

    gr = G1 // G2
    q1, q2, (k1, k2, v1, v2), w = _case(rng, B, Hkv, G1, G2, cap, D, tag,
                                        kv_len if poison else None)
    dt = torch_dtype(tag)
    T = [np_to_torch(a, dt, gpu) for a in (q1, q2, k1, k2, v1, v2, w)]
    scale, lam, lam_init, eps = 1.0 / np.sqrt(D), 0.4321, 0.2, 1e-5
    lam_t = torch.tensor([lam], dtype=torch.float32, device=gpu)
    print(f"gda_decode_heads B={B} Hkv={Hkv} G1={G1} G2={G2} cap={cap} kv_len={kv_len} D={D} "
          f"{tag}", flush=True)
    y = gda_decode_attention(*T[:6], scale, T[6], lam_t, lam_init, gr, eps, kv_len=kv_len)
    torch.cuda.synchronize()
    assert y.shape == (B, Hkv * G1, 1, 2 * D) and y.dtype == dt
    ref, tol = _bar(q1, q2, k1, k2, v1, v2, w, scale, lam, lam_init, gr, eps, kv_len, tag)
    return _check(torch_to_np(y), ref, tol)


@pytest.mark.parametrize("kv_len", [1, 17, 300, 1024, 3204])
def test_small_step_8_pairs_over_4_kv_heads(gpu, rng, kv_len):
    cap = (kv_len + 255) // 256 * 256
    excess = _run(gpu, rng, 1, 4, 2, 2, cap, kv_len, 128, "f16")
    assert excess <= 0, f"kv_len={kv_len}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("kv_len", [1, 300, 3204])
def test_small_step_bf16(gpu, rng, kv_len):
    cap = (kv_len + 255) // 256 * 256
    excess = _run(gpu, rng, 1, 4, 2, 2, cap, kv_len, 128, "bf16")
    assert excess <= 0, f"bf16 kv_len={kv_len}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("B,Hkv,G1,G2", [(2, 2, 4, 2), (1, 2, 4, 4), (1, 2, 6, 3), (1, 1, 8, 8),
                                         (1, 2, 12, 4)])
def test_column_counts(gpu, rng, B, Hkv, G1, G2):
    """G1 + G2 = 6, 8, 9, 16 and 16 columns (gr 2, 1, 2, 1, 3)."""
    excess = _run(gpu, rng, B, Hkv, G1, G2, 512, 385, 128, "f16", poison=True)
    assert excess <= 0, f"{(B, Hkv, G1, G2)}: exceeds the bar by {excess:.3e}"


def test_columns_past_16_compose(gpu, rng):
    """9 + 9 = 18 columns per KV head: no fused variant, the composed path."""
    excess = _run(gpu, rng, 1, 1, 9, 9, 256, 200, 128, "f16")
    assert excess <= 0


@pytest.mark.parametrize("D,tag", [(64, "f16"), (128, "f32")])
def test_composed_path(gpu, rng, D, tag):
    excess = _run(gpu, rng, 1, 4, 2, 2, 256, 150, D, tag)
    assert excess <= 0, f"D={D} {tag}: exceeds the bar by {excess:.3e}"


def test_matrix_cores_off_compose(gpu, rng):
    from mlx_motif import _native

    _native.set_tuning("mfma", 0)
    try:
        excess = _run(gpu, rng, 1, 4, 2, 2, 1024, 1024, 128, "f16")
    finally:
        _native.set_tuning("mfma", 1)
    assert excess <= 0


def _inputs(gpu, B, Hkv, G1, G2, cap, D, dt, seed):
    import torch

    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).to(dt)  # noqa: E731
    q1, q2 = mk(B, Hkv * G1, 1, D), mk(B, Hkv * G2, 1, D)
    caches = [mk(B, Hkv, cap, D) for _ in range(4)]
    rows = [mk(B, Hkv, 1, D) for _ in range(4)]
    w = mk(2 * D)
    lam_t = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    return q1, q2, caches, rows, w, lam_t


@pytest.mark.parametrize("kv_len", [300, 16000])
def test_one_noise_head_per_kv_head_equals_gda_decode(gpu, kv_len):
    """Hq2 == Hkv through motif_gda_decode_heads: the 12.7B layout, bit-identical
    to motif_gda_decode (same kernels, same plan)."""
    import torch

    from mlx_motif import _native
    from mlx_motif.kernels import gda_decode_attention

    B, Hkv, gr, D = 1, 8, 4, 128
    cap = (kv_len + 127) // 128 * 128
    q1, q2, caches, _, w, lam_t = _inputs(gpu, B, Hkv, gr, 1, cap, D, torch.float16, kv_len)
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode_heads vs gda_decode kv_len={kv_len}", flush=True)
    y_ref = gda_decode_attention(q1, q2, *caches, scale, w, lam_t, lam_init, gr, eps,
                                 kv_len=kv_len)
    lib = _native.lib()
    n = lib.motif_gda_decode_heads_workspace_bytes(B, Hkv * gr, Hkv, Hkv, kv_len, D)
    ws = torch.zeros(n, dtype=torch.uint8, device=gpu)
    y = torch.empty_like(y_ref)
    _native.check(lib.motif_gda_decode_heads(
        q1.data_ptr(), q2.data_ptr(), None, None, None, None, *(c.data_ptr() for c in caches),
        w.data_ptr(), lam_t.data_ptr(), 1.0 - lam_init, eps, y.data_ptr(), 0, B, Hkv * gr, Hkv,
        Hkv, D, cap, kv_len, scale, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("B,Hkv,G1,G2,cap,kv_len,tag", [
    (1, 4, 2, 2, 1024, 1, "f16"),
    (1, 4, 2, 2, 1024, 1024, "f16"),    # the last row of the capacity
    (2, 2, 4, 2, 301, 17, "f16"),       # first row of the second 16-row block
    (1, 1, 8, 8, 512, 385, "f16"),      # 16 columns: the 4-wave kernel
    (1, 4, 2, 2, 256, 150, "bf16"),
    (1, 4, 2, 2, 256, 150, "f32"),      # composed: the row copy, then the calls
])
def test_append_writes_row_then_attends(gpu, B, Hkv, G1, G2, cap, kv_len, tag):
    import torch

    from mlx_motif.kernels import gda_decode_attention

    dt = torch_dtype(tag)
    D, gr = 128, G1 // G2
    q1, q2, caches, rows, w, lam_t = _inputs(gpu, B, Hkv, G1, G2, cap, D, dt, kv_len + 3)
    for c in caches:
        c[:, :, kv_len - 1] = 1e4  # stale contents of the row being written
    expect = [c.clone() for c in caches]
    for c, r in zip(expect, rows):
        c[:, :, kv_len - 1:kv_len] = r
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode_heads append B={B} Hkv={Hkv} G1={G1} G2={G2} kv_len={kv_len} {tag}",
          flush=True)
    y = gda_decode_attention(q1, q2, *caches, scale, w, lam_t, lam_init, gr, eps, kv_len=kv_len,
                             new_kv=rows)
    y_ref = gda_decode_attention(q1, q2, *expect, scale, w, lam_t, lam_init, gr, eps,
                                 kv_len=kv_len)
    torch.cuda.synchronize()
    iv = torch.int32 if tag == "f32" else torch.int16
    for c, e in zip(caches, expect):
        assert torch.equal(c.view(iv), e.view(iv))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(iv), y_ref.view(iv))


@pytest.mark.parametrize("kv_len", [1024, 3204])
def test_fused_equals_separate_native_calls(gpu, kv_len):
    """The small step fused and as the reference's three calls through the
    separately validated native kernels agree to the bar's scale."""
    import torch

    from mlx_motif.kernels import gda_decode_attention, gda_post_split, sdpa_dual_v

    B, Hkv, G1, G2, D = 1, 4, 2, 2, 128
    q1, q2, caches, _, w, lam_t = _inputs(gpu, B, Hkv, G1, G2, kv_len, D, torch.float16, 11)
    k1, k2, v1, v2 = caches
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode_heads fused vs separate kv_len={kv_len}", flush=True)
    y = gda_decode_attention(q1, q2, *caches, scale, w, lam_t, lam_init, 1, eps, kv_len=kv_len)
    o = sdpa_dual_v(q1, k1, v1, v2, scale, kv_len=kv_len)
    n = sdpa_dual_v(q2, k2, v1, v2, scale, kv_len=kv_len)
    y2 = gda_post_split(o, n, w, lam_t, lam_init, 1, eps)
    torch.cuda.synchronize()
    a, b = torch_to_np(y), torch_to_np(y2)
    d = torch_to_np(o) - 0.4321 * torch_to_np(n)
    rms_inv = 1.0 / np.sqrt((d * d).mean(axis=-1, keepdims=True) + eps)
    tol = (rms_inv * np.abs(torch_to_np(w)) * (1 - lam_init) * 1.4321 * ATT["f16"]
           + 2 * _ulp(b, "f16") + 1e-5)
    assert float(np.max(np.abs(a - b) - tol)) <= 0
    assert np.mean(a == b) > 0.5


# ------------------------------------------------------------ packed cache ---
def _run_q(gpu, rng, B, Hkv, G1, G2, cap, kv_len, bits, gs, tag="f16"):
    import torch

    from mlx_motif.kernels import gda_decode_attention_q4

    D, gr = 128, G1 // G2
    q1, q2, ks, w = _case(rng, B, Hkv, G1, G2, cap, D, tag, kv_len)
    trips = [O.quantize(t, gs, bits, out_dtype=tag) for t in ks]
    dt = torch_dtype(tag)
    gt = [(np_to_torch(d, None, gpu), np_to_torch(s, dt, gpu), np_to_torch(b, dt, gpu))
          for d, s, b in trips]
    scale, lam, lam_init, eps = 1.0 / np.sqrt(D), 0.4321, 0.2, 1e-5
    lam_t = torch.tensor([lam], dtype=torch.float32, device=gpu)
    print(f"gda_decode_q_heads B={B} Hkv={Hkv} G1={G1} G2={G2} cap={cap} kv_len={kv_len} "
          f"bits={bits} gs={gs} {tag}", flush=True)
    y = gda_decode_attention_q4(np_to_torch(q1, dt, gpu), np_to_torch(q2, dt, gpu), *gt, scale,
                                np_to_torch(w, dt, gpu), lam_t, lam_init, gr, gs, bits, eps,
                                kv_len=kv_len)
    torch.cuda.synchronize()
    assert y.shape == (B, Hkv * G1, 1, 2 * D) and y.dtype == dt
    deq = [O.dequantize(*t, group_size=gs, bits=bits) for t in trips]
    ref, tol = _bar(q1, q2, *deq, w, scale, lam, lam_init, gr, eps, kv_len, tag)
    return _check(torch_to_np(y), ref, tol)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("kv_len", [1, 300, 1024])
def test_small_step_packed(gpu, rng, bits, kv_len):
    cap = (kv_len + 255) // 256 * 256
    excess = _run_q(gpu, rng, 1, 4, 2, 2, cap, kv_len, bits, 64)
    assert excess <= 0, f"bits={bits} kv_len={kv_len}: exceeds the bar by {excess:.3e}"


@pytest.mark.parametrize("Hkv,G1,G2,gs", [(2, 4, 4, 64), (2, 2, 2, 32), (2, 4, 2, 128),
                                          (1, 8, 8, 64), (2, 4, 4, 32)])
def test_packed_columns_and_groups(gpu, rng, Hkv, G1, G2, gs):
    """Fused while (G1 + G2 rounded up) x (128 / gs) <= 16: 8 x 2, 4 x 4 and
    8 x 1; 16 x 2 and 8 x 4 take the composed path."""
    excess = _run_q(gpu, rng, 1, Hkv, G1, G2, 512, 385, 4, gs)
    assert excess <= 0, f"{(Hkv, G1, G2, gs)}: exceeds the bar by {excess:.3e}"


def test_packed_bf16(gpu, rng):
    assert _run_q(gpu, rng, 1, 4, 2, 2, 256, 150, 8, 64, "bf16") <= 0


@pytest.mark.parametrize("bits,kv_len", [(4, 1), (4, 1024), (8, 385)])
def test_packed_append(gpu, bits, kv_len):
    """The token's rows quantised into row kv_len - 1 inside the launch,
    bit-exactly as the oracle quantizer does (nothing else touched), and y
    bit-identical to the step without append over that cache."""
    import torch

    from mlx_motif.kernels import gda_decode_attention_q4, quantize

    B, Hkv, G1, G2, D, gs = 1, 4, 2, 2, 128, 64
    cap = (kv_len + 255) // 256 * 256
    q1, q2, caches, rows, w, lam_t = _inputs(gpu, B, Hkv, G1, G2, cap, D, torch.float16,
                                             kv_len + 5)
    slots = []
    for c in caches:  # the cache's other rows: any packed contents will do
        c[:, :, kv_len - 1] = 1e3
        slots.append(quantize(c, gs, bits))
    expect = [tuple(x.clone() for x in t) for t in slots]
    for t, r in zip(expect, rows):
        for dst, src in zip(t, O.quantize(torch_to_np(r), gs, bits, out_dtype="f16")):
            dst[:, :, kv_len - 1:kv_len] = np_to_torch(src, dst.dtype if dst.dtype != torch.uint32
                                                       else None, gpu)
    scale, lam_init, eps = 1.0 / np.sqrt(D), 0.2, 1e-5
    print(f"gda_decode_q_heads append bits={bits} kv_len={kv_len}", flush=True)
    y = gda_decode_attention_q4(q1, q2, *slots, scale, w, lam_t, lam_init, 1, gs, bits, eps,
                                kv_len=kv_len, new_kv=rows)
    y_ref = gda_decode_attention_q4(q1, q2, *expect, scale, w, lam_t, lam_init, 1, gs, bits,
                                    eps, kv_len=kv_len)
    torch.cuda.synchronize()
    for t, e in zip(slots, expect):
        assert torch.equal(t[0].view(torch.int32), e[0].view(torch.int32))
        assert torch.equal(t[1].view(torch.int16), e[1].view(torch.int16))
        assert torch.equal(t[2].view(torch.int16), e[2].view(torch.int16))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
