"""Host-side logic on the CPU: the Python mirror of the reference kernel API
(assertion messages, reference paths behind MLX_MOTIF_DISABLE_KERNELS, no
silent CPU fallback) and the 4-slot caches' buffer contract (growth, trim,
state), checked against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mlx_motif import cache as C
from mlx_motif import kernels as K
from mlx_motif.kernels import _common
from oracle import oracle as O


@pytest.fixture
def disabled(monkeypatch):
    monkeypatch.setattr(_common, "_DISABLE", True)


@pytest.fixture
def enabled(monkeypatch):
    monkeypatch.setattr(_common, "_DISABLE", False)


def _t(rng, shape, dtype=torch.float16, s=1.0):
    return torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float32)).to(dtype)


# -------------------------------------------------- contract assertions ---

def test_sdpa_dual_v_assertions(enabled, rng):
    q = _t(rng, (1, 32, 2, 128))
    k = _t(rng, (1, 8, 16, 128))
    with pytest.raises(AssertionError, match="decode-only"):
        K.sdpa_dual_v(q, k, k, k, 0.1)
    with pytest.raises(AssertionError, match="multiple of 32"):
        K.sdpa_dual_v(_t(rng, (1, 4, 1, 48)), _t(rng, (1, 4, 8, 48)), *[_t(rng, (1, 4, 8, 48))] * 2,
                      0.1)
    with pytest.raises(AssertionError, match=r"kv_len=17 must be in \[0, 16\]"):
        K.sdpa_dual_v(q[:, :, :1], k, k, k, 0.1, kv_len=17)
    with pytest.raises(AssertionError, match="v1,v2 must match"):
        K.sdpa_dual_v(q[:, :, :1], k, k[:, :, :8], k, 0.1)


@pytest.mark.parametrize("D,bits,gs,pattern", [
    (256, 8, 128, r"D/32 <= 32/bits"),
    (512, 4, 128, r"qk_per_thread \| EL_PER_INT"),
    (96, 8, 32, r"qk_per_thread \| EL_PER_INT"),
    (96, 4, 32, r"qk_per_thread \| EL_PER_INT"),
    (160, 4, 32, r"qk_per_thread \| EL_PER_INT"),
])
def test_sdpa_q4_rejects_out_of_contract_shapes(enabled, rng, D, bits, gs, pattern):
    """Reference tests/test_kernels_sdpa_dual_v_q4.py:162-232."""
    q = _t(rng, (1, 4, 1, D))
    data = torch.zeros((1, 4, 64, D * bits // 32), dtype=torch.uint32)
    sc = torch.zeros((1, 4, 64, D // gs), dtype=torch.float16)
    trip = (data, sc, sc)
    with pytest.raises(AssertionError, match=pattern):
        K.sdpa_dual_v_q4(q, trip, trip, trip, 0.1, group_size=gs, bits=bits)


def test_gda_assertion(enabled, rng):
    with pytest.raises(AssertionError, match=r"q_origin=30 != q_groups\(8\) \* gr\(4\)"):
        K.gda_post_split(_t(rng, (1, 30, 1, 256)), _t(rng, (1, 8, 1, 256)), _t(rng, (256,)),
                         torch.tensor([0.3]), 0.5, 4)


def test_kernels_refuse_cpu_tensors(enabled, rng):
    """No silent CPU fallback: valid shapes on CPU tensors raise."""
    q, k = _t(rng, (1, 8, 1, 64)), _t(rng, (1, 8, 16, 64))
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.sdpa_dual_v(q, k, k, k, 0.1)
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.polynorm(_t(rng, (4, 16)), torch.ones(3), torch.zeros(1))
    with pytest.raises(RuntimeError, match="ROCm device"):
        K.quantize(_t(rng, (4, 64)), 64, 4)


# ------------------------------------------------------ reference paths ---

def test_disabled_sdpa_reference_matches_oracle(disabled, rng):
    q, k, v1, v2 = _t(rng, (1, 32, 1, 128)), *(_t(rng, (1, 8, 300, 128)) for _ in range(3))
    y = K.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(128), kv_len=257)
    ref = O.sdpa_dual_v(q.numpy(), k.numpy(), v1.numpy(), v2.numpy(), 1 / np.sqrt(128), 257)
    assert y.dtype == torch.float16 and y.shape == (1, 32, 1, 256)
    assert np.max(np.abs(y.float().numpy() - ref)) <= 2e-3


def test_disabled_rows_reference_matches_oracle(disabled, rng):
    q, k, v1, v2 = _t(rng, (1, 8, 5, 64)), *(_t(rng, (1, 4, 64, 64)) for _ in range(3))
    y = K.sdpa_dual_v_rows(q, k, v1, v2, 0.125, kv_len=40, causal=True)
    ref = O.sdpa_dual_v(q.numpy(), k.numpy(), v1.numpy(), v2.numpy(), 0.125, 40, causal=True)
    assert np.max(np.abs(y.float().numpy() - ref)) <= 2e-3


@pytest.mark.parametrize("bits", [4, 8])
def test_disabled_q4_reference_matches_oracle(disabled, rng, bits):
    q = _t(rng, (1, 8, 1, 128))
    raw = [_t(rng, (1, 4, 100, 128)) for _ in range(3)]
    trips = [K.quantize(x, 64, bits) for x in raw]
    y = K.sdpa_dual_v_q4(q, *trips, 0.09, 64, bits, kv_len=90)
    np_trips = [O.quantize(x.numpy(), 64, bits) for x in raw]
    ref = O.sdpa_dual_v_q(q.numpy(), *np_trips, 0.09, 64, bits, 90, dequant_dtype="f16")
    assert np.max(np.abs(y.float().numpy() - ref)) <= 2e-3


@pytest.mark.parametrize("dtype,tag", [(torch.float16, "f16"), (torch.bfloat16, "bf16"),
                                       (torch.float32, "f32")])
@pytest.mark.parametrize("bits", [4, 8])
def test_torch_reference_quantizer_bit_identical_to_oracle(rng, dtype, tag, bits):
    x = _t(rng, (3, 5, 128), dtype, 2.0)
    d, s, b = K.quantize_reference(x, 64, bits)
    rd, rs, rb = O.quantize(x.float().numpy(), 64, bits, out_dtype=tag)
    assert d.dtype == torch.uint32
    np.testing.assert_array_equal(d.view(torch.int32).numpy().view(np.uint32), rd)
    np.testing.assert_array_equal(s.float().numpy(), np.asarray(rs, np.float32))
    np.testing.assert_array_equal(b.float().numpy(), np.asarray(rb, np.float32))
    y = K.dequantize_reference(d, s, b, 64, bits)
    np.testing.assert_array_equal(y.float().numpy(),
                                  np.asarray(O.dequantize(rd, rs, rb, 64, bits, tag), np.float32))


def test_disabled_epilogues_match_oracle(disabled, rng):
    o, n, w = _t(rng, (1, 8, 3, 256)), _t(rng, (1, 2, 3, 256)), _t(rng, (256,))
    lam = torch.tensor([0.4321], dtype=torch.float32)
    y = K.gda_post_split(o, n, w, lam, 0.65, 4, 1e-5)
    assert y.dtype == torch.float32  # fp32 lambda promotes, as in the reference
    ref = O.gda_post_split(o.numpy(), n.numpy(), w.numpy(), 0.4321, 0.65, 4, 1e-5)
    np.testing.assert_allclose(y.numpy(), ref, rtol=1e-4, atol=1e-4)
    m = torch.cat([o, n], dim=1)
    np.testing.assert_allclose(K.gda_post(m, w, lam, 0.65, 2, 4, 1e-5).numpy(), ref, rtol=1e-4,
                               atol=1e-4)
    x = _t(rng, (3, 7, 256), torch.float32)
    pw, pb = torch.tensor([0.4, 0.3, 0.3]), torch.tensor([0.05])
    np.testing.assert_allclose(K.polynorm(x, pw, pb, 1e-6).numpy(),
                               O.polynorm(x.numpy(), pw.numpy(), pb.numpy(), 1e-6),
                               rtol=1e-4, atol=1e-4)


def test_disabled_decode_append_writes_row_and_matches_oracle(disabled, rng):
    """Reference path of ``new_kv``: the token's rows land at row kv_len - 1
    of each slot and the step matches the oracle over that cache."""
    q1, q2 = _t(rng, (1, 8, 1, 64), torch.float32), _t(rng, (1, 2, 1, 64), torch.float32)
    caches = [_t(rng, (1, 2, 40, 64), torch.float32) for _ in range(4)]
    rows = [_t(rng, (1, 2, 1, 64), torch.float32) for _ in range(4)]
    before = [c.clone() for c in caches]
    w, lam = _t(rng, (128,), torch.float32), torch.tensor([0.4321])
    y = K.gda_decode_attention(q1, q2, *caches, 0.125, w, lam, 0.2, 4, 1e-5, kv_len=31,
                               new_kv=rows)
    for c, b, r in zip(caches, before, rows):
        b[:, :, 30:31] = r
        assert torch.equal(c, b)
    ref = O.gda_decode_attention(q1.numpy(), q2.numpy(), *(c.numpy() for c in caches), 0.125,
                                 w.numpy(), 0.4321, 0.2, 4, 1e-5, 31, dtype="f32")
    np.testing.assert_allclose(y.numpy(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("bits", [4, 8])
def test_disabled_decode_q_append_quantises_row_like_oracle(disabled, rng, bits):
    q1, q2 = _t(rng, (1, 8, 1, 128)), _t(rng, (1, 2, 1, 128))
    trips = [K.quantize(_t(rng, (1, 2, 24, 128)), 64, bits) for _ in range(4)]
    rows = [_t(rng, (1, 2, 1, 128)) for _ in range(4)]
    w, lam = _t(rng, (256,)), torch.tensor([0.4321])
    K.gda_decode_attention_q4(q1, q2, *trips, 0.09, w, lam, 0.2, 4, 64, bits, 1e-5, kv_len=24,
                              new_kv=rows)
    for t, r in zip(trips, rows):
        rd, rs, rb = O.quantize(r.float().numpy(), 64, bits, out_dtype="f16")
        np.testing.assert_array_equal(t[0][:, :, 23:24].view(torch.int32).numpy().view(np.uint32),
                                      rd)
        np.testing.assert_array_equal(t[1][:, :, 23:24].float().numpy(), np.float32(rs))
        np.testing.assert_array_equal(t[2][:, :, 23:24].float().numpy(), np.float32(rb))


def test_decode_append_contract(enabled, rng):
    """Checks made before any native call: kv_len counts the new row, the
    rows' shape and dtype, and in-place (contiguous) cache buffers."""
    q1, q2 = _t(rng, (1, 4, 1, 64)), _t(rng, (1, 2, 1, 64))
    caches = [_t(rng, (1, 2, 16, 64)) for _ in range(4)]
    rows = [_t(rng, (1, 2, 1, 64)) for _ in range(4)]
    w, lam = _t(rng, (128,)), torch.tensor([0.5])
    with pytest.raises(ValueError, match="appended row"):
        K.gda_decode_attention(q1, q2, *caches, 0.1, w, lam, 0.2, 2, kv_len=0, new_kv=rows)
    with pytest.raises(ValueError, match="k1_new"):
        K.gda_decode_attention(q1, q2, *caches, 0.1, w, lam, 0.2, 2, kv_len=3, new_kv=rows[:3])
    with pytest.raises(TypeError, match="new_kv dtype"):
        K.gda_decode_attention(q1, q2, *caches, 0.1, w, lam, 0.2, 2, kv_len=3,
                               new_kv=[r.float() for r in rows])
    with pytest.raises(AssertionError, match="new_kv rows"):
        K.gda_decode_attention(q1, q2, *caches, 0.1, w, lam, 0.2, 2, kv_len=3,
                               new_kv=[r[:, :1] for r in rows])
    strided = caches[0].transpose(2, 3).contiguous().transpose(2, 3)
    with pytest.raises(ValueError, match="contiguous"):
        K.gda_decode_attention(q1, q2, strided, *caches[1:], 0.1, w, lam, 0.2, 2, kv_len=3,
                               new_kv=rows)


def test_disabled_rope_split4_reference_matches_oracle(disabled, rng):
    qg, gr, kg, kr, D, B, S = 2, 4, 2, 1, 64, 1, 6
    q = _t(rng, (B, S, qg * (gr + 1) * D), torch.float32)
    k = _t(rng, (B, S, kg * (kr + 1) * D), torch.float32)
    v = _t(rng, (B, S, 2 * kg * D), torch.float32)
    caches = [torch.full((B, kg, 32, D), 7.0) for _ in range(4)]
    out = K.rope_split4(q, k, v, qg, gr, kg, kr, 20, caches=caches)
    ref = O.rope_split4(q.numpy(), k.numpy(), v.numpy(), qg, gr, kg, kr, 20)
    np.testing.assert_allclose(out[0].numpy(), ref[0], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out[1].numpy(), ref[1], rtol=1e-5, atol=1e-5)
    for c, r in zip(caches, ref[2:]):
        np.testing.assert_allclose(c[:, :, 20:26].numpy(), r, rtol=1e-5, atol=1e-5)
        assert (c[:, :, :20] == 7.0).all() and (c[:, :, 26:] == 7.0).all()


def test_rope_split4_contract(enabled, rng):
    q, k, v = _t(rng, (1, 2, 5 * 64)), _t(rng, (1, 2, 2 * 64)), _t(rng, (1, 2, 2 * 64))
    with pytest.raises(AssertionError, match="q width"):
        K.rope_split4(q[..., :-1], k, v, 1, 4, 1, 1, 0)
    with pytest.raises(AssertionError, match="k must be"):
        K.rope_split4(q, k[..., :-64], v, 1, 4, 1, 1, 0)
    with pytest.raises(AssertionError, match="v must be"):
        K.rope_split4(q, k, v[..., :-64], 1, 4, 1, 1, 0)


def test_polynorm_zero_rows_returns_zeros(enabled):
    x = torch.zeros((0, 16))
    assert K.polynorm(x, torch.ones(3), torch.zeros(1)).shape == (0, 16)


# ------------------------------------------------------------ caches ---

def test_fp_cache_growth_and_fetch_contract(rng):
    cache = C.MotifGroupedKVCache()
    cache.step = 4
    B, H, D = 1, 4, 32
    rows = []
    for S in (3, 1, 1, 5, 1):
        new = [_t(rng, (B, H, S, D)) for _ in range(4)]
        rows.append(new)
        k1, k2, v1, v2 = cache.update_and_fetch_4(*new)
    assert cache.offset == 11
    assert k1.shape[2] >= 11 and k1.is_contiguous()
    o = cache.offset
    for i, t in enumerate((k1, k2, v1, v2)):
        np.testing.assert_array_equal(t[:, :, :o].numpy(),
                                      torch.cat([r[i] for r in rows], dim=2).numpy())
    st = cache.state
    assert all(s.shape[2] == o for s in st)
    assert cache.meta_state == ("11",)
    assert cache.trim(3) == 3 and cache.offset == 8
    assert cache.trim(100) == 8 and cache.offset == 0


def test_cache_rejects_mismatched_slot_heads(rng):
    cache = C.MotifGroupedKVCache()
    with pytest.raises(ValueError, match="share a head count"):
        cache.update_and_fetch_4(_t(rng, (1, 8, 1, 32)), *[_t(rng, (1, 4, 1, 32))] * 3)
    qc = C.MotifGroupedQuantizedKVCache(64, 4)
    with pytest.raises(ValueError, match="share a head count"):
        qc.update_and_fetch_4_quantized(_t(rng, (1, 8, 1, 64)), *[_t(rng, (1, 4, 1, 64))] * 3)


def test_update_and_fetch_single_slot_unsupported():
    with pytest.raises(NotImplementedError):
        C.MotifGroupedKVCache().update_and_fetch(None, None)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_reference_write_matches_per_slot_oracle(disabled, rng, bits):
    """Reference path: concat + one quantisation + 12 slice writes, bit-identical
    to the per-slot oracle write (reference tests/test_grouped_cache.py:168)."""
    B, H, D, gs = 1, 8, 128, 64
    cache = C.MotifGroupedQuantizedKVCache(group_size=gs, bits=bits)
    ref = [(np.zeros((B, H, 256, D * bits // 32), np.uint32), np.zeros((B, H, 256, D // gs)),
            np.zeros((B, H, 256, D // gs))) for _ in range(4)]
    off = 0
    for S in (5, 1, 1, 1):
        new = [_t(rng, (B, H, S, D)) for _ in range(4)]
        live = cache.update_and_fetch_4_quantized(*new)
        O.quant_write4(ref, *[x.numpy() for x in new], off, gs, bits)
        off += S
    assert cache.offset == off == 8
    for slot, r in zip(live, ref):
        np.testing.assert_array_equal(slot[0].view(torch.int32).numpy().view(np.uint32), r[0])
        np.testing.assert_array_equal(slot[1].float().numpy(), r[1])
        np.testing.assert_array_equal(slot[2].float().numpy(), r[2])
    meta = cache.meta_state
    assert meta == ("8", str(gs), str(bits))
    st = cache.state
    assert all(part.shape[2] == 8 for slot in st for part in slot)


@pytest.mark.parametrize("bits,tol", [(4, 0.5), (8, 0.05)])
def test_quantized_cache_dequant_bridge(disabled, rng, bits, tol):
    cache = C.MotifGroupedQuantizedKVCache(group_size=64, bits=bits)
    new = [_t(rng, (1, 8, 5, 128), s=0.1) for _ in range(4)]
    out = cache.update_and_fetch_4(*new)
    assert all(t.shape == (1, 8, 5, 128) for t in out)
    np.testing.assert_allclose(out[0].float().numpy(), new[0].float().numpy(), atol=tol, rtol=tol)


def test_to_quantized(disabled, rng):
    fc = C.MotifGroupedKVCache()
    new = [_t(rng, (1, 4, 6, 64)) for _ in range(4)]
    fc.update_and_fetch_4(*new)
    qc = fc.to_quantized(group_size=64, bits=8)
    assert qc.offset == 6 and qc.k1[0].shape == (1, 4, 6, 16)
    rd, _, _ = O.quantize(new[0].numpy(), 64, 8)
    np.testing.assert_array_equal(qc.k1[0].view(torch.int32).numpy().view(np.uint32), rd)


def test_fp_cache_state_roundtrip_and_growth(rng):
    """``state`` is the live [:offset] region and restores into a fresh
    cache, which keeps growing past the restored offset (reference
    tests/test_grouped_cache.py:269-299)."""
    B, H, D = 1, 4, 128
    cache = C.MotifGroupedKVCache()
    for _ in range(3):
        t = _t(rng, (B, H, 1, D))
        cache.update_and_fetch_4(t, t, t, t)
    saved = cache.state
    assert all(a.shape[2] == 3 for a in saved)
    restored = C.MotifGroupedKVCache()
    restored.meta_state = cache.meta_state
    restored.state = saved
    assert restored.offset == 3
    for a, b in zip(saved, restored.state):
        np.testing.assert_array_equal(a.numpy(), b.numpy())
    tb = _t(rng, (B, H, 1, D))
    out = restored.update_and_fetch_4(tb, tb, tb, tb)
    assert restored.offset == 4 and all(x.shape[2] >= 4 for x in out)
    assert all(s.shape == (B, H, 4, D) for s in restored.state)
    np.testing.assert_array_equal(restored.state[0][:, :, :3].numpy(), saved[0].numpy())
    np.testing.assert_array_equal(restored.state[0][:, :, 3:].numpy(), tb.numpy())


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_state_roundtrip_and_growth(disabled, rng, bits):
    """Quantised ``state``: every (data, scales, biases) part trimmed to the
    offset, exact round trip through ``meta_state``/``state``, growth after a
    restore that is not step-aligned (reference
    tests/test_grouped_cache.py:302-336)."""
    B, H, D = 1, 4, 128
    cache = C.MotifGroupedQuantizedKVCache(group_size=64, bits=bits)
    for _ in range(3):
        t = _t(rng, (B, H, 1, D))
        cache.update_and_fetch_4(t, t, t, t)
    saved = cache.state
    assert all(part.shape[2] == 3 for slot in saved for part in slot)
    restored = C.MotifGroupedQuantizedKVCache()
    restored.meta_state = cache.meta_state
    restored.state = saved
    assert restored.offset == 3 and (restored.group_size, restored.bits) == (64, bits)
    for a, b in zip(saved, restored.state):
        for x, y in zip(a, b):
            assert x.shape == y.shape
            np.testing.assert_array_equal(x.numpy(), y.numpy())
    tb = _t(rng, (B, H, 1, D))
    out = restored.update_and_fetch_4(tb, tb, tb, tb)
    assert all(x.shape == (B, H, 4, D) for x in out) and restored.offset == 4
    # The restored rows are unchanged by the growth and the new row is the
    # quantisation of the new token.
    grown = restored.state
    for a, b in zip(saved, grown):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x.numpy(), y[:, :, :3].numpy())
    rd, _, _ = O.quantize(tb.numpy(), 64, bits)
    np.testing.assert_array_equal(grown[0][0][:, :, 3:].view(torch.int32).numpy().view(np.uint32), rd)


def _q_trips(B, H_kv, cap, D, bits, gs, dtype=torch.float16):
    return [(torch.zeros((B, H_kv, cap, D * bits // 32), dtype=torch.uint32),
             torch.ones((B, H_kv, cap, D // gs), dtype=dtype),
             torch.zeros((B, H_kv, cap, D // gs), dtype=dtype)) for _ in range(4)]


@pytest.mark.parametrize("bits", [4, 8])
def test_decode_q_slot_contract(enabled, rng, bits):
    """Packed-slot checks both packed-cache decode wrappers make before any
    native call: data (B, H_kv, KV_cap, D*bits/32), scales and biases
    (B, H_kv, KV_cap, D/gs) in the query dtype, projections in one dtype."""
    B, H_kv, gr, D, cap, gs = 1, 2, 4, 128, 24, 64
    q1, q2 = _t(rng, (B, H_kv * gr, 1, D)), _t(rng, (B, H_kv, 1, D))
    q_proj = _t(rng, (B, 1, H_kv * (gr + 1) * D))
    k_proj, v_proj = _t(rng, (B, 1, 2 * H_kv * D)), _t(rng, (B, 1, 2 * H_kv * D))
    w, lam = _t(rng, (2 * D,)), torch.tensor([0.5])

    def step(trips):
        K.gda_decode_attention_q4(q1, q2, *trips, 0.1, w, lam, 0.2, gr, gs, bits, kv_len=8)

    def from_proj(trips, kp=k_proj, vp=v_proj):
        K.gda_decode_attention_q4_from_proj(q_proj, kp, vp, *trips, 0.1, w, lam, 0.2, gr, 7,
                                            gs, bits)

    for call in (step, from_proj):
        t = _q_trips(B, H_kv, cap, D, bits, gs)
        t[2] = (t[2][0][:, :, :16], t[2][1], t[2][2])  # one slot with another capacity
        with pytest.raises(AssertionError, match="packed data"):
            call(t)
        t = _q_trips(B, H_kv, cap, D, bits, gs)
        t[1] = (t[1][0], t[1][1][..., :1], t[1][2])  # scales of the wrong group count
        with pytest.raises(AssertionError, match="scales/biases"):
            call(t)
        t = _q_trips(B, H_kv, cap, D, bits, gs)
        t[3] = (t[3][0], t[3][1], t[3][2].float())
        with pytest.raises(TypeError, match="scales/biases dtype"):
            call(t)
        with pytest.raises(TypeError, match="packed data dtype"):
            t = _q_trips(B, H_kv, cap, D, bits, gs)
            t[0] = (t[0][0].float(), t[0][1], t[0][2])
            call(t)
    # The projection path takes D from the q width: a packed width of the
    # other bit count does not match it.
    other = _q_trips(B, H_kv, cap, D, 12 - bits, gs)
    with pytest.raises(AssertionError, match="packed data"):
        from_proj(other)
    with pytest.raises(TypeError, match="k_proj/v_proj dtype"):
        from_proj(_q_trips(B, H_kv, cap, D, bits, gs), kp=k_proj.float())
    with pytest.raises(TypeError, match="k_proj/v_proj dtype"):
        from_proj(_q_trips(B, H_kv, cap, D, bits, gs), vp=v_proj.bfloat16())
    # In contract, the CPU tensors reach the device check (no CPU fallback).
    with pytest.raises(RuntimeError, match="ROCm device"):
        from_proj(_q_trips(B, H_kv, cap, D, bits, gs))
    with pytest.raises(RuntimeError, match="ROCm device"):
        step(_q_trips(B, H_kv, cap, D, bits, gs))


def test_rope_scaling_configs(rng, monkeypatch):
    """RoPE scaling configs are read as mlx-lm's initialize_rope reads them:
    None and "default" rope at unscaled positions, "linear" (the reference's
    grouped fixture: factor 2) at positions / factor, and every other type
    is refused by every RoPE wrapper, kernels or not, instead of roping at
    the wrong positions."""
    from mlx_motif.kernels.rope import rope_position_scale

    linear = {"rope_type": "linear", "factor": 2.0, "original_max_position_embeddings": 64}
    assert rope_position_scale(None) == 1.0
    assert rope_position_scale({"rope_type": "default"}) == 1.0
    assert rope_position_scale(linear) == 0.5
    assert rope_position_scale({"type": "linear", "factor": 4.0}) == 0.25
    with pytest.raises(ValueError):
        rope_position_scale({"type": "linear", "factor": 0.0})
    llama3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
              "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    q_proj, k_proj, v_proj = _t(rng, (1, 1, 640)), _t(rng, (1, 1, 256)), _t(rng, (1, 1, 256))
    caches = [_t(rng, (1, 2, 8, 64)) for _ in range(4)]
    w, lam = _t(rng, (128,)), torch.tensor([0.5])
    for flag in (True, False):
        monkeypatch.setattr(_common, "_DISABLE", flag)
        with pytest.raises(NotImplementedError, match="llama3"):
            K.rope_split4(q_proj, k_proj, v_proj, 2, 4, 2, 1, 3, rope_scaling=llama3)
        with pytest.raises(NotImplementedError, match="llama3"):
            K.gda_decode_attention_from_proj(q_proj, k_proj, v_proj, *caches, 0.1, w, lam, 0.2, 4,
                                             3, rope_scaling=llama3)
        with pytest.raises(NotImplementedError, match="llama3"):
            K.gda_decode_attention_q4_from_proj(q_proj, k_proj, v_proj,
                                                *_q_trips(1, 2, 8, 64, 4, 64), 0.1, w, lam, 0.2,
                                                4, 3, rope_scaling=llama3)
    # The torch statement under linear scaling: position p at scale 1/2 is
    # position p / 2 unscaled (even p), and matches the float64 oracle.
    monkeypatch.setattr(_common, "_DISABLE", True)
    q4, k4, v4 = _t(rng, (1, 4, 640)), _t(rng, (1, 4, 256)), _t(rng, (1, 4, 256))
    scaled = K.rope_split4(q4, k4, v4, 2, 4, 2, 1, 6, rope_scaling=linear)
    plain = [K.rope_split4_reference(q4[:, s:s + 1], k4[:, s:s + 1], v4[:, s:s + 1], 2, 4, 2, 1,
                                     (6 + s) // 2) for s in (0, 2)]
    for s, ref in zip((0, 2), plain):
        for a, b in zip(scaled[:4], ref[:4]):
            np.testing.assert_array_equal(a[:, :, s:s + 1].float().numpy(), b.float().numpy())
    oq1, *_ = O.rope_split4(q4.numpy(), k4.numpy(), v4.numpy(), 2, 4, 2, 1, 6, scale=0.5)
    assert np.max(np.abs(scaled[0].double().numpy() - oq1)) <= 2 * 2.0 ** -10 * (
        1 + np.max(np.abs(oq1)))
