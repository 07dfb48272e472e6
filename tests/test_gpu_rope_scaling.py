"""Linear RoPE scaling on the GPU (``rope_scaling={"rope_type": "linear",
"factor": f}``, the reference's grouped fixture
swift/Tests/MotifKitTests/Fixtures/motif_config_grouped.json:17 uses f = 2):
mlx-lm's ``initialize_rope`` (model.py:414-419) ropes position p at p / f.

Checks:
  - ``rope_split4`` against the oracle's float64 RoPE at the scaled positions
    (2 ulp plus the rotation error of an fp32 angle, as the unscaled test);
  - at scale 1/2 an even position p ropes exactly as position p / 2 does
    unscaled (the kernel scales the position first, and p * 0.5 is exact);
  - the decode step and the prefill chunk from the projections (their
    kernels rope inside the attention launch) bit-identical to the scaled
    ``rope_split4`` followed by the separately validated attention calls,
    and the prefill chunk within 2e-3 of the oracle's composition.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LINEAR2 = {"rope_type": "linear", "factor": 2.0, "original_max_position_embeddings": 64}


def _ulp(x):
    return 2.0 ** -10 * 2.0 ** np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))


@pytest.mark.parametrize("factor,offset,S", [(2.0, 3203, 1), (2.0, 0, 64), (4.0, 15999, 3)])
def test_rope_split4_linear_matches_oracle(gpu, rng, factor, offset, S):
    import torch

    from mlx_motif.kernels import rope_split4

    qg, gr, kg, D, cap = 8, 4, 8, 128, offset + S + 16
    q = randn(rng, (1, S, qg * (gr + 1) * D), "f16")
    k = randn(rng, (1, S, 2 * kg * D), "f16")
    v = randn(rng, (1, S, 2 * kg * D), "f16")
    caches = [torch.full((1, kg, cap, D), 3.0, dtype=torch.float16, device=gpu)
              for _ in range(4)]
    cfg = {"type": "linear", "factor": factor}
    out = rope_split4(*(np_to_torch(a, torch.float16, gpu) for a in (q, k, v)), qg, gr, kg, 1,
                      offset, caches=caches, rope_scaling=cfg)
    torch.cuda.synchronize()
    ref = O.rope_split4(q, k, v, qg, gr, kg, 1, offset, scale=1.0 / factor)
    pos_max = (offset + S - 1) / factor
    got = [torch_to_np(out[0]), torch_to_np(out[1])]
    got += [torch_to_np(c[:, :, offset:offset + S]) for c in caches]
    for i, (g, r) in enumerate(zip(got, ref)):
        if i >= 4:
            np.testing.assert_array_equal(g, O.round_to(r, "f16"))
            continue
        half = D // 2
        n = np.sqrt(r[..., :half] ** 2 + r[..., half:] ** 2)
        bar = 2 * _ulp(r) + 1.2e-7 * pos_max * np.concatenate([n, n], axis=-1) + 1e-7
        assert float((np.abs(g - r) - bar).max()) <= 0, i


def test_half_scale_even_positions_equal_unscaled(gpu, rng):
    """Scale 1/2 at positions 100, 102, .. equals unscaled RoPE at 50, 51, ..
    bit for bit (q1/q2 and the k rows)."""
    import torch

    from mlx_motif.kernels import rope_split4

    qg, gr, kg, D = 8, 4, 8, 128
    arrays = [np_to_torch(randn(rng, (1, 1, w * D), "f16"), torch.float16, gpu)
              for w in (qg * (gr + 1), 2 * kg, 2 * kg)]
    for p in (100, 102, 3204, 16000):
        scaled = rope_split4(*arrays, qg, gr, kg, 1, p, rope_scaling=LINEAR2)
        plain = rope_split4(*arrays, qg, gr, kg, 1, p // 2)
        torch.cuda.synchronize()
        for a, b in zip(scaled[:4], plain[:4]):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), p


@pytest.mark.parametrize("offset", [0, 3203, 15999])
def test_decode_proj_linear_equals_rope_split4_then_step(gpu, offset):
    import torch

    from mlx_motif.kernels import (gda_decode_attention, gda_decode_attention_from_proj,
                                   gda_decode_attention_q4, gda_decode_attention_q4_from_proj,
                                   quantize, rope_split4)

    B, Hkv, gr, cap = 1, 8, 4, offset + 129
    g = torch.Generator(device=gpu)
    g.manual_seed(offset + 7)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).half()  # noqa: E731
    qp, kp, vp = mk(B, 1, Hkv * (gr + 1) * 128), mk(B, 1, 2 * Hkv * 128), mk(B, 1, 2 * Hkv * 128)
    caches = [mk(B, Hkv, cap, 128) for _ in range(4)]
    w = mk(256)
    lam = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    ref_caches = [c.clone() for c in caches]
    print(f"decode_proj linear x2 offset={offset}", flush=True)
    y = gda_decode_attention_from_proj(qp, kp, vp, *caches, 0.0884, w, lam, 0.2, gr, offset,
                                       rope_scaling=LINEAR2)
    q1, q2, *_ = rope_split4(qp, kp, vp, Hkv, gr, Hkv, 1, offset, caches=ref_caches,
                             rope_scaling=LINEAR2)
    y_ref = gda_decode_attention(q1, q2, *ref_caches, 0.0884, w, lam, 0.2, gr, kv_len=offset + 1)
    torch.cuda.synchronize()
    for c, r in zip(caches, ref_caches):
        assert torch.equal(c.view(torch.int16), r.view(torch.int16))
    assert torch.isfinite(y).all() and torch.equal(y.view(torch.int16), y_ref.view(torch.int16))

    # the packed cache (q4, group size 64)
    slots = [quantize(t, 64, 4) for t in caches]
    ref_slots = [tuple(x.clone() for x in t) for t in slots]
    yq = gda_decode_attention_q4_from_proj(qp, kp, vp, *slots, 0.0884, w, lam, 0.2, gr, offset,
                                           64, 4, rope_scaling=LINEAR2)
    q1, q2, *rows = rope_split4(qp, kp, vp, Hkv, gr, Hkv, 1, offset, rope_scaling=LINEAR2)
    yq_ref = gda_decode_attention_q4(q1, q2, *ref_slots, 0.0884, w, lam, 0.2, gr, 64, 4,
                                     kv_len=offset + 1, new_kv=rows)
    torch.cuda.synchronize()
    for t, r in zip(slots, ref_slots):
        assert torch.equal(t[0].view(torch.int32), r[0].view(torch.int32))
    assert torch.isfinite(yq).all() and torch.equal(yq.view(torch.int16), yq_ref.view(torch.int16))


@pytest.mark.parametrize("offset,S", [(3204, 512), (0, 256)])
def test_prefill_proj_linear(gpu, rng, offset, S):
    """The prefill chunk from the projections under linear scaling: cache
    rows bit-identical to the scaled rope_split4's, outputs within 1e-3 of
    rope_split4 + the multi-row calls and within 2e-3 of the oracle's
    composition at the scaled positions."""
    import torch

    from mlx_motif.kernels import gda_prefill_attention_from_proj, rope_split4, sdpa_dual_v_rows

    qg, gr, kg, D = 8, 4, 8, 128
    cap = (offset + S + 255) // 256 * 256
    q = randn(rng, (1, S, qg * (gr + 1) * D), "f16")
    k = randn(rng, (1, S, 2 * kg * D), "f16")
    v = randn(rng, (1, S, 2 * kg * D), "f16")
    old = [randn(rng, (1, kg, cap, D), "f16") for _ in range(4)]
    T = lambda a: np_to_torch(a, torch.float16, gpu)  # noqa: E731
    caches = [T(c) for c in old]
    ref_caches = [T(c) for c in old]
    sc = 1 / np.sqrt(D)
    print(f"prefill_proj linear x2 offset={offset} S={S}", flush=True)
    yo, yn = gda_prefill_attention_from_proj(T(q), T(k), T(v), caches, offset, qg, gr, kg, sc,
                                             rope_scaling=LINEAR2)
    q1, q2, k1, k2, v1, v2 = rope_split4(T(q), T(k), T(v), qg, gr, kg, 1, offset,
                                         caches=ref_caches, rope_scaling=LINEAR2)
    uo = sdpa_dual_v_rows(q1, k1, v1, v2, sc, kv_len=offset + S, causal=True)
    un = sdpa_dual_v_rows(q2, k2, v1, v2, sc, kv_len=offset + S, causal=True)
    torch.cuda.synchronize()
    for c, r in zip(caches, ref_caches):
        assert torch.equal(c.view(torch.int16), r.view(torch.int16))
    assert float((yo - uo).abs().max()) <= 1e-3 and float((yn - un).abs().max()) <= 1e-3
    e_o, e_n, _ = O.gda_prefill_from_proj(q, k, v, old, offset, qg, gr, kg, sc,
                                          position_scale=0.5)
    assert float(np.max(np.abs(torch_to_np(yo) - e_o))) <= 2e-3
    assert float(np.max(np.abs(torch_to_np(yn) - e_n))) <= 2e-3
