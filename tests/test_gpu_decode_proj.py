"""``motif_gda_decode_proj``: the decode step from the projection outputs,
RoPE and the token's cache write inside the attention launch.  Its output and
cache rows must equal ``rope_split4`` followed by the fused step bit for bit
(the same RoPE rounding, rope_impl.hpp), and the composition must meet the
oracle's bar (the decode step's, on the oracle's roped inputs)."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _inputs(gpu, B, Hkv, gr, cap, dt, seed):
    import torch

    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).to(dt)  # noqa: E731
    qp = mk(B, 1, Hkv * (gr + 1) * 128)
    kp, vp = mk(B, 1, 2 * Hkv * 128), mk(B, 1, 2 * Hkv * 128)
    caches = [mk(B, Hkv, cap, 128) for _ in range(4)]
    w = mk(256)
    lam = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    return qp, kp, vp, caches, w, lam


@pytest.mark.parametrize("B,Hkv,gr,cap,offset,tag,origin_first", [
    (1, 8, 4, 256, 0, "f16", False),         # the first token
    (1, 8, 4, 3328, 3203, "f16", False),     # 12.7B heads at 3204 rows
    (1, 8, 4, 16128, 15999, "f16", True),    # 16k rows, origin-first q
    (2, 2, 15, 512, 300, "f16", False),      # 16 columns (4-wave kernel)
    (1, 8, 4, 640, 600, "bf16", False),
])
def test_decode_proj_equals_rope_split4_then_step(gpu, B, Hkv, gr, cap, offset, tag,
                                                  origin_first):
    import torch

    from mlx_motif.kernels import (gda_decode_attention, gda_decode_attention_from_proj,
                                   rope_split4)

    dt = torch.float16 if tag == "f16" else torch.bfloat16
    qp, kp, vp, caches, w, lam = _inputs(gpu, B, Hkv, gr, cap, dt, offset + gr)
    ref_caches = [c.clone() for c in caches]
    print(f"decode_proj B={B} Hkv={Hkv} gr={gr} offset={offset} {tag}", flush=True)
    y = gda_decode_attention_from_proj(qp, kp, vp, *caches, 0.0884, w, lam, 0.2, gr, offset,
                                       origin_first=origin_first)
    q1, q2, *_ = rope_split4(qp, kp, vp, Hkv, gr, Hkv, 1, offset, origin_first=origin_first,
                             caches=ref_caches)
    y_ref = gda_decode_attention(q1, q2, *ref_caches, 0.0884, w, lam, 0.2, gr, kv_len=offset + 1)
    torch.cuda.synchronize()
    for c, r in zip(caches, ref_caches):
        assert torch.equal(c.view(torch.int16), r.view(torch.int16))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


def test_decode_proj_matches_oracle(gpu):
    """Against the oracle: its RoPE and split of the same projections, then
    its decode step, to the decode step's bar (tests/test_gpu_gda_decode.py)."""
    import torch

    from mlx_motif.kernels import gda_decode_attention_from_proj

    B, Hkv, gr, cap, offset = 1, 4, 4, 512, 400
    qp, kp, vp, caches, w, lam = _inputs(gpu, B, Hkv, gr, cap, torch.float16, 11)
    npy = [torch_to_np(t) for t in (qp, kp, vp, *caches, w)]
    y = gda_decode_attention_from_proj(qp, kp, vp, *caches, 0.0884, w, lam, 0.2, gr, offset)
    torch.cuda.synchronize()
    q1, q2, k1n, k2n, v1n, v2n = O.rope_split4(*npy[:3], Hkv, gr, Hkv, 1, offset)
    ks = [np.array(c) for c in npy[3:7]]
    for c, r in zip(ks, (k1n, k2n, v1n, v2n)):
        c[:, :, offset:offset + 1] = O.round_to(r, "f16")
    from test_gpu_gda_decode import _bar

    ref, tol = _bar(O.round_to(q1, "f16"), O.round_to(q2, "f16"), *ks, npy[7], 0.0884, 0.4321,
                    0.2, gr, 1e-5, offset + 1, "f16")
    err = np.abs(torch_to_np(y) - ref)
    assert float(np.max(err - tol)) <= 0
    assert float(err.mean()) <= 0.1 * float(tol.mean()) + 1e-6


@pytest.mark.parametrize("bits,gs,gr,cap,offset,origin_first,tag", [
    (4, 64, 4, 256, 0, False, "f16"),
    (4, 64, 4, 3328, 3203, False, "f16"),
    (8, 64, 4, 16128, 15999, True, "f16"),
    (4, 32, 3, 300, 250, False, "f16"),     # 4 columns x 4 groups
    (8, 128, 15, 512, 300, False, "f16"),   # 16 columns x 1 group
    (4, 32, 4, 256, 100, False, "f16"),     # 32 columns: rope_split4 + the step
    (4, 64, 4, 640, 600, False, "bf16"),
    (8, 64, 4, 3328, 3203, True, "bf16"),
])
def test_decode_q_proj_equals_rope_split4_then_step(gpu, bits, gs, gr, cap, offset,
                                                    origin_first, tag):
    """Packed cache: rows quantised after RoPE exactly as rope_split4 +
    the append step writes them, and the same output bit for bit."""
    import torch

    from mlx_motif.kernels import (gda_decode_attention_q4, gda_decode_attention_q4_from_proj,
                                   quantize, rope_split4)

    Hkv = 8 if gr <= 4 else 2
    dt = torch.float16 if tag == "f16" else torch.bfloat16
    qp, kp, vp, raw, w, lam = _inputs(gpu, 1, Hkv, gr, cap, dt, offset + bits)
    slots = [quantize(t, gs, bits) for t in raw]
    ref_slots = [tuple(x.clone() for x in t) for t in slots]
    print(f"decode_q_proj bits={bits} gs={gs} gr={gr} offset={offset} {tag}", flush=True)
    y = gda_decode_attention_q4_from_proj(qp, kp, vp, *slots, 0.0884, w, lam, 0.2, gr, offset,
                                          gs, bits, origin_first=origin_first)
    q1, q2, *rows = rope_split4(qp, kp, vp, Hkv, gr, Hkv, 1, offset, origin_first=origin_first)
    y_ref = gda_decode_attention_q4(q1, q2, *ref_slots, 0.0884, w, lam, 0.2, gr, gs, bits,
                                    kv_len=offset + 1, new_kv=rows)
    torch.cuda.synchronize()
    for t, r in zip(slots, ref_slots):
        assert torch.equal(t[0].view(torch.int32), r[0].view(torch.int32))
        assert torch.equal(t[1].view(torch.int16), r[1].view(torch.int16))
        assert torch.equal(t[2].view(torch.int16), r[2].view(torch.int16))
    assert torch.isfinite(y).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
