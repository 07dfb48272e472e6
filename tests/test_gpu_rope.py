"""Parity of ``motif_rope_split4`` (RoPE on q and k, the q1/q2, k1/k2 and
v1/v2 head split, and the 4-slot write at rows offset .. offset + S - 1)
against the oracle (float64 RoPE, model.py:580-594, 620-629, 669-679).

Bar: v rows are copies, bit-exact; q and k rows within 2 ulp of the output
type plus the rotation error of an fp32 angle, 1.2e-7 * position * |pair|
(the kernel, like mx.fast.rope, forms angle = position * inverse frequency
in fp32).  Cache rows outside the written range keep their contents.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ULP = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7, "f32": 2.0 ** -23}


def _ulp(x, tag):
    mag = np.maximum(np.abs(x), 2.0 ** -14)
    return ULP[tag] * 2.0 ** np.floor(np.log2(mag))


def _bar(ref, src_pairs_norm, pos_max, tag):
    return 2 * _ulp(ref, tag) + 1.2e-7 * pos_max * src_pairs_norm + 1e-7


@pytest.mark.parametrize("B,S,qg,gr,kg,kr,D,offset,cap,tag,origin_first", [
    (1, 1, 8, 4, 8, 1, 128, 3203, 3328, "f16", False),    # a 12.7B decode token
    (1, 512, 8, 4, 8, 1, 128, 0, 512, "f16", False),      # a 512-row prefill chunk
    (2, 7, 2, 3, 2, 1, 128, 16000, 16128, "f16", True),   # long position, origin-first q
    (1, 5, 8, 4, 8, 1, 128, 300, 320, "bf16", False),
    (1, 3, 2, 2, 2, 2, 64, 40, 64, "f32", False),         # k_ratio 2, head_dim 64
])
def test_rope_split4_matches_oracle(gpu, rng, B, S, qg, gr, kg, kr, D, offset, cap, tag,
                                    origin_first):
    import torch

    from mlx_motif.kernels import rope_split4

    dt = torch_dtype(tag)
    q = randn(rng, (B, S, qg * (gr + 1) * D), tag)
    k = randn(rng, (B, S, kg * (kr + 1) * D), tag)
    v = randn(rng, (B, S, 2 * kg * D), tag)
    caches = [torch.full((B, h, cap, D), 3.0, dtype=dt, device=gpu)
              for h in (kg * kr, kg, kg, kg)]
    print(f"rope_split4 B={B} S={S} offset={offset} {tag}", flush=True)
    out = rope_split4(*(np_to_torch(a, dt, gpu) for a in (q, k, v)), qg, gr, kg, kr, offset,
                      origin_first=origin_first, caches=caches)
    torch.cuda.synchronize()
    ref = O.rope_split4(q, k, v, qg, gr, kg, kr, offset, origin_first=origin_first)
    pos_max = offset + S - 1
    half = D // 2

    def pair_norm(x):
        x = np.asarray(x, np.float64)
        n = np.sqrt(x[..., :half] ** 2 + x[..., half:] ** 2)
        return np.concatenate([n, n], axis=-1)

    got = [torch_to_np(out[0]), torch_to_np(out[1])]
    got += [torch_to_np(c[:, :, offset:offset + S]) for c in caches]
    for i, (g, r) in enumerate(zip(got, ref)):
        if i >= 4:  # v1, v2: copies
            np.testing.assert_array_equal(g, O.round_to(r, tag))
        else:
            excess = np.abs(g - r) - _bar(r, pair_norm(r), pos_max, tag)
            assert float(excess.max()) <= 0, f"output {i}: exceeds the bar by {excess.max():.3e}"
    for c in caches:
        rest = torch.cat([c[:, :, :offset], c[:, :, offset + S:]], dim=2)
        assert bool((rest == 3.0).all())


def test_rope_split4_plain_outputs_equal_cache_writes(gpu, rng):
    """Without caches the k/v outputs are (B, H, S, D) tensors holding the
    same values the cache write stores; and the kernel agrees with the torch
    reference (fp32 angles) to 2 ulp plus what the two fp32 angles may
    differ by."""
    import torch

    from mlx_motif.kernels import rope_split4, rope_split4_reference

    dt = torch.float16
    q = np_to_torch(randn(rng, (1, 4, 40 * 128), "f16"), dt, gpu)
    k = np_to_torch(randn(rng, (1, 4, 16 * 128), "f16"), dt, gpu)
    v = np_to_torch(randn(rng, (1, 4, 16 * 128), "f16"), dt, gpu)
    plain = rope_split4(q, k, v, 8, 4, 8, 1, 77)
    caches = [torch.zeros((1, 8, 96, 128), dtype=dt, device=gpu) for _ in range(4)]
    cached = rope_split4(q, k, v, 8, 4, 8, 1, 77, caches=caches)
    ref = rope_split4_reference(q, k, v, 8, 4, 8, 1, 77)
    torch.cuda.synchronize()
    for a, b in zip(plain[2:], cached[2:]):
        assert torch.equal(a.view(torch.int16), b[:, :, 77:81].contiguous().view(torch.int16))
    # Both sides take fp32 angles (the kernel exp2 of a rounded log2(theta),
    # the reference torch's pow), each within 1.2e-7 * position of the exact
    # angle: an output may differ by 2 * 1.2e-7 * pos_max * (|x1| + |x2|) of
    # its source pair beyond the rounding (seen: 2 ulp + 5.7e-6 where the
    # rotation cancels).
    pos_max = 77 + 4 - 1
    pair = 2 * max(float(t.abs().max()) for t in (q, k, v))
    for a, b in zip(plain, ref):
        diff = np.abs(torch_to_np(a) - torch_to_np(b))
        bar = 2 * _ulp(torch_to_np(b), "f16") + 2 * 1.2e-7 * pos_max * pair + 1e-6
        assert float((diff - bar).max()) <= 0


@pytest.mark.parametrize("tag", ["f16", "bf16"])
def test_rope_split4_unaligned_rows_take_the_scalar_path(gpu, rng, tag):
    """Inputs 2 bytes off an 8-byte boundary (a view at element offset 1)
    take the element-wise path; its outputs and cache rows are bit-identical
    to the 8-byte vector path's on the same values."""
    import torch

    from mlx_motif.kernels import rope_split4

    dt = torch_dtype(tag)
    B, S, qg, gr, kg, D, offset, cap = 1, 6, 8, 4, 8, 128, 40, 64
    shapes = [(B, S, qg * (gr + 1) * D), (B, S, 2 * kg * D), (B, S, 2 * kg * D)]
    arrays = [np_to_torch(randn(rng, sh, tag), dt, gpu) for sh in shapes]

    def unaligned(t):
        buf = torch.empty(t.numel() + 1, dtype=dt, device=gpu)
        u = buf[1:].view(t.shape)
        u.copy_(t)
        assert u.data_ptr() % 8 == 2 and u.is_contiguous()
        return u

    outs = []
    for make in (lambda t: t, unaligned):
        caches = [torch.full((B, kg, cap, D), 3.0, dtype=dt, device=gpu) for _ in range(4)]
        print(f"rope_split4 {tag} {'unaligned' if make is unaligned else 'aligned'}", flush=True)
        res = rope_split4(*(make(t) for t in arrays), qg, gr, kg, 1, offset, caches=caches)
        torch.cuda.synchronize()
        outs.append([r.contiguous().view(torch.int16).cpu() for r in res[:2]] +
                    [c.view(torch.int16).cpu() for c in caches])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
