"""KV-cache state on the GPU: fill, save, trim, restore, grow, attend.

The reference's 4-slot caches (src/mlx_motif/cache.py:178-545) define the
saved format (``state``: the live ``[:offset]`` rows of k1, k2, v1, v2, as
plain arrays or MLX-affine triples; ``meta_state``: the offset, plus group
size and bits for the quantised cache, cache.py:367-388, 518-545), the
speculative rollback (``trim``, cache.py:221-224) and ``to_quantized``
(cache.py:394-404).  Here the caches are filled on the GPU through the
product path (slice writes for the fp16 cache, one ``motif_quant_write4``
dispatch per step for the packed cache), rolled back, saved, restored into a
fresh cache, grown by a decode row and attended over with
``sdpa_dual_v`` / ``sdpa_dual_v_q4``.

Bars: restored and grown slots bit-identical to the rows written (packed
words, scales and biases against the oracle's quantizer); ``to_quantized``
bit-exact against the oracle's ``quantize``; attention within 2e-3 of the
oracle (fp16 outputs, fp32 accumulation).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

B, H, HQ, D, GS = 1, 8, 32, 128, 64
TOL = 2e-3


def _steps(rng, sizes):
    return [tuple(randn(rng, (B, H, S, D), "f16") for _ in range(4)) for S in sizes]


def _dev(x, gpu):
    import torch

    return np_to_torch(x, torch.float16, gpu)


def _fill(cache, steps, gpu, quantized):
    for st in steps:
        args = [_dev(x, gpu) for x in st]
        if quantized:
            cache.update_and_fetch_4_quantized(*args)
        else:
            cache.update_and_fetch_4(*args)


def _live_rows(steps, n):
    """The first n rows of each slot as written by `steps` (numpy fp16)."""
    return [np.concatenate([st[i] for st in steps], axis=2)[:, :, :n] for i in range(4)]


def _attend_fp(gpu, rng, slots, kv_len):
    from mlx_motif.kernels import sdpa_dual_v

    q = randn(rng, (B, HQ, 1, D), "f16")
    k1, _, v1, v2 = slots
    y = sdpa_dual_v(_dev(q, gpu), k1, v1, v2, 1.0 / np.sqrt(D), kv_len=kv_len)
    ref = O.sdpa_dual_v(q, torch_to_np(k1), torch_to_np(v1), torch_to_np(v2), 1.0 / np.sqrt(D),
                        kv_len=kv_len)
    return float(np.max(np.abs(torch_to_np(y) - ref)))


def _attend_q(gpu, rng, slots, kv_len, bits):
    from mlx_motif.kernels import sdpa_dual_v_q4

    q = randn(rng, (B, HQ, 1, D), "f16")
    k1, _, v1, v2 = slots
    y = sdpa_dual_v_q4(_dev(q, gpu), k1, v1, v2, 1.0 / np.sqrt(D), group_size=GS, bits=bits,
                       kv_len=kv_len)
    host = [tuple(torch_to_np(x) for x in s) for s in (k1, v1, v2)]
    host = [(d.astype(np.uint32), s, b) for d, s, b in host]
    ref = O.sdpa_dual_v_q(q, host[0], host[1], host[2], 1.0 / np.sqrt(D), GS, bits, kv_len)
    return float(np.max(np.abs(torch_to_np(y) - ref)))


def _check_fp_rows(slots, rows):
    for got, want in zip(slots, rows):
        n = want.shape[2]
        assert np.array_equal(torch_to_np(got)[:, :, :n], want.astype(np.float64))


def _check_q_rows(slots, rows, bits):
    for got, want in zip(slots, rows):
        rd, rs, rb = O.quantize(want, GS, bits)
        n = want.shape[2]
        d, s, b = (torch_to_np(x)[:, :, :n] for x in got)
        assert np.array_equal(d.astype(np.uint32), rd)
        assert np.array_equal(s, rs.astype(np.float64))
        assert np.array_equal(b, rb.astype(np.float64))


def test_fp16_cache_rollback_save_restore_attend(gpu, rng):
    """fp16 cache: 700-row prefill + 5 speculative decode rows, trim(3), save,
    restore into a fresh cache, one more decode row, attend."""
    from mlx_motif.cache import MotifGroupedKVCache

    steps = _steps(rng, [700, 1, 1, 1, 1, 1])
    cache = MotifGroupedKVCache()
    _fill(cache, steps, gpu, quantized=False)
    assert cache.offset == 705 and cache.k1.shape[2] == 768
    assert cache.trim(3) == 3 and cache.offset == 702

    saved, meta = cache.state, cache.meta_state
    assert meta == ("702",) and all(s.shape == (B, H, 702, D) for s in saved)
    _check_fp_rows(saved, _live_rows(steps, 702))

    restored = MotifGroupedKVCache()
    restored.meta_state = meta
    restored.state = saved
    assert restored.offset == 702
    err = _attend_fp(gpu, rng, restored.state, 702)  # exact-length buffers
    assert err <= TOL, err

    new = _steps(rng, [1])[0]
    out = restored.update_and_fetch_4(*[_dev(x, gpu) for x in new])
    assert restored.offset == 703 and all(t.shape == (B, H, 702 + 256, D) for t in out)
    rows = [np.concatenate([r, n], axis=2) for r, n in zip(_live_rows(steps, 702), new)]
    _check_fp_rows(out, rows)
    assert _attend_fp(gpu, rng, out, 703) <= TOL

    # The rolled-back original overwrites its speculative rows in place.
    out2 = cache.update_and_fetch_4(*[_dev(x, gpu) for x in new])
    assert cache.offset == 703 and out2[0].shape[2] == 768
    _check_fp_rows(out2, rows)
    assert _attend_fp(gpu, rng, out2, 703) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_rollback_save_restore_attend(gpu, rng, bits):
    """Packed cache written by motif_quant_write4: 700-row prefill + 5
    speculative rows, trim(3), save, restore, grow by one row, attend."""
    from mlx_motif.cache import MotifGroupedQuantizedKVCache

    steps = _steps(rng, [700, 1, 1, 1, 1, 1])
    cache = MotifGroupedQuantizedKVCache(group_size=GS, bits=bits)
    _fill(cache, steps, gpu, quantized=True)
    assert cache.offset == 705 and cache.k1[0].shape[2] == 768
    cache.trim(3)

    saved, meta = cache.state, cache.meta_state
    assert meta == ("702", str(GS), str(bits))
    assert all(p.shape[2] == 702 for slot in saved for p in slot)
    _check_q_rows(saved, _live_rows(steps, 702), bits)

    restored = MotifGroupedQuantizedKVCache()
    restored.meta_state = meta
    restored.state = saved
    assert (restored.offset, restored.group_size, restored.bits) == (702, GS, bits)
    assert _attend_q(gpu, rng, restored.state, 702, bits) <= TOL

    new = _steps(rng, [1])[0]
    out = restored.update_and_fetch_4_quantized(*[_dev(x, gpu) for x in new])
    assert restored.offset == 703 and all(p.shape[2] == 702 + 256 for s in out for p in s)
    rows = [np.concatenate([r, n], axis=2) for r, n in zip(_live_rows(steps, 702), new)]
    _check_q_rows(out, rows, bits)
    assert _attend_q(gpu, rng, out, 703, bits) <= TOL

    out2 = cache.update_and_fetch_4_quantized(*[_dev(x, gpu) for x in new])
    assert cache.offset == 703
    _check_q_rows(out2, rows, bits)
    assert _attend_q(gpu, rng, out2, 703, bits) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_to_quantized_then_attend(gpu, rng, bits):
    """fp16 cache on the GPU -> to_quantized: live rows packed bit-exactly as
    the oracle's quantizer packs them; the quantised cache keeps growing and
    attends within tolerance."""
    from mlx_motif.cache import MotifGroupedKVCache

    steps = _steps(rng, [300, 1, 1])
    fc = MotifGroupedKVCache()
    _fill(fc, steps, gpu, quantized=False)
    qc = fc.to_quantized(group_size=GS, bits=bits)
    assert (qc.offset, qc.group_size, qc.bits) == (302, GS, bits)
    assert all(p.shape[2] == 302 for slot in (qc.k1, qc.k2, qc.v1, qc.v2) for p in slot)
    _check_q_rows((qc.k1, qc.k2, qc.v1, qc.v2), _live_rows(steps, 302), bits)

    new = _steps(rng, [1])[0]
    out = qc.update_and_fetch_4_quantized(*[_dev(x, gpu) for x in new])
    assert qc.offset == 303
    rows = [np.concatenate([r, n], axis=2) for r, n in zip(_live_rows(steps, 302), new)]
    _check_q_rows(out, rows, bits)
    assert _attend_q(gpu, rng, out, 303, bits) <= TOL


def test_empty_cache_state(gpu):
    """A cache that was never written saves as four None slots and offset 0."""
    from mlx_motif.cache import MotifGroupedKVCache, MotifGroupedQuantizedKVCache

    for c in (MotifGroupedKVCache(), MotifGroupedQuantizedKVCache(group_size=GS, bits=4)):
        assert c.state == (None, None, None, None)
        assert c.meta_state[0] == "0"
