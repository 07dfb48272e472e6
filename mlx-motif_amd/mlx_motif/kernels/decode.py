"""One GDA decode-attention step of a layer: the origin and noise dual-V
passes and the ``gda_post_split`` epilogue in one call.

The reference runs this as three kernel calls (DUAL_V path of
``src/mlx_motif/model.py:749-768``)::

    attn_origin = sdpa_dual_v(q1, k1, v1, v2, scale, kv_len=kv_seq)
    attn_noise = sdpa_dual_v(q2, k2, v1, v2, scale, kv_len=kv_seq)
    out = gda_post_split(attn_origin, attn_noise, subln.weight, lam, lambda_init, gr, eps)

``gda_decode_attention`` returns the same ``out``.  On the fp16 or bf16 cache
at head_dim 128, ``motif_gda_decode`` serves both passes from one attention
launch that reads each KV head's k1, k2, v1 and v2 rows once (the separate
calls read v1 and v2 twice), and applies the epilogue in the split merge.
``q2`` may hold any multiple of H_kv noise heads (the reference's calls are
GQA calls, and ``gda_post_split`` pairs origin head h with noise head
h // gr): one per KV head is the 12.7B layout (``motif_gda_decode``), more
take ``motif_gda_decode_heads`` (e.g. 8 origin and 8 noise heads over 4 KV
heads, gr = 1).
Other shapes compose the separate native calls inside the library.
``gda_decode_attention_q4`` is the same step over the packed q4/q8 cache
(QUANT_SDPA path, ``model.py:717-748``: two ``sdpa_dual_v_q4`` calls).

With ``new_kv=(k1_new, k2_new, v1_new, v2_new)`` either function also
writes the decode token's rows into the cache first -- the reference's
``update_and_fetch_4`` / ``update_and_fetch_4_quantized``
(``src/mlx_motif/cache.py:337, 467``) for one token -- at row ``kv_len - 1``
(``kv_len`` then counts the new row).  The fused fp16 / packed kernels store
the rows inside the attention launch, before the one wave that reads that
row block loads it; other shapes write the row first and then run the step.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common
from .attention import _q_contract, sdpa_dual_v_q4_reference, sdpa_dual_v_reference
from .gda import gda_post_split_reference
from .quant import quantize_reference


def gda_decode_attention_reference(q1, q2, k1, k2, v1, v2, scale: float, subln_weight,
                                   lambda_full, lambda_init: float, gr: int, eps: float = 1e-5,
                                   kv_len: int | None = None):
    """Torch-op composition of the reference's three calls; the attention
    outputs are rounded to ``q1.dtype`` as the reference's kernels return
    them, and the epilogue's fp32 result is rounded to ``q1.dtype``."""
    if kv_len is None:
        kv_len = k1.shape[2]
    sl = (Ellipsis, slice(0, kv_len), slice(None))
    o = sdpa_dual_v_reference(q1, k1[sl], v1[sl], v2[sl], scale).to(q1.dtype)
    n = sdpa_dual_v_reference(q2, k2[sl], v1[sl], v2[sl], scale).to(q1.dtype)
    y = gda_post_split_reference(o, n, subln_weight.to(q1.dtype), lambda_full, lambda_init, gr,
                                 eps)
    return y.to(q1.dtype)


def _new_rows(new_kv, B, H_kv, D, dtype, kv_len):
    """Checks the decode token's four (B, H_kv, 1, D) rows."""
    if len(new_kv) != 4:
        raise ValueError("new_kv must be (k1_new, k2_new, v1_new, v2_new)")
    if kv_len < 1:
        raise ValueError(f"kv_len={kv_len} must count the appended row (>= 1)")
    for t in new_kv:
        assert tuple(t.shape) == (B, H_kv, 1, D), "new_kv rows must be (B, H_kv, 1, D)"
        if t.dtype != dtype:
            raise TypeError(f"new_kv dtype {t.dtype} must match q1 dtype {dtype}")
    return tuple(_common.contiguous(t) for t in new_kv)


def _write_rows_reference(caches, new_kv, kv_len):
    """Torch-op cache write of one token at row ``kv_len - 1``."""
    for c, r in zip(caches, new_kv):
        c[:, :, kv_len - 1:kv_len, :] = r


def _write_rows_q_reference(slots, new_kv, kv_len, group_size, bits):
    """Quantise the token's rows (``quantize_reference``) and store the
    (data, scales, biases) triples at row ``kv_len - 1``."""
    for t, r in zip(slots, new_kv):
        for dst, src in zip(t, quantize_reference(r, group_size, bits)):
            dst[:, :, kv_len - 1:kv_len, :] = src


def _check_q_slots(slots, B, H_kv, KV_cap, D, bits, group_size, dtype):
    """Checks the four packed ``(data, scales, biases)`` slots against the
    step's shape: data (B, H_kv, KV_cap, D*bits/32) uint32, scales and biases
    (B, H_kv, KV_cap, D/group_size) of the query dtype.  The native entry
    points take bare pointers, so this is the only shape check they get."""
    n_uint = D * bits // 32
    if len(slots) != 4 or any(len(t) != 3 for t in slots):
        raise ValueError("packed slots must be four (data, scales, biases) triples")
    for t in slots:
        assert tuple(t[0].shape) == (B, H_kv, KV_cap, n_uint), (
            f"packed data {tuple(t[0].shape)} must be (B, H_kv, KV_cap, D*bits/32) = "
            f"{(B, H_kv, KV_cap, n_uint)}")
        if t[0].dtype not in (torch.uint32, torch.int32):
            raise TypeError(f"packed data dtype {t[0].dtype} must be uint32")
        for x in t[1:]:
            assert tuple(x.shape) == (B, H_kv, KV_cap, D // group_size), (
                f"scales/biases {tuple(x.shape)} must be (B, H_kv, KV_cap, D/group_size) = "
                f"{(B, H_kv, KV_cap, D // group_size)}")
            if x.dtype != dtype:
                raise TypeError(f"scales/biases dtype {x.dtype} must match q dtype {dtype}")


def _noise_heads(q1, q2, H_kv, gr, name):
    """Noise heads of the step (q2's head count): the reference's contract
    q_origin == q_groups * gr (gda.py:248), with q_groups a multiple of H_kv
    since the noise pass is a GQA call (attention.py:237-243)."""
    B, H_o, S_q, D = q1.shape
    assert S_q == 1 and q2.shape[2] == 1, f"{name} is decode-only"
    H_n = q2.shape[1]
    assert q2.shape == (B, H_n, 1, D), "q2 must be (B, q_groups, 1, D)"
    assert H_o == H_n * gr, f"q_origin={H_o} != q_groups({H_n}) * gr({gr})"
    assert H_n % H_kv == 0, f"q_groups={H_n} must be a multiple of H_kv={H_kv}"
    return H_n


def _require_in_place(tensors):
    for t in tensors:
        if not t.is_contiguous():
            raise ValueError("new_kv writes the cache in place: cache buffers must be "
                             "contiguous")


def gda_decode_attention(q1, q2, k1, k2, v1, v2, scale: float, subln_weight, lambda_full,
                         lambda_init: float, gr: int, eps: float = 1e-5,
                         kv_len: int | None = None, new_kv=None):
    """``q1`` (B, q_groups*gr, 1, D) origin queries, ``q2`` (B, q_groups, 1, D)
    noise queries with q_groups a multiple of H_kv (H_kv in the 12.7B
    layout); ``k1, k2, v1, v2`` (B, H_kv, KV_cap, D) full-capacity 4-slot
    cache buffers with ``kv_len`` live rows (default ``KV_cap``).  With
    ``new_kv`` the token's rows are first written at row ``kv_len - 1``.
    Returns (B, q_groups*gr, 1, 2D) in ``q1.dtype``."""
    if kv_len is None:
        kv_len = k1.shape[2]
    if new_kv is not None:
        new_kv = _new_rows(new_kv, q1.shape[0], k1.shape[1], q1.shape[3], q1.dtype, kv_len)
        _require_in_place((k1, k2, v1, v2))
    if _common._DISABLE:
        if new_kv is not None:
            assert kv_len <= k1.shape[2], f"kv_len={kv_len} exceeds KV_cap={k1.shape[2]}"
            _write_rows_reference((k1, k2, v1, v2), new_kv, kv_len)
        return gda_decode_attention_reference(q1, q2, k1, k2, v1, v2, scale, subln_weight,
                                              lambda_full, lambda_init, gr, eps, kv_len)
    B, H_o, S_q, D = q1.shape
    _, H_kv, KV_cap, _ = k1.shape
    H_n = _noise_heads(q1, q2, H_kv, gr, "gda_decode_attention")
    assert D % 32 == 0, f"D={D} must be a multiple of 32"
    for t in (k2, v1, v2):
        assert t.shape == (B, H_kv, KV_cap, D), "k2,v1,v2 must match (B, H_kv, KV_cap, D)"
    assert 0 <= kv_len <= KV_cap, f"kv_len={kv_len} must be in [0, {KV_cap}]"
    dev = _native.require_device(q1, q2, k1, k2, v1, v2, *(new_kv or ()))
    for t in (q2, k1, k2, v1, v2):
        if t.dtype != q1.dtype:
            raise TypeError(f"dtype {t.dtype} must match q1 dtype {q1.dtype}")
    q1, q2, k1, k2, v1, v2 = (_common.contiguous(t) for t in (q1, q2, k1, k2, v1, v2))
    w = subln_weight.to(device=dev, dtype=q1.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty((B, H_o, 1, 2 * D), dtype=q1.dtype, device=dev)
    lib = _native.lib()
    caches = (k1.data_ptr(), k2.data_ptr(), v1.data_ptr(), v2.data_ptr())
    if H_n != H_kv:  # several noise heads per KV head
        ws = _native.workspace(dev, lib.motif_gda_decode_heads_workspace_bytes(
            B, H_o, H_n, H_kv, kv_len, D))
        rows = tuple(t.data_ptr() for t in new_kv) if new_kv is not None else (None,) * 4
        _native.check(lib.motif_gda_decode_heads(
            q1.data_ptr(), q2.data_ptr(), *rows, *caches, w.data_ptr(), lam.data_ptr(),
            float(1.0 - lambda_init), float(eps), y.data_ptr(), _native.dtype_code(q1.dtype), B,
            H_o, H_n, H_kv, D, KV_cap, kv_len, float(scale), ws.data_ptr(), ws.numel(),
            _native.stream_of(dev)))
        return y
    n = lib.motif_gda_decode_workspace_bytes(B, H_kv, gr, kv_len, D)
    ws = _native.workspace(dev, n)
    tail = (w.data_ptr(), lam.data_ptr(), float(1.0 - lambda_init), float(eps), y.data_ptr(),
            _native.dtype_code(q1.dtype), B, H_kv, gr, D, KV_cap, kv_len, float(scale),
            ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    if new_kv is None:
        rc = lib.motif_gda_decode(q1.data_ptr(), q2.data_ptr(), *caches, *tail)
    else:
        rc = lib.motif_gda_decode_append(q1.data_ptr(), q2.data_ptr(),
                                         *(t.data_ptr() for t in new_kv), *caches, *tail)
    _native.check(rc)
    return y


def gda_decode_attention_q4_reference(q1, q2, k1_q, k2_q, v1_q, v2_q, scale: float,
                                      subln_weight, lambda_full, lambda_init: float, gr: int,
                                      group_size: int = 64, bits: int = 4, eps: float = 1e-5,
                                      kv_len: int | None = None):
    """Torch-op composition of the packed-cache step (model.py:717-748)."""
    o = sdpa_dual_v_q4_reference(q1, k1_q, v1_q, v2_q, scale, group_size, bits,
                                 kv_len).to(q1.dtype)
    n = sdpa_dual_v_q4_reference(q2, k2_q, v1_q, v2_q, scale, group_size, bits,
                                 kv_len).to(q1.dtype)
    y = gda_post_split_reference(o, n, subln_weight.to(q1.dtype), lambda_full, lambda_init, gr,
                                 eps)
    return y.to(q1.dtype)


def gda_decode_attention_q4(q1, q2, k1_q: tuple, k2_q: tuple, v1_q: tuple, v2_q: tuple,
                            scale: float, subln_weight, lambda_full, lambda_init: float, gr: int,
                            group_size: int = 64, bits: int = 4, eps: float = 1e-5,
                            kv_len: int | None = None, new_kv=None):
    """The decode step over the packed cache: each ``*_q`` is a ``(data
    uint32, scales, biases)`` triple of (B, H_kv, KV_cap, ...) tensors as
    ``sdpa_dual_v_q4`` takes them.  With ``new_kv`` the token's rows (in
    ``q1.dtype``) are first quantised into row ``kv_len - 1``.  ``q2`` as
    for ``gda_decode_attention``.  Returns (B, q_groups*gr, 1, 2D) in
    ``q1.dtype``."""
    B, H_o, S_q, D = q1.shape
    _, H_kv, KV_cap, n_uint = k1_q[0].shape
    if kv_len is None:
        kv_len = KV_cap
    slots = (k1_q, k2_q, v1_q, v2_q)
    if new_kv is not None:
        new_kv = _new_rows(new_kv, B, H_kv, D, q1.dtype, kv_len)
        _require_in_place([x for t in slots for x in t])
    if _common._DISABLE:
        if new_kv is not None:
            assert kv_len <= KV_cap, f"kv_len={kv_len} exceeds KV_cap={KV_cap}"
            _write_rows_q_reference(slots, new_kv, kv_len, group_size, bits)
        return gda_decode_attention_q4_reference(q1, q2, k1_q, k2_q, v1_q, v2_q, scale,
                                                 subln_weight, lambda_full, lambda_init, gr,
                                                 group_size, bits, eps, kv_len)
    assert n_uint * (32 // bits) == D, (
        f"k_data last axis = {n_uint} ⇒ packed D = {n_uint * (32 // bits)}, expected {D}"
    )
    H_n = _noise_heads(q1, q2, H_kv, gr, "gda_decode_attention_q4")
    _q_contract(D, H_o, H_kv, group_size, bits, kv_len, KV_cap)
    _check_q_slots(slots, B, H_kv, KV_cap, D, bits, group_size, q1.dtype)
    dev = _native.require_device(q1, q2, *(x for t in slots for x in t), *(new_kv or ()))
    if q2.dtype != q1.dtype:
        raise TypeError(f"q2 dtype {q2.dtype} must match q1 dtype {q1.dtype}")
    q1, q2 = _common.contiguous(q1), _common.contiguous(q2)
    slots = tuple(tuple(_common.contiguous(x) for x in t) for t in slots)
    w = subln_weight.to(device=dev, dtype=q1.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty((B, H_o, 1, 2 * D), dtype=q1.dtype, device=dev)
    lib = _native.lib()
    ptrs = [x.data_ptr() for t in slots for x in t]
    if H_n != H_kv:  # several noise heads per KV head
        ws = _native.workspace(dev, lib.motif_gda_decode_heads_workspace_bytes(
            B, H_o, H_n, H_kv, kv_len, D))
        rows = tuple(t.data_ptr() for t in new_kv) if new_kv is not None else (None,) * 4
        _native.check(lib.motif_gda_decode_q_heads(
            q1.data_ptr(), q2.data_ptr(), *rows, *ptrs, w.data_ptr(), lam.data_ptr(),
            float(1.0 - lambda_init), float(eps), y.data_ptr(), _native.dtype_code(q1.dtype), B,
            H_o, H_n, H_kv, D, KV_cap, kv_len, bits, group_size, float(scale), ws.data_ptr(),
            ws.numel(), _native.stream_of(dev)))
        return y
    ws = _native.workspace(dev, lib.motif_gda_decode_workspace_bytes(B, H_kv, gr, kv_len, D))
    tail = (w.data_ptr(), lam.data_ptr(), float(1.0 - lambda_init), float(eps), y.data_ptr(),
            _native.dtype_code(q1.dtype), B, H_kv, gr, D, KV_cap, kv_len, bits, group_size,
            float(scale), ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    if new_kv is None:
        rc = lib.motif_gda_decode_q(q1.data_ptr(), q2.data_ptr(), *ptrs, *tail)
    else:
        rc = lib.motif_gda_decode_q_append(q1.data_ptr(), q2.data_ptr(),
                                           *(t.data_ptr() for t in new_kv), *ptrs, *tail)
    _native.check(rc)
    return y


def gda_decode_attention_from_proj(q_proj, k_proj, v_proj, k1, k2, v1, v2, scale: float,
                                   subln_weight, lambda_full, lambda_init: float, gr: int,
                                   offset: int, theta: float = 10000.0, eps: float = 1e-5,
                                   origin_first: bool = False, rope_scaling=None):
    """A layer's whole decode attention from the projection outputs:
    ``q_proj`` (B, 1, H_kv*(gr+1)*D), ``k_proj`` and ``v_proj`` (B, 1,
    2*H_kv*D) (k_ratio 1).  RoPE at position ``offset`` (``rope_split4``'s
    rounding), the token's rows written at row ``offset`` of the 4-slot fp
    cache ``k1, k2, v1, v2``, then the step over ``offset + 1`` rows.  On the
    fp16/bf16 cache at head_dim 128 this is ``motif_gda_decode_proj`` (the
    attention launch ropes and writes; then the merge); otherwise
    ``rope_split4`` followed by ``gda_decode_attention``.  ``rope_scaling``:
    None, or a default / linear config (``rope.rope_position_scale``)."""
    from .rope import rope_position_scale, rope_split4, rope_split4_reference

    pscale = rope_position_scale(rope_scaling)

    B, S, nq = q_proj.shape
    H_kv = k1.shape[1]
    assert S == 1, "gda_decode_attention_from_proj is decode-only"
    D = nq // (H_kv * (gr + 1))
    assert nq == H_kv * (gr + 1) * D, "q width must be H_kv*(gr+1)*D"
    kv_len = offset + 1
    if _common._DISABLE:
        q1, q2, *_ = rope_split4_reference(q_proj, k_proj, v_proj, H_kv, gr, H_kv, 1, offset,
                                           theta, origin_first, caches=(k1, k2, v1, v2),
                                           position_scale=pscale)
        return gda_decode_attention_reference(q1, q2, k1, k2, v1, v2, scale, subln_weight,
                                              lambda_full, lambda_init, gr, eps, kv_len)
    assert k_proj.shape == (B, 1, 2 * H_kv * D) and v_proj.shape == (B, 1, 2 * H_kv * D), (
        "k_proj and v_proj must be (B, 1, 2*H_kv*D)")
    KV_cap = k1.shape[2]
    for t in (k1, k2, v1, v2):
        assert t.shape == (B, H_kv, KV_cap, D), "cache slots must be (B, H_kv, KV_cap, D)"
    _require_in_place((k1, k2, v1, v2))
    assert 0 <= offset < KV_cap, f"offset={offset} must be in [0, {KV_cap})"
    dev = _native.require_device(q_proj, k_proj, v_proj, k1, k2, v1, v2)
    for t in (k_proj, v_proj, k1, k2, v1, v2):
        if t.dtype != q_proj.dtype:
            raise TypeError(f"dtype {t.dtype} must match q dtype {q_proj.dtype}")
    q_proj, k_proj, v_proj = (_common.contiguous(t) for t in (q_proj, k_proj, v_proj))
    w = subln_weight.to(device=dev, dtype=q_proj.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty((B, H_kv * gr, 1, 2 * D), dtype=q_proj.dtype, device=dev)
    lib = _native.lib()
    ws = _native.workspace(dev, lib.motif_gda_decode_workspace_bytes(B, H_kv, gr, kv_len, D))
    rc = lib.motif_gda_decode_proj_scaled(
        q_proj.data_ptr(), k_proj.data_ptr(), v_proj.data_ptr(), k1.data_ptr(), k2.data_ptr(),
        v1.data_ptr(), v2.data_ptr(), w.data_ptr(), lam.data_ptr(), float(1.0 - lambda_init),
        float(eps), y.data_ptr(), _native.dtype_code(q_proj.dtype), B, H_kv, gr, D, KV_cap,
        kv_len, float(scale), float(theta), float(pscale), int(bool(origin_first)),
        ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    if rc == _native.MOTIF_ERR_UNSUPPORTED:  # the two native calls
        q1, q2, *_ = rope_split4(q_proj, k_proj, v_proj, H_kv, gr, H_kv, 1, offset, theta,
                                 origin_first, caches=(k1, k2, v1, v2),
                                 rope_scaling=rope_scaling)
        return gda_decode_attention(q1, q2, k1, k2, v1, v2, scale, subln_weight, lambda_full,
                                    lambda_init, gr, eps, kv_len=kv_len)
    _native.check(rc)
    return y


def gda_decode_attention_q4_from_proj(q_proj, k_proj, v_proj, k1_q: tuple, k2_q: tuple,
                                      v1_q: tuple, v2_q: tuple, scale: float, subln_weight,
                                      lambda_full, lambda_init: float, gr: int, offset: int,
                                      group_size: int = 64, bits: int = 4,
                                      theta: float = 10000.0, eps: float = 1e-5,
                                      origin_first: bool = False, rope_scaling=None):
    """``gda_decode_attention_from_proj`` over the packed cache: the token's
    roped k rows and v rows are quantised into row ``offset`` of the packed
    slots.  ``motif_gda_decode_q_proj`` when the fused kernel takes the
    shape, else ``rope_split4`` then ``gda_decode_attention_q4(new_kv=...)``
    (the same values bit for bit).  ``rope_scaling``: None, or a default /
    linear config."""
    from .rope import rope_position_scale, rope_split4, rope_split4_reference

    pscale = rope_position_scale(rope_scaling)

    B, S, nq = q_proj.shape
    H_kv = k1_q[0].shape[1]
    assert S == 1, "gda_decode_attention_q4_from_proj is decode-only"
    D = nq // (H_kv * (gr + 1))
    assert nq == H_kv * (gr + 1) * D, "q width must be H_kv*(gr+1)*D"
    kv_len = offset + 1
    slots = (k1_q, k2_q, v1_q, v2_q)
    if _common._DISABLE:
        q1, q2, *rows = rope_split4_reference(q_proj, k_proj, v_proj, H_kv, gr, H_kv, 1, offset,
                                              theta, origin_first, position_scale=pscale)
        return gda_decode_attention_q4(q1, q2, *slots, scale, subln_weight, lambda_full,
                                       lambda_init, gr, group_size, bits, eps, kv_len=kv_len,
                                       new_kv=rows)
    KV_cap = k1_q[0].shape[2]
    _q_contract(D, H_kv * gr, H_kv, group_size, bits, kv_len, KV_cap)
    assert k_proj.shape == (B, 1, 2 * H_kv * D) and v_proj.shape == (B, 1, 2 * H_kv * D), (
        "k_proj and v_proj must be (B, 1, 2*H_kv*D)")
    for t in (k_proj, v_proj):
        if t.dtype != q_proj.dtype:
            raise TypeError(f"k_proj/v_proj dtype {t.dtype} must match q dtype {q_proj.dtype}")
    _check_q_slots(slots, B, H_kv, KV_cap, D, bits, group_size, q_proj.dtype)
    _require_in_place([x for t in slots for x in t])
    dev = _native.require_device(q_proj, k_proj, v_proj, *(x for t in slots for x in t))
    q_proj, k_proj, v_proj = (_common.contiguous(t) for t in (q_proj, k_proj, v_proj))
    w = subln_weight.to(device=dev, dtype=q_proj.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty((B, H_kv * gr, 1, 2 * D), dtype=q_proj.dtype, device=dev)
    lib = _native.lib()
    ws = _native.workspace(dev, lib.motif_gda_decode_workspace_bytes(B, H_kv, gr, kv_len, D))
    rc = lib.motif_gda_decode_q_proj_scaled(
        q_proj.data_ptr(), k_proj.data_ptr(), v_proj.data_ptr(),
        *(x.data_ptr() for t in slots for x in t), w.data_ptr(), lam.data_ptr(),
        float(1.0 - lambda_init), float(eps), y.data_ptr(), _native.dtype_code(q_proj.dtype), B,
        H_kv, gr, D, KV_cap, kv_len, bits, group_size, float(scale), float(theta), float(pscale),
        int(bool(origin_first)), ws.data_ptr(), ws.numel(), _native.stream_of(dev))
    if rc == _native.MOTIF_ERR_UNSUPPORTED:  # the two native calls
        q1, q2, *rows = rope_split4(q_proj, k_proj, v_proj, H_kv, gr, H_kv, 1, offset, theta,
                                    origin_first, rope_scaling=rope_scaling)
        return gda_decode_attention_q4(q1, q2, *slots, scale, subln_weight, lambda_full,
                                       lambda_init, gr, group_size, bits, eps, kv_len=kv_len,
                                       new_kv=rows)
    _native.check(rc)
    return y
