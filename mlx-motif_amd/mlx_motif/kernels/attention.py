"""Shared-QK dual-V SDPA decode: ``sdpa_dual_v`` and ``sdpa_dual_v_q4``.

``y = [softmax(scale * q K^T) V1  ||  softmax(scale * q K^T) V2]`` for every
query head, with query head ``h`` reading KV head ``h // (H_q / H_kv)``.
Same call signatures, defaults, assertion messages and output layout as
``src/mlx_motif/kernels/attention.py:181-260, 473-645``; the work runs in
the split-KV HIP kernels of ``libmotif_hip`` (``motif_sdpa_dual_v``,
``motif_sdpa_dual_v_q``).

``sdpa_dual_v_rows`` / ``sdpa_dual_v_q4_rows`` extend the decode kernels to
``S_q > 1`` query rows with the bottom-right causal mask of a
speculative-verify or chunked-prefill step (row ``i`` sees keys
``[0, kv_len - S_q + i]``); the reference runs that case through four masked
``mx.fast.scaled_dot_product_attention`` calls (``model.py:769-807``).
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common
from .quant import dequantize_reference


# ------------------------------------------------------------ reference ---
def _sdpa_reference(q, k, v, scale, mask=None):
    """fp32 softmax attention with MLX's GQA broadcast (head h -> h // G)."""
    H_q, H_kv = q.shape[1], k.shape[1]
    if H_q != H_kv:
        g = H_q // H_kv
        k = torch.repeat_interleave(k, g, dim=1)
        v = torch.repeat_interleave(v, g, dim=1)
    qf = q.to(torch.float32) * scale
    kt = k.to(torch.float32).transpose(-1, -2).contiguous()
    s = torch.matmul(qf, kt)
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v.to(torch.float32).contiguous())


def _causal_mask(S_q: int, kv_len: int, device) -> torch.Tensor:
    rows = torch.arange(S_q, device=device)[:, None]
    cols = torch.arange(kv_len, device=device)[None, :]
    return cols <= (kv_len - S_q + rows)


def sdpa_dual_v_reference(q, k, v1, v2, scale: float, mask=None):
    """``cat(SDPA(q,k,v1), SDPA(q,k,v2), axis=-1)`` in fp32 torch ops, cast to
    ``q.dtype`` (the reference: ``attention.py:181-187``)."""
    a1 = _sdpa_reference(q, k, v1, scale, mask)
    a2 = _sdpa_reference(q, k, v2, scale, mask)
    return torch.cat([a1, a2], dim=-1).to(q.dtype)


def sdpa_dual_v_q4_reference(q, k_q, v1_q, v2_q, scale, group_size=64, bits=4, kv_len=None):
    """Dequantise K, V1, V2 (live region) then ``sdpa_dual_v_reference``
    (the reference: ``attention.py:473-507``)."""
    if kv_len is not None:
        k_q = tuple(x[..., :kv_len, :] for x in k_q)
        v1_q = tuple(x[..., :kv_len, :] for x in v1_q)
        v2_q = tuple(x[..., :kv_len, :] for x in v2_q)
    k = dequantize_reference(*k_q, group_size=group_size, bits=bits)
    v1 = dequantize_reference(*v1_q, group_size=group_size, bits=bits)
    v2 = dequantize_reference(*v2_q, group_size=group_size, bits=bits)
    return sdpa_dual_v_reference(q, k, v1, v2, scale)


# -------------------------------------------------------------- kernels ---
def _ws(dev, B, H_q, H_kv, S_q, kv_len, D):
    n = _native.lib().motif_sdpa_workspace_bytes(B, H_q, H_kv, S_q, kv_len, D)
    buf = _native.workspace(dev, n)
    return buf.data_ptr(), buf.numel()


def sdpa_dual_v(q, k, v1, v2, scale: float, kv_len: int | None = None):
    """Shared-QK, dual-V SDPA decode with native GQA broadcast.

    ``q`` (B, H_q, 1, D); ``k, v1, v2`` (B, H_kv, KV_cap, D) full-capacity
    cache buffers; ``kv_len`` live rows (default ``KV_cap``), rows past it are
    never read.  Returns (B, H_q, 1, 2D) in ``q.dtype``.
    """
    if kv_len is None:
        kv_len = k.shape[2]

    if _common._DISABLE:
        k = k[..., :kv_len, :]
        v1 = v1[..., :kv_len, :]
        v2 = v2[..., :kv_len, :]
        return sdpa_dual_v_reference(q, k, v1, v2, scale)

    B, H_q, S_q, D = q.shape
    _, H_kv, KV_cap, _ = k.shape
    assert S_q == 1, "sdpa_dual_v is decode-only"
    assert D % 32 == 0, f"D={D} must be a multiple of 32"
    assert H_q % H_kv == 0, f"H_q={H_q} must be a multiple of H_kv={H_kv}"
    assert v1.shape == v2.shape == (B, H_kv, KV_cap, D), "v1,v2 must match (B, H_kv, KV_cap, D)"
    assert k.shape[-1] == D, "K head_dim must match Q"
    assert 0 <= kv_len <= KV_cap, f"kv_len={kv_len} must be in [0, {KV_cap}]"
    return _sdpa_fp_call(q, k, v1, v2, scale, kv_len, causal=False)


def sdpa_dual_v_rows(q, k, v1, v2, scale: float, kv_len: int | None = None, causal: bool = True):
    """Multi-row dual-V SDPA: ``q`` (B, H_q, S_q, D) against the cache with the
    bottom-right causal mask (``causal=True``) or no mask.  Returns
    (B, H_q, S_q, 2D)."""
    if kv_len is None:
        kv_len = k.shape[2]
    B, H_q, S_q, D = q.shape
    if _common._DISABLE:
        mask = _causal_mask(S_q, kv_len, q.device) if causal else None
        return sdpa_dual_v_reference(
            q, k[..., :kv_len, :], v1[..., :kv_len, :], v2[..., :kv_len, :], scale, mask
        )
    _, H_kv, KV_cap, _ = k.shape
    assert D % 32 == 0, f"D={D} must be a multiple of 32"
    assert H_q % H_kv == 0, f"H_q={H_q} must be a multiple of H_kv={H_kv}"
    assert v1.shape == v2.shape == (B, H_kv, KV_cap, D), "v1,v2 must match (B, H_kv, KV_cap, D)"
    assert k.shape[-1] == D, "K head_dim must match Q"
    assert 0 <= kv_len <= KV_cap, f"kv_len={kv_len} must be in [0, {KV_cap}]"
    return _sdpa_fp_call(q, k, v1, v2, scale, kv_len, causal=causal)


def _sdpa_fp_call(q, k, v1, v2, scale, kv_len, causal):
    dev = _native.require_device(q, k, v1, v2)
    for t in (k, v1, v2):
        if t.dtype != q.dtype:
            raise TypeError(f"k/v dtype {t.dtype} must match q dtype {q.dtype}")
    q, k, v1, v2 = (_common.contiguous(t) for t in (q, k, v1, v2))
    B, H_q, S_q, D = q.shape
    _, H_kv, KV_cap, _ = k.shape
    y = torch.empty((B, H_q, S_q, 2 * D), dtype=q.dtype, device=dev)
    ws, ws_n = _ws(dev, B, H_q, H_kv, S_q, kv_len, D)
    lib = _native.lib()
    stream = _native.stream_of(dev)
    code = _native.dtype_code(q.dtype)
    if S_q == 1 and not causal:
        st = lib.motif_sdpa_dual_v(
            q.data_ptr(), k.data_ptr(), v1.data_ptr(), v2.data_ptr(), y.data_ptr(), code,
            B, H_q, H_kv, D, KV_cap, kv_len, float(scale), ws, ws_n, stream,
        )
    else:
        st = lib.motif_sdpa_dual_v_rows(
            q.data_ptr(), k.data_ptr(), v1.data_ptr(), v2.data_ptr(), y.data_ptr(), code,
            B, H_q, H_kv, S_q, D, KV_cap, kv_len, int(causal), float(scale), ws, ws_n, stream,
        )
    _native.check(st)
    return y


def sdpa_dual_v_q4(q, k_q: tuple, v1_q: tuple, v2_q: tuple, scale: float, group_size: int = 64,
                   bits: int = 4, kv_len: int | None = None):
    """Quantised-input shared-QK dual-V SDPA decode reading the packed cache.

    ``k_q, v1_q, v2_q`` are ``(data uint32, scales, biases)`` triples of
    (B, H_kv, KV_cap, D) tensors quantised with ``group_size`` / ``bits``.
    Returns (B, H_q, 1, 2D) in ``q.dtype``.
    """
    if _common._DISABLE:
        return sdpa_dual_v_q4_reference(q, k_q, v1_q, v2_q, scale, group_size, bits, kv_len)

    k_data = k_q[0]
    B, H_q, S_q, D = q.shape
    _, H_kv, KV_cap, n_uint = k_data.shape
    if kv_len is None:
        kv_len = KV_cap
    el_per_int = 32 // bits
    assert n_uint * el_per_int == D, (
        f"k_data last axis = {n_uint} ⇒ packed D = {n_uint * el_per_int}, expected {D}"
    )
    assert S_q == 1, "sdpa_dual_v_q4 is decode-only"
    _q_contract(D, H_q, H_kv, group_size, bits, kv_len, KV_cap)
    return _sdpa_q_call(q, k_q, v1_q, v2_q, scale, group_size, bits, kv_len, causal=False)


def sdpa_dual_v_q4_rows(q, k_q, v1_q, v2_q, scale, group_size=64, bits=4, kv_len=None,
                        causal=True):
    """Multi-row (verify-slab) variant of ``sdpa_dual_v_q4``; ``q`` is
    (B, H_q, S_q, D), mask as in ``sdpa_dual_v_rows``."""
    k_data = k_q[0]
    B, H_q, S_q, D = q.shape
    _, H_kv, KV_cap, n_uint = k_data.shape
    if kv_len is None:
        kv_len = KV_cap
    if _common._DISABLE:
        sl = lambda t: tuple(x[..., :kv_len, :] for x in t)  # noqa: E731
        k = dequantize_reference(*sl(k_q), group_size=group_size, bits=bits)
        v1 = dequantize_reference(*sl(v1_q), group_size=group_size, bits=bits)
        v2 = dequantize_reference(*sl(v2_q), group_size=group_size, bits=bits)
        mask = _causal_mask(S_q, kv_len, q.device) if causal else None
        return sdpa_dual_v_reference(q, k, v1, v2, scale, mask)
    assert n_uint * (32 // bits) == D, (
        f"k_data last axis = {n_uint} ⇒ packed D = {n_uint * (32 // bits)}, expected {D}"
    )
    _q_contract(D, H_q, H_kv, group_size, bits, kv_len, KV_cap)
    return _sdpa_q_call(q, k_q, v1_q, v2_q, scale, group_size, bits, kv_len, causal=causal)


def _q_contract(D, H_q, H_kv, group_size, bits, kv_len, KV_cap):
    """The packed-layout contract of the reference wrapper (attention.py:559-608).

    Each of the reference's 32 lanes takes D/32 contiguous channels from ONE
    packed word and ONE scale group, so the wrapper rejects head dims whose
    lane block would straddle a word or a group.  The HIP kernels keep this
    contract unchanged so the two libraries accept the same shapes.
    """
    assert D % 32 == 0
    assert D % group_size == 0
    assert H_q % H_kv == 0
    assert bits in (4, 8)
    assert 0 <= kv_len <= KV_cap, f"kv_len={kv_len} must be in [0, {KV_cap}]"
    assert (32 // bits) % (D // 32) == 0, (
        f"sdpa_dual_v_q4 requires qk_per_thread | EL_PER_INT so each lane's D/32 "
        f"channels come from ONE packed uint32 (implies D/32 <= 32/bits); got "
        f"D={D}, bits={bits} -> qk_per_thread={D // 32}, EL_PER_INT={32 // bits}"
    )
    assert group_size % (D // 32) == 0, (
        f"sdpa_dual_v_q4 requires qk_per_thread | group_size so each lane's D/32 "
        f"channels share ONE scale/bias group; got D={D}, group_size={group_size} "
        f"-> qk_per_thread={D // 32}"
    )


def _sdpa_q_call(q, k_q, v1_q, v2_q, scale, group_size, bits, kv_len, causal):
    tensors = [q, *k_q, *v1_q, *v2_q]
    dev = _native.require_device(*tensors)
    for t in (k_q[1], k_q[2], v1_q[1], v1_q[2], v2_q[1], v2_q[2]):
        if t.dtype != q.dtype:
            raise TypeError(f"scales/biases dtype {t.dtype} must match q dtype {q.dtype}")
    q = _common.contiguous(q)
    k_q, v1_q, v2_q = (tuple(_common.contiguous(x) for x in t) for t in (k_q, v1_q, v2_q))
    B, H_q, S_q, D = q.shape
    _, H_kv, KV_cap, _ = k_q[0].shape
    y = torch.empty((B, H_q, S_q, 2 * D), dtype=q.dtype, device=dev)
    ws, ws_n = _ws(dev, B, H_q, H_kv, S_q, kv_len, D)
    lib = _native.lib()
    stream = _native.stream_of(dev)
    code = _native.dtype_code(q.dtype)
    ptrs = [x.data_ptr() for t in (k_q, v1_q, v2_q) for x in t]
    if S_q == 1 and not causal:
        st = lib.motif_sdpa_dual_v_q(
            q.data_ptr(), *ptrs, y.data_ptr(), code, B, H_q, H_kv, D, KV_cap, kv_len, bits,
            group_size, float(scale), ws, ws_n, stream,
        )
    else:
        st = lib.motif_sdpa_dual_v_q_rows(
            q.data_ptr(), *ptrs, y.data_ptr(), code, B, H_q, H_kv, S_q, D, KV_cap, kv_len,
            int(causal), bits, group_size, float(scale), ws, ws_n, stream,
        )
    _native.check(st)
    return y
