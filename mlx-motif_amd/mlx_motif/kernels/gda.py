"""Fused GDA (grouped differential attention) epilogue: ``gda_post_split``
and the merged-layout ``gda_post``.

``y = (o - lambda * n[h // gr]) * rsqrt(mean(d^2) + eps) * w * (1 - lambda_init)``
per output row, with the signatures, defaults and assertion of
``src/mlx_motif/kernels/gda.py:108-124, 207-341``.  The work runs in
``motif_gda_post_split`` / ``motif_gda_post``; ``lambda_full`` stays on the
device (a 1-element fp32 tensor), so no host synchronisation happens.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common


def gda_post_split_reference(attn_o, attn_n, subln_weight, lambda_full, lambda_init: float,
                             gr: int, eps: float):
    """Torch-op reference (``gda.py:207-220``).  As in the reference, an fp32
    ``lambda_full`` promotes the result to fp32."""
    n_broadcast = torch.repeat_interleave(attn_n, gr, dim=1)
    lam = lambda_full if isinstance(lambda_full, torch.Tensor) else torch.tensor(
        [float(lambda_full)], dtype=torch.float32, device=attn_o.device)
    diff = attn_o - lam.to(attn_o.device) * n_broadcast
    rms_inv = torch.rsqrt((diff * diff).mean(dim=-1, keepdim=True) + eps)
    return diff * rms_inv * subln_weight.to(attn_o.device) * (1.0 - lambda_init)


def gda_post_reference(merged, subln_weight, lambda_full, lambda_init: float, q_groups: int,
                       gr: int, eps: float):
    """Torch-op reference of the merged-layout epilogue (``gda.py:108-124``)."""
    q_origin = q_groups * gr
    return gda_post_split_reference(merged[:, :q_origin], merged[:, q_origin:], subln_weight,
                                    lambda_full, lambda_init, gr, eps)


def gda_post_split(attn_o, attn_n, subln_weight, lambda_full, lambda_init: float, gr: int,
                   eps: float = 1e-5):
    """Fused epilogue on split inputs: ``attn_o`` (B, q_origin, S, C),
    ``attn_n`` (B, q_groups, S, C) -> (B, q_origin, S, C) in ``attn_o.dtype``."""
    if _common._DISABLE:
        return gda_post_split_reference(attn_o, attn_n, subln_weight, lambda_full, lambda_init,
                                        gr, eps)
    B, q_origin, S, channels = attn_o.shape
    _, q_groups, _, _ = attn_n.shape
    assert q_origin == q_groups * gr, f"q_origin={q_origin} != q_groups({q_groups}) * gr({gr})"
    dev = _native.require_device(attn_o, attn_n)
    if attn_n.dtype != attn_o.dtype:
        raise TypeError(f"attn_n dtype {attn_n.dtype} must match attn_o dtype {attn_o.dtype}")
    o = _common.contiguous(attn_o)
    n = _common.contiguous(attn_n)
    w = subln_weight.to(device=dev, dtype=attn_o.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty_like(o)
    _native.check(
        _native.lib().motif_gda_post_split(
            o.data_ptr(), n.data_ptr(), w.data_ptr(), y.data_ptr(),
            _native.dtype_code(o.dtype), B, q_origin, q_groups, gr, S, channels,
            lam.data_ptr(), float(1.0 - lambda_init), float(eps), _native.stream_of(dev),
        )
    )
    return y


def gda_post(merged, subln_weight, lambda_full, lambda_init: float, q_groups: int, gr: int,
             eps: float = 1e-5):
    """Fused epilogue on the merged layout ``(B, q_groups*gr + q_groups, S, C)``
    -> (B, q_groups*gr, S, C)."""
    if _common._DISABLE:
        return gda_post_reference(merged, subln_weight, lambda_full, lambda_init, q_groups, gr,
                                  eps)
    B, q_heads, S, channels = merged.shape
    q_origin = q_groups * gr
    assert q_heads == q_origin + q_groups, f"q_heads={q_heads} expected {q_origin}+{q_groups}"
    dev = _native.require_device(merged)
    m = _common.contiguous(merged)
    w = subln_weight.to(device=dev, dtype=merged.dtype).contiguous()
    lam = _common.f32_scalar_tensor(lambda_full, dev)
    y = torch.empty((B, q_origin, S, channels), dtype=merged.dtype, device=dev)
    _native.check(
        _native.lib().motif_gda_post(
            m.data_ptr(), w.data_ptr(), y.data_ptr(), _native.dtype_code(m.dtype), B, q_groups,
            gr, S, channels, lam.data_ptr(), float(1.0 - lambda_init), float(eps),
            _native.stream_of(dev),
        )
    )
    return y
