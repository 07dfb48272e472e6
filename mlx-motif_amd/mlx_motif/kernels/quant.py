"""MLX-affine quantisation of the KV cache: ``quantize`` / ``dequantize``.

These stand where the reference calls ``mx.quantize`` / ``mx.dequantize``
(``src/mlx_motif/cache.py:398-402, 457-463, 498``).  Format per group of
``group_size`` values along the last axis: packed ``uint32`` words holding
``32 // bits`` unsigned codes each (value ``i`` at bits
``[(i % (32//bits)) * bits, +bits)`` of word ``i // (32//bits)``), and one
``scale`` and ``bias`` of the input dtype; ``value = scale * code + bias``.

``quantize`` runs the HIP kernel (bit-exact restatement of MLX's fp32
quantizer); ``quantize_reference`` is the same algorithm in torch ops, used
when ``MLX_MOTIF_DISABLE_KERNELS`` is set.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common


def _check_args(D: int, group_size: int, bits: int) -> None:
    assert bits in (4, 8), f"bits={bits} must be 4 or 8"
    assert group_size in (32, 64, 128), f"group_size={group_size} must be 32, 64 or 128"
    assert D % group_size == 0, f"last axis {D} must be a multiple of group_size={group_size}"


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """Quantise ``w (..., D)`` -> ``(data uint32 (..., D*bits/32),
    scales (..., D/group_size), biases (..., D/group_size))``."""
    *lead, D = w.shape
    _check_args(D, group_size, bits)
    if _common._DISABLE:
        return quantize_reference(w, group_size, bits)
    dev = _native.require_device(w)
    x = _common.contiguous(w)
    rows = x.numel() // D if D else 0
    data = torch.empty((*lead, D * bits // 32), dtype=torch.uint32, device=dev)
    scales = torch.empty((*lead, D // group_size), dtype=w.dtype, device=dev)
    biases = torch.empty_like(scales)
    _native.check(
        _native.lib().motif_quantize(
            x.data_ptr(), data.data_ptr(), scales.data_ptr(), biases.data_ptr(),
            _native.dtype_code(w.dtype), rows, D, bits, group_size, _native.stream_of(dev),
        )
    )
    return data, scales, biases


def dequantize(data: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """``dtype(float(scale) * code + float(bias))`` with dtype = scales.dtype."""
    *lead, n_uint = data.shape
    D = n_uint * (32 // bits)
    _check_args(D, group_size, bits)
    if _common._DISABLE:
        return dequantize_reference(data, scales, biases, group_size, bits)
    dev = _native.require_device(data, scales, biases)
    d = _common.contiguous(data)
    s = _common.contiguous(scales)
    b = _common.contiguous(biases)
    rows = d.numel() // n_uint if n_uint else 0
    y = torch.empty((*lead, D), dtype=scales.dtype, device=dev)
    _native.check(
        _native.lib().motif_dequantize(
            d.data_ptr(), s.data_ptr(), b.data_ptr(), y.data_ptr(),
            _native.dtype_code(scales.dtype), rows, D, bits, group_size, _native.stream_of(dev),
        )
    )
    return y


# ----------------------------------------------------------- references ---
def quantize_reference(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """Torch-op statement of the MLX affine quantizer (fp32 arithmetic):

    per group: scale = max((max-min)/n_bins, 1e-7); the larger-magnitude side
    is the edge and fixes the sign of scale; q0 = rint(edge/scale); if
    q0 != 0 then scale = edge/q0 and bias = edge, else bias = 0;
    code = clamp(rint((w - bias)/scale), 0, n_bins).
    """
    *lead, D = w.shape
    _check_args(D, group_size, bits)
    el = 32 // bits
    x = w.reshape(-1, D // group_size, group_size).to(torch.float32)
    n_bins = float((1 << bits) - 1)
    w_max = x.amax(dim=-1)
    w_min = x.amin(dim=-1)
    scale = torch.maximum((w_max - w_min) / n_bins, torch.tensor(1e-7, dtype=torch.float32))
    side = w_min.abs() > w_max.abs()
    scale = torch.where(side, scale, -scale)
    edge = torch.where(side, w_min, w_max)
    q0 = torch.round(edge / scale)
    nz = q0 != 0
    scale = torch.where(nz, edge / torch.where(nz, q0, torch.ones_like(q0)), scale)
    bias = torch.where(nz, edge, torch.zeros_like(edge))
    codes = torch.round((x - bias[..., None]) / scale[..., None]).clamp_(0.0, n_bins)
    codes = codes.to(torch.int64).reshape(-1, D // el, el)
    shifts = torch.arange(el, device=w.device, dtype=torch.int64) * bits
    words = (codes << shifts).sum(dim=-1)  # disjoint bit fields: sum == or
    data = words.to(torch.uint32).reshape(*lead, D // el)
    scales = scale.to(w.dtype).reshape(*lead, D // group_size)
    biases = bias.to(w.dtype).reshape(*lead, D // group_size)
    return data, scales, biases


def dequantize_reference(data: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                         group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """Torch-op dequantisation: ``dtype(float(scale) * code + float(bias))``."""
    *lead, n_uint = data.shape
    el = 32 // bits
    D = n_uint * el
    words = data.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(el, device=data.device, dtype=torch.int64) * bits
    codes = ((words[..., None] >> shifts) & ((1 << bits) - 1)).reshape(*lead, D)
    g = D // group_size
    s = scales.to(torch.float32).reshape(*lead, g, 1)
    b = biases.to(torch.float32).reshape(*lead, g, 1)
    out = s * codes.reshape(*lead, g, group_size).to(torch.float32) + b
    return out.reshape(*lead, D).to(scales.dtype)
