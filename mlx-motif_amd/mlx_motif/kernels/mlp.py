"""Fused PolyNorm and the dequant probe (test helper).

``polynorm(x, weight, bias, eps=1e-6)``:
``y = w0*rms(x^3) + w1*rms(x^2) + w2*rms(x) + b`` with
``rms(z) = z * rsqrt(mean(z^2) + eps)`` over the last axis, as in
``src/mlx_motif/kernels/mlp.py:108-157``; runs ``motif_polynorm``, which reads
x from HBM once.  ``_dequant_probe`` keeps the probe's signature
(``mlp.py:213-255``) over ``motif_dequantize``.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common
from .quant import dequantize


def polynorm_reference(x, weight, bias, eps: float):
    """Torch-op reference (``mlp.py:108-116``)."""

    def _rms(z):
        return z * torch.rsqrt((z * z).mean(dim=-1, keepdim=True) + eps)

    x2 = x * x
    x3 = x2 * x
    return weight[0] * _rms(x3) + weight[1] * _rms(x2) + weight[2] * _rms(x) + bias


def polynorm(x, weight, bias, eps: float = 1e-6):
    """Fused PolyNorm over the last axis; ``weight`` (3,), ``bias`` (1,) are cast
    to ``x.dtype`` first (as the reference wrapper does)."""
    if _common._DISABLE:
        return polynorm_reference(x, weight, bias, eps)
    *lead, D = x.shape
    rows = 1
    for n in lead:
        rows *= n
    if rows == 0:
        return torch.zeros_like(x)
    dev = _native.require_device(x)
    xf = _common.contiguous(x)
    w = weight.to(device=dev, dtype=x.dtype).contiguous()
    b = bias.to(device=dev, dtype=x.dtype).contiguous()
    y = torch.empty_like(xf)
    _native.check(
        _native.lib().motif_polynorm(
            xf.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), _native.dtype_code(x.dtype),
            rows, D, float(eps), _native.stream_of(dev),
        )
    )
    return y.reshape(x.shape)


def _dequant_probe(data, scales, biases, group_size: int = 64, bits: int = 4):
    """Dequantise packed MLX-affine triples; output dtype = ``scales.dtype``."""
    *lead, n_uint = data.shape
    el_per_int = 32 // bits
    D = n_uint * el_per_int
    assert D % 32 == 0 and D % group_size == 0
    rows = 1
    for n in lead:
        rows *= n
    if rows == 0:
        return torch.zeros((*lead, D), dtype=scales.dtype, device=data.device)
    return dequantize(data, scales, biases, group_size=group_size, bits=bits)
