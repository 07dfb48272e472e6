"""Disable flag and small helpers shared by the kernel wrappers.

``MLX_MOTIF_DISABLE_KERNELS`` is read once, at import, with the same falsy set
as the reference (``src/mlx_motif/kernels/_common.py:10``).  When set, every
wrapper returns its ``*_reference`` (torch ops on whatever device the inputs
live on).  Otherwise the wrappers call the HIP kernels through the C ABI and
raise if that is impossible; there is no silent fallback.

Wrappers look the flag up as ``_common._DISABLE`` at call time, so a test can
switch it with ``monkeypatch.setattr(_common, "_DISABLE", ...)``.
"""

from __future__ import annotations

import os

import torch

_DISABLE = os.environ.get("MLX_MOTIF_DISABLE_KERNELS", "0") not in ("0", "", "false", "False")


def contiguous(t: torch.Tensor) -> torch.Tensor:
    """Row-contiguous view or copy (the reference kernels run on
    ``ensure_row_contiguous`` inputs)."""
    return t if t.is_contiguous() else t.contiguous()


def f32_scalar_tensor(value, device: torch.device) -> torch.Tensor:
    """A 1-element fp32 device tensor from a tensor or a Python number, without
    a host synchronisation when it is already a device tensor."""
    if isinstance(value, torch.Tensor):
        return value.reshape(-1)[:1].to(device=device, dtype=torch.float32).contiguous()
    return torch.tensor([float(value)], dtype=torch.float32, device=device)
