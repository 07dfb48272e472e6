"""Test configuration: import paths, the ``gpu`` marker, shared helpers.

CPU tests (``-m "not gpu"``) cover the oracle against its pins, the C ABI
surface (library loads, symbols, contract rejections that never touch the
GPU) and the host-side logic.  GPU tests (``-m gpu``) are the parity tests:
they call the HIP kernels through the C ABI and compare with the oracle.
"""

from __future__ import annotations

import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mlx-motif_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device); parity tests")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    return torch.device("cuda:0")


def np_to_torch(a: np.ndarray, dtype, device):
    """numpy (float16 / float32 holding bf16 values / uint32) -> torch tensor."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).view(torch.uint32).to(device)
    return torch.from_numpy(a.astype(np.float32)).to(dtype=dtype, device=device)


def torch_to_np(t):
    """torch tensor -> numpy (float64 for floats, uint32 for packed words)."""
    import torch

    t = t.detach().cpu()
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.to(torch.float32).numpy().astype(np.float64)


DTYPE_TAGS = {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}


def torch_dtype(tag: str):
    import torch

    return getattr(torch, DTYPE_TAGS[tag])


def randn(rng, shape, tag: str, scale: float = 1.0):
    """Seeded N(0, scale^2) values rounded to the element type (numpy)."""
    from oracle.oracle import round_to

    x = rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
    return round_to(x, tag).astype(np.float32) if tag != "f16" else round_to(x, tag)


@pytest.fixture
def rng():
    return np.random.default_rng(int(os.environ.get("MOTIF_TEST_SEED", "0")))
