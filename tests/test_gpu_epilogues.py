"""Parity of the fused epilogues against the oracle: ``gda_post_split`` /
``gda_post`` (``motif_gda_post_split`` / ``motif_gda_post``) and PolyNorm
(``motif_polynorm``).

Shapes follow the reference's tests/test_kernels_gda_post_split.py (12.7B
decode/prefill shapes, edge channels 2d in {384, 40, 34}),
tests/test_kernels_gda.py (merged layout) and tests/test_kernels.py
(PolyNorm shapes up to (1,1,4096)), plus the prefill workloads: gda on
[1,16,3204,128] and [1,32,3204,256]/[1,8,3204,256], PolyNorm on
[3204,13824].  Outputs are fp16/bf16, so the bar is ulps of the oracle
rounded once to the output type: |gpu - ref| <= 1 ulp(ref) + 1e-5 for
fp16/bf16 outputs, 64 ulp(ref) + 1e-5 for fp32 outputs.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ULP = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7, "f32": 2.0 ** -23}


def _excess(got, ref, tag, ulps=1.0, abs_extra=1e-5):
    """max(|got - ref| - (ulps * ulp(ref) + abs_extra)): <= 0 means within the
    bar.  ulp is the output type's spacing at |ref|; abs_extra covers fp32
    rounding of terms that cancel (|terms| <= ~20 here, fp32 eps 6e-8)."""
    mag = np.maximum(np.abs(ref), 2.0 ** -14)
    ulp = ULP[tag] * 2.0 ** np.floor(np.log2(mag))
    return float(np.max(np.abs(got - ref) - (ulps * ulp + abs_extra)))


@pytest.mark.parametrize("B,q_groups,gr,S,d", [
    (1, 8, 4, 1, 128), (1, 8, 4, 32, 128), (2, 4, 4, 1, 128), (1, 2, 4, 1, 64),
])
@pytest.mark.parametrize("tag", ["f16", "bf16", "f32"])
def test_gda_post_split(gpu, rng, B, q_groups, gr, S, d, tag):
    import torch

    from mlx_motif.kernels import gda_post_split

    C = 2 * d
    q_origin = q_groups * gr
    o = randn(rng, (B, q_origin, S, C), tag)
    n = randn(rng, (B, q_groups, S, C), tag)
    w = randn(rng, (C,), tag)
    lam, lam_init, eps = 0.4321, 0.65, 1e-5
    dt = torch_dtype(tag)
    y = gda_post_split(np_to_torch(o, dt, gpu), np_to_torch(n, dt, gpu), np_to_torch(w, dt, gpu),
                       torch.tensor([lam], dtype=torch.float32, device=gpu), lam_init, gr, eps)
    assert y.shape == (B, q_origin, S, C) and y.dtype == dt
    ref = O.gda_post_split(o, n, w, lam, lam_init, gr, eps)
    assert _excess(torch_to_np(y), ref, tag, 1.0 if tag != "f32" else 64.0) <= 0


@pytest.mark.parametrize("d", [192, 20, 17])
def test_gda_post_split_edge_channels(gpu, rng, d):
    import torch

    from mlx_motif.kernels import gda_post_split

    B, q_groups, gr, S = 1, 2, 4, 3
    C = 2 * d
    o = randn(rng, (B, q_groups * gr, S, C), "f32")
    n = randn(rng, (B, q_groups, S, C), "f32")
    w = randn(rng, (C,), "f32")
    y = gda_post_split(np_to_torch(o, torch.float32, gpu), np_to_torch(n, torch.float32, gpu),
                       np_to_torch(w, torch.float32, gpu), torch.tensor([0.4321], device=gpu),
                       0.65, gr, 1e-5)
    ref = O.gda_post_split(o, n, w, 0.4321, 0.65, gr, 1e-5)
    np.testing.assert_allclose(torch_to_np(y), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,q_groups,gr,S,d", [(1, 8, 4, 1, 128), (1, 8, 4, 32, 128),
                                                (2, 2, 4, 3, 64)])
def test_gda_post_merged(gpu, rng, B, q_groups, gr, S, d):
    import torch

    from mlx_motif.kernels import gda_post

    C = 2 * d
    m = randn(rng, (B, q_groups * gr + q_groups, S, C), "f16")
    w = randn(rng, (C,), "f16")
    y = gda_post(np_to_torch(m, torch.float16, gpu), np_to_torch(w, torch.float16, gpu),
                 torch.tensor([0.3], device=gpu), 0.5, q_groups, gr, 1e-5)
    ref = O.gda_post(m, w, 0.3, 0.5, q_groups, gr, 1e-5)
    assert _excess(torch_to_np(y), ref, "f16") <= 0


@pytest.mark.parametrize("shape,gr", [((1, 16, 3204, 128), 1), ((1, 32, 3204, 256), 4)])
def test_gda_prefill_workloads(gpu, rng, shape, gr):
    import torch

    from mlx_motif.kernels import gda_post_split

    B, q_origin, S, C = shape
    o = randn(rng, shape, "f16")
    n = randn(rng, (B, q_origin // gr, S, C), "f16")
    w = O.round_to(rng.uniform(0.0, 1.0, C), "f16")
    y = gda_post_split(np_to_torch(o, torch.float16, gpu), np_to_torch(n, torch.float16, gpu),
                       np_to_torch(w, torch.float16, gpu), torch.tensor([0.37], device=gpu),
                       0.2, gr, 1e-6)
    ref = O.gda_post_split(o, n, w, 0.37, 0.2, gr, 1e-6)
    assert _excess(torch_to_np(y), ref, "f16") <= 0


@pytest.mark.parametrize("shape", [(2, 4, 16), (1, 1, 64), (3, 7, 256), (1, 1, 4096),
                                   (5, 13824), (2, 3, 20), (4, 100000), (700, 4096),
                                   (300, 8200), (513, 2056)])
@pytest.mark.parametrize("tag", ["f32", "f16", "bf16"])
def test_polynorm(gpu, rng, shape, tag):
    from mlx_motif.kernels import polynorm

    x = randn(rng, shape, tag)
    w = O.round_to(np.array([0.4, 0.3, 0.3]), tag)
    b = O.round_to(np.array([0.05]), tag)
    dt = torch_dtype(tag)
    y = polynorm(np_to_torch(x, dt, gpu), np_to_torch(w, dt, gpu), np_to_torch(b, dt, gpu), 1e-6)
    assert y.shape == x.shape and y.dtype == dt
    ref = O.polynorm(x, w, b, 1e-6)
    assert _excess(torch_to_np(y), ref, tag, 1.0 if tag != "f32" else 64.0) <= 0


def test_polynorm_prefill_workload(gpu, rng):
    """x [3204, 13824] fp16 ~ N(0,1), w ~ U(0,1)^3, b = 0."""
    import torch

    from mlx_motif.kernels import polynorm

    x = randn(rng, (3204, 13824), "f16")
    w = O.round_to(rng.uniform(0.0, 1.0, 3), "f16")
    b = O.round_to(np.zeros(1), "f16")
    y = polynorm(np_to_torch(x, torch.float16, gpu), np_to_torch(w, torch.float16, gpu),
                 np_to_torch(b, torch.float16, gpu), 1e-6)
    ref = O.polynorm(x, w, b, 1e-6)
    assert _excess(torch_to_np(y), ref, "f16") <= 0


def test_polynorm_golden_vector(gpu):
    """The reference's own golden vector (tests/golden/polynorm_reference_2x3.json)."""
    import json
    import pathlib

    import torch

    from mlx_motif.kernels import polynorm

    case = json.loads((pathlib.Path(__file__).parent / "golden" /
                       "polynorm_reference_2x3.json").read_text())
    x = torch.tensor(case["input"], dtype=torch.float32, device=gpu)
    y = polynorm(x, torch.tensor(case["weight"], device=gpu), torch.tensor(case["bias"],
                 device=gpu), case["eps"])
    np.testing.assert_allclose(torch_to_np(y), np.array(case["expected"]), rtol=2e-6, atol=2e-6)
