"""head_dim 64 on the fp16/bf16 matrix-core decode kernel (the reference's
"smaller d" shapes, tests/test_kernels_sdpa_dual_v.py:20 and :91), through
the C ABI (``motif_sdpa_dual_v``).

Checks, against the oracle's float64 attention (fp16 2e-3, bf16 1e-2):
  - GQA 1, 2, 4, 8 and 16 (every heads-per-workgroup variant), short
    contexts (4-wave blocks) and long ones (8-wave blocks), with the cache
    padding past kv_len poisoned;
  - batch 2 and kv_len 1;
  - the matrix-core and VALU formulations within the bar of each other;
  - a K cache that is 8-byte but not 16-byte aligned (the matrix-core kernel
    reads K 16 bytes per lane) takes the VALU kernel and stays within the bar.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_dtype, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = {"f16": 2e-3, "bf16": 1e-2}
D = 64


def _inputs(rng, B, Hq, Hkv, cap, kv_len, tag):
    q = randn(rng, (B, Hq, 1, D), tag)
    k, v1, v2 = (randn(rng, (B, Hkv, cap, D), tag) for _ in range(3))
    for t in (k, v1, v2):
        t[:, :, kv_len:] = 1e4  # poisoned padding
    return q, k, v1, v2


def _attend(gpu, arrays, kv_len, tag, k_offset=0):
    import torch

    from mlx_motif.kernels import sdpa_dual_v

    dt = torch_dtype(tag)
    q, k, v1, v2 = (np_to_torch(a, dt, gpu) for a in arrays)
    if k_offset:  # the same K values at a byte offset of 2 * k_offset
        buf = torch.empty(k.numel() + k_offset, dtype=dt, device=gpu)
        kk = buf[k_offset:].view(k.shape)
        kk.copy_(k)
        assert kk.data_ptr() % 16 == 2 * k_offset % 16
        k = kk
    y = sdpa_dual_v(q, k, v1, v2, 1.0 / np.sqrt(D), kv_len=kv_len)
    torch.cuda.synchronize()
    assert y.shape == (q.shape[0], q.shape[1], 1, 2 * D) and y.dtype == dt
    return torch_to_np(y)


@pytest.mark.parametrize("tag", ["f16", "bf16"])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (32, 4), (32, 2)])
@pytest.mark.parametrize("kv_len,cap", [(300, 384), (3204, 3328), (16000, 16128)])
def test_head_dim_64_matches_oracle(gpu, rng, tag, Hq, Hkv, kv_len, cap):
    arrays = _inputs(rng, 1, Hq, Hkv, cap, kv_len, tag)
    print(f"d64 {tag} Hq={Hq} Hkv={Hkv} kv_len={kv_len}", flush=True)
    y = _attend(gpu, arrays, kv_len, tag)
    ref = O.sdpa_dual_v(*arrays, 1.0 / np.sqrt(D), kv_len)
    err = float(np.max(np.abs(y - ref)))
    assert err <= TOL[tag], f"{tag} {(Hq, Hkv, kv_len)}: {err:.3e}"


@pytest.mark.parametrize("B,Hq,Hkv,cap,kv_len", [(2, 16, 8, 256, 200), (2, 32, 8, 1024, 1),
                                                  (1, 40, 8, 512, 385)])
def test_head_dim_64_batched_and_short(gpu, rng, B, Hq, Hkv, cap, kv_len):
    arrays = _inputs(rng, B, Hq, Hkv, cap, kv_len, "f16")
    y = _attend(gpu, arrays, kv_len, "f16")
    ref = O.sdpa_dual_v(*arrays, 1.0 / np.sqrt(D), kv_len)
    assert float(np.max(np.abs(y - ref))) <= TOL["f16"]


@pytest.mark.parametrize("tag", ["f16", "bf16"])
def test_head_dim_64_matrix_cores_agree_with_valu(gpu, rng, tag):
    from mlx_motif import _native

    arrays = _inputs(rng, 1, 32, 8, 4096, 4000, tag)
    out = []
    for mfma in (1, 0):
        _native.set_tuning("mfma", mfma)
        try:
            out.append(_attend(gpu, arrays, 4000, tag))
        finally:
            _native.set_tuning("mfma", 1)
    ref = O.sdpa_dual_v(*arrays, 1.0 / np.sqrt(D), 4000)
    for y in out:
        assert float(np.max(np.abs(y - ref))) <= TOL[tag]
    assert float(np.max(np.abs(out[0] - out[1]))) <= TOL[tag]


def test_head_dim_64_unaligned_k_takes_the_valu_kernel(gpu, rng):
    arrays = _inputs(rng, 1, 32, 8, 2048, 2000, "f16")
    y = _attend(gpu, arrays, 2000, "f16", k_offset=4)  # 8-byte aligned K
    ref = O.sdpa_dual_v(*arrays, 1.0 / np.sqrt(D), 2000)
    assert float(np.max(np.abs(y - ref))) <= TOL["f16"]
