"""Parity of the multi-row kernel with LDS-shared K/V tiles (fp16 and bf16
caches, head_dim 128), which ``motif_sdpa_dual_v_rows`` uses once a KV head has at
least 64 virtual heads (query heads x query rows): chunked prefill and long
verify slabs.  Against the oracle with the bottom-right causal mask of the
multi-row fallback (model.py:769-807) or no mask; max |gpu - oracle| <= 2e-3
for fp16 (fp32 accumulation, fp16 output) and 1e-2 for bf16 (the softmax
weights enter the bf16 matrix cores rounded to bf16; bf16 output).

Cases: query blocks of 4 and 8 waves, row splits with the merge launch (few
query blocks) and without (many), causal rows that see no key (kv_len < S),
poisoned padding past kv_len, and agreement with the chunked decode kernels
(mfma switched off routes the same call through the VALU kernels).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import np_to_torch, randn, torch_to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _run(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal, poison=False, scale_qk=1.0, tag="f16"):
    import torch

    from conftest import torch_dtype
    from mlx_motif.kernels import sdpa_dual_v_rows

    D = 128
    q = randn(rng, (B, Hq, S, D), tag, scale_qk)
    k, v1, v2 = (randn(rng, (B, Hkv, cap, D), tag) for _ in range(3))
    if poison and kv_len < cap:
        for t in (k, v1, v2):
            t[:, :, kv_len:] = 1e4
    T = lambda a: np_to_torch(a, torch_dtype(tag), gpu)  # noqa: E731
    print(f"prefill B={B} Hq={Hq} Hkv={Hkv} S={S} cap={cap} kv_len={kv_len} causal={causal} "
          f"{tag}", flush=True)
    y = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(D), kv_len=kv_len, causal=causal)
    torch.cuda.synchronize()
    assert y.shape == (B, Hq, S, 2 * D)
    ref = O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(D), kv_len, causal)
    got = torch_to_np(y)
    assert np.isfinite(got).all()
    return float(np.max(np.abs(got - ref))), y, (q, k, v1, v2)


@pytest.mark.parametrize("B,Hq,Hkv,S,cap,kv_len", [
    (1, 32, 8, 16, 3328, 3204),    # 64 heads per KV head: one 4-wave block, row splits
    (1, 32, 8, 64, 1280, 1100),    # 256 heads: 8-wave blocks? (few units -> splits)
    (1, 32, 8, 200, 1024, 1000),   # ragged last block
    (2, 8, 2, 96, 512, 400),       # batch 2
    (1, 40, 8, 33, 768, 700),      # GQA 5, ragged
])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_oracle(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal):
    err, *_ = _run(gpu, rng, B, Hq, Hkv, S, cap, kv_len, causal)
    assert err <= 2e-3, f"S={S} kv_len={kv_len} causal={causal}: {err:.3e}"


@pytest.mark.parametrize("B,Hq,Hkv,S,cap,kv_len", [
    (1, 32, 8, 16, 3328, 3204),    # 4-wave blocks, row splits
    (1, 32, 8, 200, 1024, 1000),   # ragged last block
    (1, 32, 8, 512, 3840, 3716),   # 8-wave blocks, the 512-row chunk
])
def test_prefill_bf16_matches_oracle(gpu, rng, B, Hq, Hkv, S, cap, kv_len):
    err, *_ = _run(gpu, rng, B, Hq, Hkv, S, cap, kv_len, True, poison=True, tag="bf16")
    assert err <= 1e-2, f"bf16 S={S} kv_len={kv_len}: {err:.3e}"


def test_prefill_long_chunk(gpu, rng):
    """A 512-row prefill chunk over a 3716-row cache (many query blocks, no
    row split)."""
    err, *_ = _run(gpu, rng, 1, 32, 8, 512, 3840, 3716, True)
    assert err <= 2e-3, f"{err:.3e}"


def test_prefill_rows_without_keys_and_poison(gpu, rng):
    """kv_len < S: with the bottom-right mask the first S - kv_len rows see
    no key and come out zero; rows past kv_len are poisoned."""
    err, y, _ = _run(gpu, rng, 1, 16, 4, 80, 256, 50, True, poison=True)
    assert err <= 2e-3
    assert not torch_to_np(y)[:, :, :30].any()


def test_prefill_agrees_with_valu_kernels(gpu, rng):
    import torch

    from mlx_motif import _native
    from mlx_motif.kernels import sdpa_dual_v_rows

    err, y, (q, k, v1, v2) = _run(gpu, rng, 1, 32, 8, 24, 640, 600, True)
    T = lambda a: np_to_torch(a, torch.float16, gpu)  # noqa: E731
    _native.set_tuning("mfma", 0)
    try:
        y2 = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(128), kv_len=600, causal=True)
        torch.cuda.synchronize()
    finally:
        _native.set_tuning("mfma", 1)
    assert float(np.max(np.abs(torch_to_np(y) - torch_to_np(y2)))) <= 2e-3


@pytest.mark.parametrize("S,cap,kv_len,tag", [
    (64, 3328, 3204, "f16"),     # 2048 partial rows over 16 splits: two batches of 8
    (512, 3840, 3716, "f16"),    # the 512-row chunk: 16384 rows, 2 splits
    (64, 3328, 3204, "bf16"),
])
def test_merge_launch_row_per_wave(gpu, rng, S, cap, kv_len, tag):
    """From 2048 partial rows the merge launch runs one wave per row (splits
    in batches of 8, the running maximum rescaling earlier batches); it
    matches the oracle and the one-wave-per-slice merge it replaces."""
    import torch

    from conftest import torch_dtype
    from mlx_motif import _native
    from mlx_motif.kernels import sdpa_dual_v_rows

    err, y, (q, k, v1, v2) = _run(gpu, rng, 1, 32, 8, S, cap, kv_len, True, tag=tag)
    assert err <= (2e-3 if tag == "f16" else 1e-2), f"{err:.3e}"
    T = lambda a: np_to_torch(a, torch_dtype(tag), gpu)  # noqa: E731
    _native.set_tuning("merge_rows", 0)
    try:
        y2 = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(128), kv_len=kv_len, causal=True)
        torch.cuda.synchronize()
    finally:
        _native.set_tuning("merge_rows", 1)
    d = float(np.max(np.abs(torch_to_np(y) - torch_to_np(y2))))
    assert d <= (1e-3 if tag == "f16" else 8e-3), f"{d:.3e}"


@pytest.mark.parametrize("B,Hq,Hkv,S,cap,kv_len,tag", [
    (1, 32, 8, 200, 1024, 1000, "f16"),   # 800 heads per KV head: a ragged 256-head block
    (2, 40, 8, 130, 512, 400, "f16"),     # batch 2, GQA 5
    (1, 32, 8, 512, 3840, 3716, "f16"),   # the 512-row chunk (2 blocks per wave by default)
    (1, 32, 8, 512, 3840, 3716, "bf16"),
])
@pytest.mark.parametrize("ncb", [1, 2])
def test_prefill_column_blocks_per_wave(gpu, rng, B, Hq, Hkv, S, cap, kv_len, tag, ncb):
    """The 8-wave kernel with one or two 16-head column blocks per wave (two:
    each K/V fragment read from LDS feeds both blocks' MFMAs) against the
    oracle."""
    from mlx_motif import _native

    _native.set_tuning("prefill_ncb", ncb)
    try:
        err, *_ = _run(gpu, rng, B, Hq, Hkv, S, cap, kv_len, True, poison=True, tag=tag)
    finally:
        _native.set_tuning("prefill_ncb", 0)
    assert err <= (2e-3 if tag == "f16" else 1e-2), f"ncb={ncb} S={S} {tag}: {err:.3e}"


@pytest.mark.parametrize("S,cap,kv_len,tag", [
    (64, 3328, 3204, "f16"),     # 2048 partial rows over 16 splits
    (512, 3840, 3716, "f16"),    # the 512-row chunk
    (512, 3840, 3716, "bf16"),
    (512, 1024, 600, "f16"),     # causal rows of splits that see no key
])
def test_fp16_split_partials(gpu, rng, S, cap, kv_len, tag):
    """The shared-tile kernels store split partials as fp16 o / l when the
    row-per-wave merge reads them (half the partial bytes); the result stays
    within the oracle bar and within 1e-3 (bf16: 8e-3) of fp32 partials."""
    import torch

    from conftest import torch_dtype
    from mlx_motif import _native
    from mlx_motif.kernels import sdpa_dual_v_rows

    err, y, (q, k, v1, v2) = _run(gpu, rng, 1, 32, 8, S, cap, kv_len, True, tag=tag)
    assert err <= (2e-3 if tag == "f16" else 1e-2), f"{err:.3e}"
    T = lambda a: np_to_torch(a, torch_dtype(tag), gpu)  # noqa: E731
    _native.set_tuning("part_f16", 0)
    try:
        y2 = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(128), kv_len=kv_len,
                              causal=True)
        torch.cuda.synchronize()
    finally:
        _native.set_tuning("part_f16", 1)
    ref = O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(128), kv_len, True)
    assert float(np.max(np.abs(torch_to_np(y2) - ref))) <= (2e-3 if tag == "f16" else 1e-2)
    d = float(np.max(np.abs(torch_to_np(y) - torch_to_np(y2))))
    assert d <= (1e-3 if tag == "f16" else 8e-3), f"{d:.3e}"


def test_bf16_split_partials_beyond_fp16_range(gpu, rng):
    """Split partials over a bf16 cache stay fp32: o / l is a convex
    combination of V rows, which a bf16 cache may hold beyond fp16's 65504
    (here V = 2e5 + N(0, 1e4^2), so every output is near 2e5), where fp16
    partials would read inf.  2048 partial rows (the row-per-wave merge) over
    16 splits; the bf16 bar scales with the V magnitude."""
    import torch

    from mlx_motif.kernels import sdpa_dual_v_rows

    S, cap, kv_len, D, vs = 64, 3328, 3204, 128, 2.5e5
    q = randn(rng, (1, 32, S, D), "bf16")
    k = randn(rng, (1, 8, cap, D), "bf16")
    v1, v2 = (O.round_to(randn(rng, (1, 8, cap, D), "f32", 1e4) + np.float32(2e5),
                         "bf16").astype(np.float32) for _ in range(2))
    T = lambda a: np_to_torch(a, torch.bfloat16, gpu)  # noqa: E731
    print(f"bf16 prefill S={S} kv_len={kv_len} v ~ 2e5", flush=True)
    y = sdpa_dual_v_rows(T(q), T(k), T(v1), T(v2), 1 / np.sqrt(D), kv_len=kv_len, causal=True)
    torch.cuda.synchronize()
    got = torch_to_np(y)
    ref = O.sdpa_dual_v(q, k, v1, v2, 1 / np.sqrt(D), kv_len, True)
    assert np.isfinite(got).all()
    assert float(np.min(np.abs(ref))) > 65504  # every output lies past fp16's range
    err = float(np.max(np.abs(got - ref)))
    assert err <= 1e-2 * vs, f"{err:.3e}"
