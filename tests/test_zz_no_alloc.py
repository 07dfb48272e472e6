"""motif_sdpa_dual_v_noalloc (static per-device scratch, allocates nothing)
against motif_sdpa_dual_v with a caller workspace, both through the C ABI:
bit-identical outputs on two calls in a row (the second smaller), with the
split merge as a second launch and inside the attention launch (whose
counters the scratch carries from call to call)."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def _inputs(gpu, seed, dtype, B, Hq, Hkv, cap, D=128):
    import torch

    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).to(dtype)  # noqa: E731
    return mk(B, Hq, 1, D), mk(B, Hkv, cap, D), mk(B, Hkv, cap, D), mk(B, Hkv, cap, D)


def _call_both(gpu, dtype, B, Hq, Hkv, cap, kv_len, seed):
    import torch

    from mlx_motif import _native

    lib = _native.lib()
    q, k, v1, v2 = _inputs(gpu, seed, dtype, B, Hq, Hkv, cap)
    D = q.shape[-1]
    code = _native.dtype_code(dtype)
    st = _native.stream_of(gpu)
    y_ws = torch.full((B, Hq, 1, 2 * D), float("nan"), dtype=dtype, device=gpu)
    y_na = torch.full((B, Hq, 1, 2 * D), float("nan"), dtype=dtype, device=gpu)
    nbytes = lib.motif_sdpa_workspace_bytes(B, Hq, Hkv, 1, kv_len, D)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    args = (code, B, Hq, Hkv, D, cap, kv_len, 0.0884)
    print(f"sdpa_dual_v workspace dtype={dtype} B={B} Hq={Hq} Hkv={Hkv} kv_len={kv_len}",
          flush=True)
    _native.check(lib.motif_sdpa_dual_v(q.data_ptr(), k.data_ptr(), v1.data_ptr(), v2.data_ptr(),
                                        y_ws.data_ptr(), *args, ws.data_ptr(), nbytes, st))
    print("sdpa_dual_v_noalloc, same inputs", flush=True)
    _native.check(lib.motif_sdpa_dual_v_noalloc(q.data_ptr(), k.data_ptr(), v1.data_ptr(),
                                                v2.data_ptr(), y_na.data_ptr(), *args, st))
    torch.cuda.synchronize()
    assert torch.isfinite(y_ws.float()).all()
    return y_ws, y_na


def _bits(t):
    import torch

    return t.view(torch.int16)


@pytest.mark.parametrize("fused", [0, 1])
def test_noalloc_matches_workspace_entry_twice(gpu, fused):
    import torch

    from mlx_motif import _native

    _native.set_tuning("fused_merge", fused)
    try:
        # the 16k decode workload, then a smaller call reusing the scratch
        for B, Hq, Hkv, cap, kv_len, seed in ((1, 32, 8, 16128, 16000, 1),
                                              (1, 16, 4, 3328, 3204, 2)):
            y_ws, y_na = _call_both(gpu, torch.float16, B, Hq, Hkv, cap, kv_len, seed)
            assert torch.equal(_bits(y_ws), _bits(y_na)), (fused, kv_len)
    finally:
        _native.set_tuning("fused_merge", 0)


def test_noalloc_bf16_and_small_shapes(gpu):
    import torch

    for B, Hq, Hkv, cap, kv_len, seed in ((2, 8, 2, 1024, 1000, 3), (1, 4, 4, 64, 1, 4),
                                          (3, 32, 8, 4096, 4096, 5)):
        y_ws, y_na = _call_both(gpu, torch.bfloat16, B, Hq, Hkv, cap, kv_len, seed)
        assert torch.equal(_bits(y_ws), _bits(y_na)), (B, Hq, kv_len)


def test_noalloc_counters_survive_a_small_call(gpu):
    """In-kernel merge (its arrival counters live in the scratch): a call with
    few rows, then a split call with more than 64 (b, KV head) units.  The
    first call's partials must not land on the counters the second one uses,
    or the second call's last workgroups never see their final ticket and
    leave rows unwritten."""
    import torch

    from mlx_motif import _native

    _native.set_tuning("fused_merge", 1)
    try:
        for B, Hq, Hkv, cap, kv_len, seed in ((1, 32, 8, 16128, 16000, 6),
                                              (4, 32, 32, 3072, 3000, 7),
                                              (1, 32, 8, 16128, 16000, 8)):
            y_ws, y_na = _call_both(gpu, torch.float16, B, Hq, Hkv, cap, kv_len, seed)
            assert torch.equal(_bits(y_ws), _bits(y_na)), (B, Hq, Hkv, kv_len)
    finally:
        _native.set_tuning("fused_merge", 0)
