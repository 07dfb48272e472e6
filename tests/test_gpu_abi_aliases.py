"""The reference-named aliases (motif_sdpa_dual_v_q4, motif_sdpa_dual_v_verify,
motif_sdpa_dual_v_q4_verify) return exactly what the entry points they
forward to return, through the C ABI."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def _setup(gpu, S_q, kv_len, cap, bits):
    import torch

    from mlx_motif import _native
    from mlx_motif.kernels import quantize

    g = torch.Generator(device=gpu)
    g.manual_seed(31 + S_q + bits)
    mk = lambda *s: torch.randn(*s, generator=g, device=gpu).half()  # noqa: E731
    q = mk(1, 32, S_q, 128)
    raw = [mk(1, 8, cap, 128) for _ in range(3)]
    trips = [quantize(t, 64, bits) for t in raw]
    lib = _native.lib()
    ws = _native.workspace(gpu, lib.motif_sdpa_workspace_bytes(1, 32, 8, S_q, kv_len, 128))
    return torch, _native, lib, q, raw, trips, ws


@pytest.mark.parametrize("bits", [4, 8])
def test_q4_alias_equals_q_entry(gpu, bits):
    torch, _native, lib, q, _, trips, ws = _setup(gpu, 1, 3000, 3072, bits)
    ptrs = [x.data_ptr() for t in trips for x in t]
    ys = []
    for fn in (lib.motif_sdpa_dual_v_q, lib.motif_sdpa_dual_v_q4):
        y = torch.empty((1, 32, 1, 256), dtype=torch.float16, device=gpu)
        _native.check(fn(q.data_ptr(), *ptrs, y.data_ptr(), 0, 1, 32, 8, 128, 3072, 3000, bits,
                         64, 0.0884, ws.data_ptr(), ws.numel(), _native.stream_of(gpu)))
        ys.append(y)
    torch.cuda.synchronize()
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))


def test_verify_aliases_equal_rows_entries(gpu):
    torch, _native, lib, q, raw, trips, ws = _setup(gpu, 5, 3000, 3072, 8)
    st = _native.stream_of(gpu)
    fp = [t.data_ptr() for t in raw]
    packed = [x.data_ptr() for t in trips for x in t]
    out = {}
    for name, fn, args in (
        ("rows", lib.motif_sdpa_dual_v_rows, fp),
        ("verify", lib.motif_sdpa_dual_v_verify, fp),
    ):
        y = torch.empty((1, 32, 5, 256), dtype=torch.float16, device=gpu)
        _native.check(fn(q.data_ptr(), *args, y.data_ptr(), 0, 1, 32, 8, 5, 128, 3072, 3000, 1,
                         0.0884, ws.data_ptr(), ws.numel(), st))
        out[name] = y
    for name, fn in (("q_rows", lib.motif_sdpa_dual_v_q_rows),
                     ("q4_verify", lib.motif_sdpa_dual_v_q4_verify)):
        y = torch.empty((1, 32, 5, 256), dtype=torch.float16, device=gpu)
        _native.check(fn(q.data_ptr(), *packed, y.data_ptr(), 0, 1, 32, 8, 5, 128, 3072, 3000, 1,
                         8, 64, 0.0884, ws.data_ptr(), ws.numel(), st))
        out[name] = y
    torch.cuda.synchronize()
    assert torch.equal(out["rows"].view(torch.int16), out["verify"].view(torch.int16))
    assert torch.equal(out["q_rows"].view(torch.int16), out["q4_verify"].view(torch.int16))
