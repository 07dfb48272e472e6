"""HIP graph capture of the native calls, as a decode loop would capture a
layer: every replay must equal the eager call bit for bit, with eager work
and synchronisations between the replays.  The decode step with the token's
cache write (``new_kv``) is replayed over a cache whose target row is
overwritten before each replay, so each replay is seen writing the row
itself.  No entry point records a memset; the workspace is zeroed by a fill
kernel when first allocated.
"""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def _gen(gpu, seed):
    import torch

    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return lambda *s: torch.randn(*s, generator=g, device=gpu).half()  # noqa: E731


def _capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    torch.cuda.synchronize()
    return graph, out


def _replay_and_check(gpu, graph, before, check, n=4):
    import torch

    for i in range(n):
        before()
        noise = torch.randn(1 << 20, device=gpu)  # eager work between replays
        float(noise.sum())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(i)


def _same(a, b):
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("kv_len,cap", [(16000, 16128), (3204, 3328)])
def test_graph_sdpa_dual_v_f16(gpu, kv_len, cap):
    from mlx_motif.kernels import sdpa_dual_v

    mk = _gen(gpu, kv_len)
    q, k, v1, v2 = mk(1, 32, 1, 128), mk(1, 8, cap, 128), mk(1, 8, cap, 128), mk(1, 8, cap, 128)
    print(f"graph sdpa_dual_v f16 kv_len={kv_len}", flush=True)
    ref = sdpa_dual_v(q, k, v1, v2, 0.0884, kv_len=kv_len).clone()
    graph, out = _capture(lambda: sdpa_dual_v(q, k, v1, v2, 0.0884, kv_len=kv_len))

    def before():
        out.fill_(0)

    def check(i):
        assert _same(out, ref), f"replay {i}"

    _replay_and_check(gpu, graph, before, check)


@pytest.mark.parametrize("bits", [4, 8])
def test_graph_sdpa_dual_v_q(gpu, bits):
    from mlx_motif.kernels import quantize, sdpa_dual_v_q4

    mk = _gen(gpu, 100 + bits)
    q = mk(1, 32, 1, 128)
    trips = [quantize(mk(1, 8, 16128, 128), 64, bits) for _ in range(3)]
    print(f"graph sdpa_dual_v_q4 bits={bits}", flush=True)
    ref = sdpa_dual_v_q4(q, *trips, 0.0884, 64, bits, kv_len=16000).clone()
    graph, out = _capture(lambda: sdpa_dual_v_q4(q, *trips, 0.0884, 64, bits, kv_len=16000))

    def before():
        out.fill_(0)

    def check(i):
        assert _same(out, ref), f"replay {i}"

    _replay_and_check(gpu, graph, before, check)


@pytest.mark.parametrize("bits", [None, 4, 8])
def test_graph_decode_step_with_token_write(gpu, bits):
    """The fused step with new_kv: each replay rewrites row kv_len - 1 (set to
    stale values before it) and returns the eager result."""
    import torch

    from mlx_motif.kernels import gda_decode_attention, gda_decode_attention_q4, quantize

    mk = _gen(gpu, 7 if bits is None else bits)
    kv_len, cap, gr = 3204, 3328, 4
    q1, q2 = mk(1, 32, 1, 128), mk(1, 8, 1, 128)
    rows = [mk(1, 8, 1, 128) for _ in range(4)]
    w = mk(256)
    lam = torch.tensor([0.4321], dtype=torch.float32, device=gpu)
    raw = [mk(1, 8, cap, 128) for _ in range(4)]
    print(f"graph gda_decode append bits={bits}", flush=True)
    if bits is None:
        cache = raw

        def step():
            return gda_decode_attention(q1, q2, *cache, 0.0884, w, lam, 0.2, gr, 1e-5,
                                        kv_len=kv_len, new_kv=rows)

        def stale():
            for c in cache:
                c[:, :, kv_len - 1] = 1e4

        tensors = cache
    else:
        cache = [quantize(t, 64, bits) for t in raw]

        def step():
            return gda_decode_attention_q4(q1, q2, *cache, 0.0884, w, lam, 0.2, gr, 64, bits,
                                           1e-5, kv_len=kv_len, new_kv=rows)

        def stale():
            for t in cache:
                t[0].view(torch.int32)[:, :, kv_len - 1] = 0
                t[1][:, :, kv_len - 1] = 7.0
                t[2][:, :, kv_len - 1] = -3.0

        tensors = [x for t in cache for x in t]
    stale()
    ref = step().clone()
    written = [t.clone() for t in tensors]
    graph, out = _capture(step)

    def before():
        stale()
        out.fill_(0)

    def check(i):
        assert _same(out, ref), f"replay {i}: output"
        for t, e in zip(tensors, written):
            if t.dtype == torch.uint32:
                assert torch.equal(t.view(torch.int32), e.view(torch.int32)), f"replay {i}"
            else:
                assert _same(t, e), f"replay {i}: cache"

    _replay_and_check(gpu, graph, before, check)


def test_graph_epilogues(gpu):
    import torch

    from mlx_motif.kernels import gda_post_split, polynorm

    mk = _gen(gpu, 11)
    o, n, w = mk(1, 16, 512, 128), mk(1, 16, 512, 128), mk(128)
    lam = torch.tensor([0.37], dtype=torch.float32, device=gpu)
    x, pw, pb = mk(700, 4096), mk(3), mk(1)
    print("graph gda_post_split + polynorm", flush=True)
    ref_g = gda_post_split(o, n, w, lam, 0.2, 1, 1e-6).clone()
    ref_p = polynorm(x, pw, pb, 1e-6).clone()
    graph, (yg, yp) = _capture(lambda: (gda_post_split(o, n, w, lam, 0.2, 1, 1e-6),
                                        polynorm(x, pw, pb, 1e-6)))

    def before():
        yg.fill_(0)
        yp.fill_(0)

    def check(i):
        assert torch.equal(yg.float(), ref_g.float()), f"replay {i}: gda_post_split"
        assert _same(yp, ref_p), f"replay {i}: polynorm"

    _replay_and_check(gpu, graph, before, check)


def test_graph_survives_workspace_growth(gpu):
    """A decode step captured on a stream, then a larger call on the same
    stream grows that stream's workspace.  The superseded buffer must stay
    allocated: tensors made afterwards on the stream (filled with a marker)
    must not receive the graph's partials, and every replay still equals
    the eager step."""
    import torch

    from mlx_motif import _native
    from mlx_motif.kernels import gda_decode_attention, sdpa_dual_v

    mk = _gen(gpu, 21)
    kv_len, cap, gr = 16000, 16128, 4
    q1, q2 = mk(1, 32, 1, 128), mk(1, 8, 1, 128)
    cache = [mk(1, 8, cap, 128) for _ in range(4)]
    w = mk(256)
    lam = torch.tensor([0.4321], dtype=torch.float32, device=gpu)

    def step():
        return gda_decode_attention(q1, q2, *cache, 0.0884, w, lam, 0.2, gr, 1e-5,
                                    kv_len=kv_len)

    print("graph gda_decode, then workspace growth on the capture stream", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ref = step().clone()
        old = _native.workspace(gpu, 0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = step()
    torch.cuda.synchronize()
    n_retired = len(_native._retired)
    _native.set_tuning("rows_per_split", 16)  # ~1000 splits: a workspace far past the old one
    try:
        with torch.cuda.stream(s):
            sdpa_dual_v(q1, cache[0], cache[2], cache[3], 0.0884, kv_len=kv_len)
            grown = _native.workspace(gpu, 0)
    finally:
        _native.set_tuning("rows_per_split", 0)
    torch.cuda.synchronize()
    assert grown.numel() >= 2 * old.numel() and len(_native._retired) == n_retired + 1
    old_ptr, old_bytes = old.data_ptr(), old.numel()
    del old
    with torch.cuda.stream(s):
        marks = [torch.full((old_bytes,), 0x5A, dtype=torch.uint8, device=gpu) for _ in range(4)]
    torch.cuda.synchronize()
    assert all(m.data_ptr() != old_ptr for m in marks)

    def before():
        out.fill_(0)

    def check(i):
        assert _same(out, ref), f"replay {i}"
        for m in marks:
            assert bool((m == 0x5A).all()), f"replay {i} wrote into memory of a later tensor"

    with torch.cuda.stream(s):
        _replay_and_check(gpu, graph, before, check)
    del graph, out
    torch.cuda.synchronize()
    assert _native.release_retired_workspaces() >= old_bytes
