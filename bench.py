#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Metric: decode-attn µs/call and achieved HBM GB/s (% of peak) at KV = 16k for
the fp16 4-slot cache (the headline ``value``) and the packed q4 / q8 caches.

Workload (one "step" = one call of the hot path over one layer's cache):
  shared-QK dual-V decode, batch 1, 32 query heads over 8 KV heads,
  head_dim 128, kv_len 16000 live rows of a 16128-row cache, scale 1/sqrt(128),
  synthetic N(0,1) fp16 from a fixed seed; q4/q8 caches quantised MLX-affine
  with group size 64.
Each call reads a different layer's buffers (fp16: 8 sets = 0.79 GB, q4: 24
sets = 0.67 GB, q8: 16 sets = 0.84 GB), so the 256 MB Infinity Cache cannot
serve them.  The K timed calls are replayed from one HIP graph (captured after
W eager warm-up calls), bracketed by HIP events on the launch stream; the
graph is replayed 21 times and the median replay is reported.

Algorithmic bytes per call count each live K/V1/V2 row once (plus scales and
biases for packed caches) and q and y:
  fp16 98,328,576 B, q4 27,672,576 B, q8 52,248,576 B.

cpu_baseline: the oracle's C/OpenMP port (oracle/motif_oracle.c) on the host
cores, one full fp16 call (32 heads x 16000 rows), median of 21 runs after 3
warm-ups.  It is a reported baseline, not the target.

stdout carries exactly one JSON line.  --extra adds µs/call lines for the
other workloads of the path on stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import csv
import hashlib
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "mlx-motif_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_HBM_GBPS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 matrix-core peak
METRIC = "decode-attn µs/call + achieved HBM GB/s (% peak) at KV=16k, fp16 & q4 cache"

B, HQ, HKV, D = 1, 32, 8, 128
KV_LEN, CAP = 16000, 16128
GS = 64


def alg_bytes(kind: str, kv_len: int = KV_LEN, hq: int = HQ, hkv: int = HKV, s_q: int = 1) -> int:
    qy = hq * s_q * D * 2 + hq * s_q * 2 * D * 2
    if kind == "f16":
        return 3 * B * hkv * kv_len * D * 2 + qy
    bits = 4 if kind == "q4" else 8
    return 3 * B * hkv * kv_len * (D * bits // 8 + 2 * (D // GS) * 2) + qy


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


REPEATS = 21  # timed replays per workload (at least 20); the median is reported


def time_calls_stats(torch, calls, steps: int, warmup: int, use_graph: bool = True,
                     repeats: int = REPEATS):
    """µs per call over `steps` calls cycling through `calls`: the graph of
    the `steps` calls (or the eager sequence) is timed `repeats` times, each
    between two HIP events on the launch stream.  Returns (median, min, max)
    over the repeats."""
    for i in range(warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    g = None
    if use_graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                calls[i % len(calls)]()
        g.replay()  # warm replay
        torch.cuda.synchronize()
    per_call = []
    for _ in range(repeats):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        if g is not None:
            g.replay()
        else:
            for i in range(steps):
                calls[i % len(calls)]()
        end.record(stream)
        torch.cuda.synchronize()
        per_call.append(start.elapsed_time(end) * 1000.0 / steps)
    return statistics.median(per_call), min(per_call), max(per_call)


def time_calls(torch, calls, steps: int, warmup: int, use_graph: bool = True,
               repeats: int = REPEATS):
    """Median µs per call (see time_calls_stats)."""
    return time_calls_stats(torch, calls, steps, warmup, use_graph, repeats)[0]


def make_fp16_calls(torch, lib, dev, nsets, kv_len=KV_LEN, cap=CAP, hq=HQ, hkv=HKV, s_q=1,
                    bf16=False):
    """fp16-cache calls (``bf16``: the same over a bf16 cache)."""
    from mlx_motif import _native

    dt, code = (torch.bfloat16, 1) if bf16 else (torch.float16, 0)
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    q = torch.randn((B, hq, s_q, D), generator=g, device=dev).to(dt)
    sets = []
    for _ in range(nsets):
        k, v1, v2 = (torch.randn((B, hkv, cap, D), generator=g, device=dev).to(dt)
                     for _ in range(3))
        sets.append((k, v1, v2, torch.empty((B, hq, s_q, 2 * D), dtype=dt, device=dev)))
    nbytes = lib.motif_sdpa_workspace_bytes(B, hq, hkv, s_q, kv_len, D)
    ws = torch.zeros(max(nbytes, 16 << 20), dtype=torch.uint8, device=dev)
    scale = 1.0 / D ** 0.5

    def mk(k, v1, v2, y):
        def call():
            stream = torch.cuda.current_stream().cuda_stream
            if s_q == 1:
                st = lib.motif_sdpa_dual_v(q.data_ptr(), k.data_ptr(), v1.data_ptr(),
                                           v2.data_ptr(), y.data_ptr(), code, B, hq, hkv, D, cap,
                                           kv_len, scale, ws.data_ptr(), ws.numel(), stream)
            else:
                st = lib.motif_sdpa_dual_v_rows(q.data_ptr(), k.data_ptr(), v1.data_ptr(),
                                                v2.data_ptr(), y.data_ptr(), code, B, hq, hkv, s_q,
                                                D, cap, kv_len, 1, scale, ws.data_ptr(),
                                                ws.numel(), stream)
            _native.check(st)
        return call

    return [mk(*s) for s in sets], (q, sets)


def make_decode_calls(torch, lib, dev, nsets, kv_len=KV_LEN, cap=CAP, fused=True, gr=4,
                      bits=None, append=None, bf16=False):
    """One GDA decode-attention step per call over distinct layer caches
    (k1, k2, v1, v2 of HKV heads): motif_gda_decode / motif_gda_decode_q
    (fused) or the reference's three calls (two motif_sdpa_dual_v(_q) +
    motif_gda_post_split).  ``bits`` 4/8: packed cache, group size 64.
    ``append``: also write the token's four rows at row kv_len - 1, inside
    the step ("fused": motif_gda_decode(_q)_append) or before it ("write":
    the cache write -- four row copies, or motif_quant_write4 -- then the
    fused step).  ``bf16``: bf16 activations, cache (or scales and biases)
    and output."""
    from mlx_motif import _native
    from mlx_motif.kernels import quantize

    dt, code = (torch.bfloat16, 1) if bf16 else (torch.float16, 0)
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    q1 = torch.randn((B, HKV * gr, 1, D), generator=g, device=dev).to(dt)
    q2 = torch.randn((B, HKV, 1, D), generator=g, device=dev).to(dt)
    w = torch.rand(2 * D, generator=g, device=dev).to(dt)
    lam = torch.tensor([0.37], dtype=torch.float32, device=dev)
    sets = [tuple(torch.randn((B, HKV, cap, D), generator=g, device=dev).to(dt)
                  for _ in range(4)) for _ in range(nsets)]
    if bits:
        sets = [tuple(quantize(t, GS, bits) for t in st) for st in sets]
        torch.cuda.synchronize()
    rows = [torch.randn((B, HKV, 1, D), generator=g, device=dev).to(dt) for _ in range(4)]
    rp = [r.data_ptr() for r in rows]
    y = torch.empty((B, HKV * gr, 1, 2 * D), dtype=dt, device=dev)
    o = torch.empty((B, HKV * gr, 1, 2 * D), dtype=dt, device=dev)
    n = torch.empty((B, HKV, 1, 2 * D), dtype=dt, device=dev)
    nbytes = max(lib.motif_gda_decode_workspace_bytes(B, HKV, gr, kv_len, D),
                 lib.motif_sdpa_workspace_bytes(B, HKV * gr, HKV, 1, kv_len, D))
    ws = torch.zeros(max(nbytes, 16 << 20), dtype=torch.uint8, device=dev)
    scale = 1.0 / D ** 0.5

    def mk_q(k1, k2, v1, v2):
        p = lambda t: [x.data_ptr() for x in t]  # noqa: E731

        slots = (k1, k2, v1, v2)
        data = (ctypes.c_void_p * 4)(*(t[0].data_ptr() for t in slots))
        scl = (ctypes.c_void_p * 4)(*(t[1].data_ptr() for t in slots))
        bia = (ctypes.c_void_p * 4)(*(t[2].data_ptr() for t in slots))

        def call():
            st = torch.cuda.current_stream().cuda_stream
            tail = (w.data_ptr(), lam.data_ptr(), 0.8, 1e-5, y.data_ptr(), code, B, HKV, gr, D,
                    cap, kv_len, bits, GS, scale, ws.data_ptr(), ws.numel(), st)
            if append == "fused":
                _native.check(lib.motif_gda_decode_q_append(
                    q1.data_ptr(), q2.data_ptr(), *rp, *p(k1), *p(k2), *p(v1), *p(v2), *tail))
                return
            if append == "write":
                _native.check(lib.motif_quant_write4(*rp, data, scl, bia, code, B, HKV, 1, D, cap,
                                                     kv_len - 1, bits, GS, st))
            if fused:
                _native.check(lib.motif_gda_decode_q(
                    q1.data_ptr(), q2.data_ptr(), *p(k1), *p(k2), *p(v1), *p(v2), *tail))
                return
            _native.check(lib.motif_sdpa_dual_v_q(
                q1.data_ptr(), *p(k1), *p(v1), *p(v2), o.data_ptr(), code, B, HKV * gr, HKV, D,
                cap, kv_len, bits, GS, scale, ws.data_ptr(), ws.numel(), st))
            _native.check(lib.motif_sdpa_dual_v_q(
                q2.data_ptr(), *p(k2), *p(v1), *p(v2), n.data_ptr(), code, B, HKV, HKV, D,
                cap, kv_len, bits, GS, scale, ws.data_ptr(), ws.numel(), st))
            _native.check(lib.motif_gda_post_split(
                o.data_ptr(), n.data_ptr(), w.data_ptr(), y.data_ptr(), code, B, HKV * gr, HKV, gr,
                1, 2 * D, lam.data_ptr(), 0.8, 1e-5, st))
        return call

    def mk(k1, k2, v1, v2):
        def call():
            st = torch.cuda.current_stream().cuda_stream
            if append == "fused":
                _native.check(lib.motif_gda_decode_append(
                    q1.data_ptr(), q2.data_ptr(), *rp, k1.data_ptr(), k2.data_ptr(),
                    v1.data_ptr(), v2.data_ptr(), w.data_ptr(), lam.data_ptr(), 0.8, 1e-5,
                    y.data_ptr(), code, B, HKV, gr, D, cap, kv_len, scale, ws.data_ptr(),
                    ws.numel(), st))
                return
            if append == "write":  # the fp cache's write: a slice copy per slot
                for c, r in zip((k1, k2, v1, v2), rows):
                    c[:, :, kv_len - 1:kv_len].copy_(r)
            if fused:
                _native.check(lib.motif_gda_decode(
                    q1.data_ptr(), q2.data_ptr(), k1.data_ptr(), k2.data_ptr(), v1.data_ptr(),
                    v2.data_ptr(), w.data_ptr(), lam.data_ptr(), 0.8, 1e-5, y.data_ptr(), code, B,
                    HKV, gr, D, cap, kv_len, scale, ws.data_ptr(), ws.numel(), st))
                return
            _native.check(lib.motif_sdpa_dual_v(
                q1.data_ptr(), k1.data_ptr(), v1.data_ptr(), v2.data_ptr(), o.data_ptr(), code, B,
                HKV * gr, HKV, D, cap, kv_len, scale, ws.data_ptr(), ws.numel(), st))
            _native.check(lib.motif_sdpa_dual_v(
                q2.data_ptr(), k2.data_ptr(), v1.data_ptr(), v2.data_ptr(), n.data_ptr(), code, B,
                HKV, HKV, D, cap, kv_len, scale, ws.data_ptr(), ws.numel(), st))
            _native.check(lib.motif_gda_post_split(
                o.data_ptr(), n.data_ptr(), w.data_ptr(), y.data_ptr(), code, B, HKV * gr, HKV, gr,
                1, 2 * D, lam.data_ptr(), 0.8, 1e-5, st))
        return call

    return [(mk_q if bits else mk)(*t) for t in sets], (q1, q2, w, lam, sets, y, o, n, ws)


def make_small_step_calls(torch, lib, dev, nsets, kv_len=1024, fused=True):
    """The small GDA decode step: q1, q2 (1, 8, 1, D) over k1/k2/v1/v2 (1, 4,
    kv_len, D) fp16 into y (1, 8, 1, 2D): one motif_gda_decode_heads call
    (attention launch + merge with the epilogue), or (fused=False) the
    reference's three calls, two motif_sdpa_dual_v (GQA 2) then
    motif_gda_post_split with gr 1."""
    from mlx_motif import _native

    g = torch.Generator(device=dev)
    g.manual_seed(11)
    q1, q2 = (torch.randn((1, 8, 1, D), generator=g, device=dev).half() for _ in range(2))
    w = torch.rand(2 * D, generator=g, device=dev).half()
    lam = torch.tensor([0.37], dtype=torch.float32, device=dev)
    sets = [tuple(torch.randn((1, 4, kv_len, D), generator=g, device=dev).half()
                  for _ in range(4)) for _ in range(nsets)]
    o, n, y = (torch.empty((1, 8, 1, 2 * D), dtype=torch.float16, device=dev) for _ in range(3))
    nbytes = max(lib.motif_sdpa_workspace_bytes(1, 8, 4, 1, kv_len, D),
                 lib.motif_gda_decode_heads_workspace_bytes(1, 8, 8, 4, kv_len, D))
    ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
    scale = 1.0 / D ** 0.5

    def mk(k1, k2, v1, v2):
        def call():
            st = torch.cuda.current_stream().cuda_stream
            if fused:
                _native.check(lib.motif_gda_decode_heads(
                    q1.data_ptr(), q2.data_ptr(), None, None, None, None, k1.data_ptr(),
                    k2.data_ptr(), v1.data_ptr(), v2.data_ptr(), w.data_ptr(), lam.data_ptr(),
                    0.8, 1e-5, y.data_ptr(), 0, 1, 8, 8, 4, D, kv_len, kv_len, scale,
                    ws.data_ptr(), ws.numel(), st))
                return
            for q, k, out in ((q1, k1, o), (q2, k2, n)):
                _native.check(lib.motif_sdpa_dual_v(
                    q.data_ptr(), k.data_ptr(), v1.data_ptr(), v2.data_ptr(), out.data_ptr(), 0,
                    1, 8, 4, D, kv_len, kv_len, scale, ws.data_ptr(), ws.numel(), st))
            _native.check(lib.motif_gda_post_split(
                o.data_ptr(), n.data_ptr(), w.data_ptr(), y.data_ptr(), 0, 1, 8, 8, 1, 1, 2 * D,
                lam.data_ptr(), 0.8, 1e-5, st))
        return call

    return [mk(*t) for t in sets], (q1, q2, w, lam, sets, o, n, y, ws)


def decode_bytes(kv_len: int, fused: bool, gr: int = 4, bits=None) -> int:
    """Cache bytes of one decode step: 4 streams fused, 6 for the three calls
    (v1 and v2 read by both passes), plus q and y.  A packed row holds
    D*bits/8 code bytes and 2*D/64 fp16 scales and biases."""
    streams = 4 if fused else 6
    heads = HKV * gr + HKV
    row = D * 2 if not bits else D * bits // 8 + 2 * (D // GS) * 2
    return streams * B * HKV * kv_len * row + heads * D * 2 + HKV * gr * 2 * D * 2


def make_q_calls(torch, lib, dev, nsets, bits, kv_len=KV_LEN, cap=CAP, hq=HQ, hkv=HKV, s_q=1,
                 bf16=False):
    """Packed-cache calls (``bf16``: bf16 activations, scales and biases)."""
    from mlx_motif import _native
    from mlx_motif.kernels import quantize

    dt, code = (torch.bfloat16, 1) if bf16 else (torch.float16, 0)
    g = torch.Generator(device=dev)
    g.manual_seed(4321 + bits)
    q = torch.randn((B, hq, s_q, D), generator=g, device=dev).to(dt)
    sets = []
    for _ in range(nsets):
        trips = []
        for _ in range(3):
            x = torch.randn((B, hkv, cap, D), generator=g, device=dev).to(dt)
            trips.append(quantize(x, group_size=GS, bits=bits))
            del x
        sets.append((trips, torch.empty((B, hq, s_q, 2 * D), dtype=dt, device=dev)))
    nbytes = lib.motif_sdpa_workspace_bytes(B, hq, hkv, s_q, kv_len, D)
    ws = torch.zeros(max(nbytes, 16 << 20), dtype=torch.uint8, device=dev)
    scale = 1.0 / D ** 0.5

    def mk(trips, y):
        ptrs = [t.data_ptr() for trip in trips for t in trip]

        def call():
            stream = torch.cuda.current_stream().cuda_stream
            if s_q == 1:
                st = lib.motif_sdpa_dual_v_q(q.data_ptr(), *ptrs, y.data_ptr(), code, B, hq, hkv,
                                             D, cap, kv_len, bits, GS, scale, ws.data_ptr(),
                                             ws.numel(), stream)
            else:
                st = lib.motif_sdpa_dual_v_q_rows(q.data_ptr(), *ptrs, y.data_ptr(), code, B, hq,
                                                  hkv, s_q, D, cap, kv_len, 1, bits, GS, scale,
                                                  ws.data_ptr(), ws.numel(), stream)
            _native.check(st)
        return call

    return [mk(*s) for s in sets], (q, sets)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


CPU_REPEATS = 21  # timed runs of each CPU-baseline leg (at least 20)


def cpu_baseline():
    """The oracle's C/OpenMP port timed on the host: one full fp16 call and
    one full q4 call, on every OpenMP thread and on one thread."""
    import numpy as np

    from oracle import c_oracle

    rng = np.random.default_rng(99)
    q = rng.standard_normal((B, HQ, 1, D)).astype(np.float16)
    k, v1, v2 = (rng.standard_normal((B, HKV, CAP, D)).astype(np.float16) for _ in range(3))
    trips = [c_oracle.quantize_f16(t, GS, 4) for t in (k, v1, v2)]
    threads = c_oracle.max_threads()
    scale = 1 / np.sqrt(D)

    def median_us(fn, reps=CPU_REPEATS, warm=3):
        times = []
        for i in range(reps + warm):
            t0 = time.perf_counter()
            fn()
            t1 = time.perf_counter()
            if i >= warm:
                times.append((t1 - t0) * 1e6)
        return statistics.median(times)

    def f16(n, fast=False):
        return c_oracle.sdpa_dual_v_f16(q, k, v1, v2, scale, KV_LEN, nthreads=n, fast=fast)

    def q4(n, fast=False):
        return c_oracle.sdpa_dual_v_q_f16(q, *trips, scale, GS, 4, KV_LEN, nthreads=n, fast=fast)

    us = median_us(lambda: f16(threads))
    us_q4 = median_us(lambda: q4(threads))
    us_1 = median_us(lambda: f16(1))
    us_q4_1 = median_us(lambda: q4(1))
    fus = median_us(lambda: f16(threads, True))
    fus_q4 = median_us(lambda: q4(threads, True))
    fus_1 = median_us(lambda: f16(1, True))
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {
        "value": round(us, 1),
        "unit": "us/call",
        "cores": threads,
        "kind": "port",
        "sample": "one full sdpa_dual_v call (32 heads x 16000 rows, D 128) of the C/OpenMP "
                  "port oracle/motif_oracle.c, fp16 cache (value) and q4 cache, on `cores` "
                  f"OpenMP threads and on one thread (each the median of {CPU_REPEATS} runs "
                  "after 3 warm-ups); value: gcc -O2 -mf16c -ffp-contract=off (scalar, the "
                  "checker's build); "
                  "`vectorised`: the same source built gcc -O3 -march=x86-64-v3 -ffast-math",
        "gbps": round(alg_bytes("f16") / us / 1e3, 2),
        "one_thread_us": round(us_1, 1),
        "q4_us": round(us_q4, 1),
        "q4_gbps": round(alg_bytes("q4") / us_q4 / 1e3, 2),
        "q4_one_thread_us": round(us_q4_1, 1),
        "vectorised": {"us": round(fus, 1), "gbps": round(alg_bytes("f16") / fus / 1e3, 2),
                       "one_thread_us": round(fus_1, 1), "q4_us": round(fus_q4, 1),
                       "q4_gbps": round(alg_bytes("q4") / fus_q4 / 1e3, 2),
                       "flags": "gcc -O3 -fopenmp -march=x86-64-v3 -ffast-math"},
        "cpu_model": _cpu_model(),
        "nproc": os.cpu_count(),
        "affinity_cpus": affinity,
    }


# Files whose content decides the kernels' code: a traffic profile records
# their digest, and the JSON line says whether the tree it runs from matches.
SOURCE_GLOBS = ("mlx-motif_amd/csrc/*.hip", "mlx-motif_amd/csrc/*.hpp",
                "mlx-motif_amd/csrc/Makefile", "include/motif_hip.h")


def sources_digest() -> str:
    h = hashlib.sha256()
    for p in sorted({f for g in SOURCE_GLOBS for f in ROOT.glob(g)}):
        h.update(p.relative_to(ROOT).as_posix().encode() + b"\0" + p.read_bytes())
    return h.hexdigest()[:16]


def load_traffic(kind: str):
    """HBM bytes per call from profiles/traffic_sdpa_dual_v_<kind>_kv16000.json
    (two rocprofv3 --pmc passes, summarised by --summarize-traffic), with the
    commit and source digest it was measured at."""
    p = ROOT / "profiles" / f"traffic_sdpa_dual_v_{kind}_kv16000.json"
    try:
        prof = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    return {"bytes": prof.get("hbm_bytes_per_launch"), "file": p.relative_to(ROOT).as_posix(),
            "commit": prof.get("commit"),
            "matches_sources": prof.get("sources_digest") == sources_digest()}


def roofline(kind: str, r: dict, basis: str) -> dict:
    prof = load_traffic(kind)
    return {
        "bound": "hbm",
        "achieved": r["gbps"],
        "peak": PEAK_HBM_GBPS,
        "unit": "GB/s",
        "frac": round(r["gbps"] / PEAK_HBM_GBPS, 4),
        "traffic": prof["bytes"] if prof else None,
        "traffic_profile": None if prof is None else {
            "file": prof["file"], "commit": prof["commit"],
            "matches_sources": prof["matches_sources"]},
        "basis": basis,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other rows' shapes (decode step, verify slabs, prefill chunks)")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches")
    ap.add_argument("--extra", action="store_true", help="also time the other workloads")
    ap.add_argument("--valu", action="store_true",
                    help="route attention through the VALU kernels (matrix cores off), "
                         "for comparison")
    ap.add_argument("--traffic", nargs="?", const="f16",
                    choices=("f16", "q4", "q8", "prefill", "slab_q4", "slab_q8"),
                    help="counter pass: one 256 MiB copy, then 16 eager decode calls on the "
                         "given cache (default f16), or 6 prefill-chunk calls (512 rows over "
                         "3716, fp16), or 6 verify-slab calls (5 rows over 32768, q4 / q8); "
                         "no timing, no JSON; run under rocprofv3 --pmc")
    ap.add_argument("--summarize-traffic", nargs=3, metavar=("KIND", "FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic_sdpa_dual_v_<KIND>_kv16000.json from the CSV "
                         "directories of the FETCH_SIZE and WRITE_SIZE passes (no GPU)")
    args = ap.parse_args()
    if args.summarize_traffic:
        return summarize_traffic(*args.summarize_traffic)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        return 2

    import torch

    from mlx_motif import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    if args.traffic:
        return traffic_pass(torch, lib, dev, args.traffic)
    if args.valu:
        _native.set_tuning("mfma", 0)
    graph = not args.no_graph
    res = {}
    for kind, nsets in (("f16", 8), ("q4", 24), ("q8", 16)):
        if kind == "f16":
            calls, keep = make_fp16_calls(torch, lib, dev, nsets)
        else:
            calls, keep = make_q_calls(torch, lib, dev, nsets, 4 if kind == "q4" else 8)
        us, us_min, us_max = time_calls_stats(torch, calls, args.steps, args.warmup, graph)
        gbps = alg_bytes(kind) / us / 1e3
        res[kind] = {"us_per_call": round(us, 3), "us_min": round(us_min, 3),
                     "us_max": round(us_max, 3), "repeats": REPEATS, "gbps": round(gbps, 1),
                     "pct_peak": round(100 * gbps / PEAK_HBM_GBPS, 1),
                     "alg_bytes": alg_bytes(kind), "buffer_sets": nsets}
        log(f"{kind}: {us:.3f} us/call (median of {REPEATS}; {us_min:.3f}..{us_max:.3f})  "
            f"{gbps:.1f} GB/s  ({100 * gbps / PEAK_HBM_GBPS:.1f}% of {PEAK_HBM_GBPS:.0f})")
        del calls, keep
        torch.cuda.empty_cache()

    if args.extra:
        run_extra(torch, lib, dev, args)
    sec = None if args.no_secondary else secondary(torch, lib, dev)

    f16 = res["f16"]
    basis = ("algorithmic bytes / median us per call; a call is the attention launch plus the "
             "split-merge launch (HIP events around graph-replayed calls, median of "
             f"{REPEATS} replays of --steps calls)")
    out = {
        "metric": METRIC,
        "value": f16["us_per_call"],
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(f16["us_per_call"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) fp16 K/V/q from a fixed seed (random cache, no checkpoint)",
        "config": {
            "workload": "sdpa_dual_v decode on the fp16 4-slot cache: B=1, 32 q-heads over 8 "
                        "KV heads, head_dim 128, kv_len 16000 (cap 16128); q4/q8 at the same "
                        "shape, group_size 64",
            "cache_dtype": "f16", "kv_len": KV_LEN, "kv_cap": CAP, "heads_q": HQ,
            "heads_kv": HKV, "head_dim": D, "accumulate": "f32",
            "timing": "hip graph replay" if graph else "eager",
            "kernels": "valu" if args.valu else "matrix-core where compiled",
        },
        "gbps": f16["gbps"],
        "pct_peak": f16["pct_peak"],
        "q4": dict(res["q4"], roofline=roofline("q4", res["q4"], basis)),
        "q8": dict(res["q8"], roofline=roofline("q8", res["q8"], basis)),
        "roofline": roofline("f16", f16, basis),
        "sources_digest": sources_digest(),
        "secondary": sec,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(),
    }
    print(json.dumps(out), flush=True)
    return 0


def traffic_pass(torch, lib, dev, kind: str = "f16") -> int:
    """Dispatches for the hardware counters: a plain copy of known size
    (256 MiB read + 256 MiB written; calibrates FETCH_SIZE / WRITE_SIZE) and
    16 decode calls over 8 buffer sets of the given cache type."""
    src = torch.empty(128 << 20, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    if kind == "prefill":
        calls, keep = make_fp16_calls(torch, lib, dev, 2, kv_len=3716, cap=3840, s_q=512)
        for i in range(6):
            calls[i % len(calls)]()
        torch.cuda.synchronize()
        log("traffic pass: copy 268435456 B + 6 prefill calls (512 rows over 3716)")
        del calls, keep
        return 0
    if kind.startswith("slab_"):
        bits = 4 if kind == "slab_q4" else 8
        calls, keep = make_q_calls(torch, lib, dev, 2, bits, kv_len=32768, cap=32768, s_q=5)
        for i in range(6):
            calls[i % len(calls)]()
        torch.cuda.synchronize()
        log(f"traffic pass: copy 268435456 B + 6 q{bits} slab calls (5 rows over 32768)")
        del calls, keep
        return 0
    if kind == "f16":
        calls, keep = make_fp16_calls(torch, lib, dev, 8)
    else:
        calls, keep = make_q_calls(torch, lib, dev, 8, 4 if kind == "q4" else 8)
    for i in range(16):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    log(f"traffic pass: copy 268435456 B + 16 {kind} decode calls of {alg_bytes(kind)} B")
    del calls, keep
    return 0


def summarize_traffic(kind: str, fetch_dir: str, write_dir: str) -> int:
    """Writes profiles/traffic_sdpa_dual_v_<kind>_kv16000.json from the CSV
    output of the two counter passes over ``bench.py --traffic <kind>``:
    per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the attention and merge
    kernels, scaled by what the same counters read for the 256 MiB copy."""
    import subprocess
    from collections import defaultdict

    def per_kernel(d: str):
        vals = defaultdict(list)
        files = sorted(pathlib.Path(d).rglob("*counter_collection.csv"))
        if not files:
            raise SystemExit(f"no *counter_collection.csv under {d}")
        for row in csv.DictReader(open(files[0])):
            vals[row["Kernel_Name"]].append(float(row["Counter_Value"]))
        return vals

    F, W = per_kernel(fetch_dir), per_kernel(write_dir)
    copy = next(k for k in F if "copyBuffer" in k)
    ff, wf = 262144.0 / F[copy][0], 262144.0 / W[copy][0]
    att = next(k for k in F if "sdpa_" in k and "merge" not in k)
    mer = next(k for k in F if "sdpa_merge" in k)
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    rd = round((mean(F[att]) + mean(F[mer])) * ff * 1024)
    wr = round((mean(W[att]) + mean(W[mer])) * wf * 1024)
    alg = alg_bytes(kind)
    try:
        commit = subprocess.run(["git", "rev-parse", "--short", "HEAD"], cwd=ROOT,
                                capture_output=True, text=True, check=True).stdout.strip()
        dirty = bool(subprocess.run(["git", "status", "--porcelain", "--"] + list(SOURCE_GLOBS),
                                    cwd=ROOT, capture_output=True, text=True).stdout.strip())
    except (OSError, subprocess.CalledProcessError):
        commit, dirty = "unknown", None
    flag = "" if kind == "f16" else f" {kind}"
    out = {
        "workload": "B=1, 32 q-heads over 8 KV heads, head_dim 128, kv_len 16000, cap 16128"
                    + ("" if kind == "f16" else f"; {kind}, group_size 64"),
        "commit": commit, "sources_dirty": dirty, "sources_digest": sources_digest(),
        "commands": [
            f"timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE --output-format csv -d {fetch_dir} "
            f"-o fetch -- python3 bench.py --traffic{flag}",
            f"timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE --output-format csv -d {write_dir} "
            f"-o write -- python3 bench.py --traffic{flag}",
            f"python3 bench.py --summarize-traffic {kind} {fetch_dir} {write_dir}"],
        "calibration": {"kernel": copy.split("(")[0] + " (torch copy_ of 268435456 B)",
                        "fetch_kib": F[copy][0], "write_kib": W[copy][0],
                        "expected_kib": 262144, "fetch_factor": round(ff, 5),
                        "write_factor": round(wf, 5)},
        "dispatches_per_kernel": len(F[att]),
        "attention_kernel": {"name": att, "fetch_kib": round(mean(F[att]), 1),
                             "write_kib": round(mean(W[att]), 1),
                             "read_bytes": round(mean(F[att]) * ff * 1024),
                             "write_bytes": round(mean(W[att]) * wf * 1024)},
        "merge_kernel": {"name": mer, "fetch_kib": round(mean(F[mer]), 1),
                         "write_kib": round(mean(W[mer]), 1),
                         "read_bytes": round(mean(F[mer]) * ff * 1024),
                         "write_bytes": round(mean(W[mer]) * wf * 1024)},
        "hbm_read_bytes_per_launch": rd, "hbm_write_bytes_per_launch": wr,
        "hbm_bytes_per_launch": rd + wr, "algorithmic_bytes_per_launch": alg,
        "traffic_over_algorithmic": round((rd + wr) / alg, 4),
        "note": "per call (attention + merge kernel). Above the algorithmic bytes: the split "
                "partials (32 virtual heads x 32 splits x 258 floats = 1.06 MB) written by the "
                "attention kernel and read back once by the merge kernel.",
    }
    dst = ROOT / "profiles" / f"traffic_sdpa_dual_v_{kind}_kv16000.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    log(f"{dst.name}: {rd + wr} B per call, {out['traffic_over_algorithmic']}x algorithmic")
    return 0


def secondary(torch, lib, dev, steps: int = 50, warm: int = 5) -> dict:
    """The other rows' headline shapes, timed as the decode calls are (graph
    replay, HIP events): the small GDA step (8 signal/noise pairs over 4 KV
    heads at 1024 rows, fused and as three calls), the fused GDA decode step
    at 16k and, with the
    token's write, at 3204 over 48 layer caches, the 5-row verify
    slabs over 32768 rows (fp16 and q8), the 512-row prefill chunk over 3716
    rows and a 12.7B layer's 512-row chunk at offset 3204 from the
    projections (RoPE + 4-slot write + both passes in one launch)."""
    from mlx_motif.kernels import gda_prefill_attention_from_proj

    from mlx_motif.kernels import gda_post_split, polynorm

    out = {}

    def hbm(name, st, nbytes):
        us = st[0]
        gbps = nbytes / us / 1e3
        out[name] = {"us_per_call": round(us, 3), "us_min": round(st[1], 3),
                     "us_max": round(st[2], 3), "gbps": round(gbps, 1),
                     "pct_peak_hbm": round(100 * gbps / PEAK_HBM_GBPS, 1)}

    def mfma(name, st, flops):
        us = st[0]
        tf = flops / us / 1e6
        out[name] = {"us_per_call": round(us, 3), "us_min": round(st[1], 3),
                     "us_max": round(st[2], 3), "tflops": round(tf, 1),
                     "pct_peak_f16_mfma": round(100 * tf / PEAK_F16_TFLOPS, 1)}

    timed = lambda calls, n=steps: time_calls_stats(torch, calls, n, warm)  # noqa: E731

    # one GDA decode step of the small layer the CPU reference runs: 8
    # signal/noise head pairs over 4 KV heads (GQA 2), fp16 cache of 1024
    # rows: the fused step (bytes: 4 cache streams, q1, q2, y) and the
    # reference's three calls (two sdpa_dual_v + gda_post_split, gr 1: 6
    # streams, and o, n written and read back)
    calls, keep = make_small_step_calls(torch, lib, dev, 16)
    hbm("gda_step_f16_8pairs_4kv_kv1024", timed(calls), 4 * 4 * 1024 * D * 2 + 16 * D * 2 +
        8 * 2 * D * 2)
    del calls, keep
    calls, keep = make_small_step_calls(torch, lib, dev, 16, fused=False)
    hbm("gda_step_f16_8pairs_4kv_kv1024_three_calls", timed(calls),
        6 * 4 * 1024 * D * 2 + 16 * D * 2 + 3 * 8 * 2 * D * 2)
    del calls, keep
    # the 12.7B layer call at kv 3204, 48 back-to-back calls over 48
    # distinct layer buffers
    calls, keep = make_fp16_calls(torch, lib, dev, 48, kv_len=3204, cap=3328)
    hbm("sdpa_dual_v_f16_kv3204_x48_layers", timed(calls, 48 * 4), alg_bytes("f16", 3204))
    del calls, keep
    torch.cuda.empty_cache()
    calls, keep = make_decode_calls(torch, lib, dev, 6, fused=True)
    hbm("gda_decode_step_f16_kv16000", timed(calls), decode_bytes(KV_LEN, True))
    del calls, keep
    # the 12.7B layer's decode step at kv 3204 with the token's row written
    # inside the launch, over 48 distinct layer caches
    calls, keep = make_decode_calls(torch, lib, dev, 48, kv_len=3204, cap=3328, append="fused")
    hbm("gda_decode_step_append_f16_kv3204_x48_layers", timed(calls, 48 * 4),
        decode_bytes(3204, True))
    del calls, keep
    torch.cuda.empty_cache()
    # the packed 16k decode with bf16 activations, scales and biases
    for bits, nsets in ((4, 24), (8, 16)):
        calls, keep = make_q_calls(torch, lib, dev, nsets, bits, bf16=True)
        hbm(f"sdpa_dual_v_q{bits}_bf16_kv16000", timed(calls), alg_bytes(f"q{bits}"))
        del calls, keep
        torch.cuda.empty_cache()
    # the fused epilogues at prefill length 3204
    g7 = torch.Generator(device=dev)
    g7.manual_seed(7)
    o = [torch.randn((1, 16, 3204, 128), generator=g7, device=dev).half() for _ in range(8)]
    n = [torch.randn((1, 16, 3204, 128), generator=g7, device=dev).half() for _ in range(8)]
    w = torch.rand(128, generator=g7, device=dev).half()
    lam = torch.tensor([0.37], device=dev)
    hbm("gda_post_split_1x16x3204x128",
        timed([lambda i=i: gda_post_split(o[i], n[i], w, lam, 0.2, 1, 1e-6) for i in range(8)]),
        3 * 16 * 3204 * 128 * 2)
    del o, n
    xs = [torch.randn((3204, 13824), generator=g7, device=dev).half() for _ in range(4)]
    pw = torch.rand(3, generator=g7, device=dev).half()
    pb = torch.zeros(1, device=dev).half()
    hbm("polynorm_3204x13824", timed([lambda i=i: polynorm(xs[i], pw, pb, 1e-6)
                                      for i in range(4)]), 2 * 3204 * 13824 * 2)
    del xs
    torch.cuda.empty_cache()
    calls, keep = make_fp16_calls(torch, lib, dev, 6, kv_len=32768, cap=32768, s_q=5)
    hbm("verify_slab_f16_5x32768", timed(calls), alg_bytes("f16", 32768, s_q=5))
    del calls, keep
    torch.cuda.empty_cache()
    calls, keep = make_q_calls(torch, lib, dev, 8, 8, kv_len=32768, cap=32768, s_q=5)
    hbm("verify_slab_q8_5x32768", timed(calls), alg_bytes("q8", 32768, s_q=5))
    del calls, keep
    torch.cuda.empty_cache()
    calls, keep = make_fp16_calls(torch, lib, dev, 4, kv_len=3716, cap=3840, s_q=512)
    mfma("prefill_f16_512x3716_causal", timed(calls), 2 * HQ * 512 * 3716 * D * 3)
    del calls, keep
    torch.cuda.empty_cache()
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    off, S = 3204, 512
    cap = (off + S + 255) // 256 * 256
    sets = [(torch.randn((B, S, 40 * D), generator=g, device=dev).half(),
             torch.randn((B, S, 16 * D), generator=g, device=dev).half(),
             torch.randn((B, S, 16 * D), generator=g, device=dev).half(),
             [torch.randn((B, HKV, cap, D), generator=g, device=dev).half() for _ in range(4)])
            for _ in range(4)]
    calls = [lambda st=st: gda_prefill_attention_from_proj(st[0], st[1], st[2], st[3], off, 8, 4,
                                                           8, D ** -0.5) for st in sets]
    mfma("prefill_layer_chunk_f16_512_at_3204", timed(calls),
         2 * (HQ + HKV) * D * 3 * sum(off + s + 1 for s in range(S)))
    del calls, sets
    torch.cuda.empty_cache()
    return out


def run_extra(torch, lib, dev, args):
    """µs/call of the other workloads of the path (stderr, one JSON per line)."""
    from mlx_motif.cache import MotifGroupedQuantizedKVCache
    from mlx_motif.kernels import gda_post_split, polynorm

    steps, warm = max(20, args.steps // 4), 5

    def report(name, us, nbytes):
        gbps = nbytes / us / 1e3
        log("EXTRA " + json.dumps({"workload": name, "us_per_call": round(us, 3),
                                   "gbps": round(gbps, 1),
                                   "pct_peak": round(100 * gbps / PEAK_HBM_GBPS, 1)}))

    # the headline shape over a bf16 cache (bf16 matrix-core kernel)
    calls, keep = make_fp16_calls(torch, lib, dev, 8, bf16=True)
    report("sdpa_dual_v bf16 kv16000", time_calls(torch, calls, steps, warm), alg_bytes("f16"))
    del calls, keep
    torch.cuda.empty_cache()
    # 48 back-to-back layer calls at kv_len 3204 over 48 distinct layer buffers
    calls, keep = make_fp16_calls(torch, lib, dev, 48, kv_len=3204, cap=3328)
    report("sdpa_dual_v f16 kv3204 x48 layers", time_calls(torch, calls, 48 * 4, warm),
           alg_bytes("f16", 3204))
    del calls, keep
    # one GDA decode-attention step (origin + noise passes + gda_post_split)
    # at kv_len 16000: fused entry vs the reference's three calls; GB/s over
    # the bytes each one must move (4 vs 6 cache streams)
    for bits, nsets in ((None, 6), (4, 18), (8, 12)):
        for fused in (True, False):
            calls, keep = make_decode_calls(torch, lib, dev, nsets, fused=fused, bits=bits)
            cache = "f16" if not bits else f"q{bits}"
            report(f"gda decode step {cache} kv16000 ({'fused' if fused else 'three calls'})",
                   time_calls(torch, calls, steps, warm), decode_bytes(KV_LEN, fused, bits=bits))
            del calls, keep
            torch.cuda.empty_cache()
    # the same step with the token's cache write: inside the attention launch
    # vs the cache write (4 slice copies / motif_quant_write4) before the step
    for bits, nsets in ((None, 6), (4, 18), (8, 12)):
        cache = "f16" if not bits else f"q{bits}"
        row = D * 2 if not bits else D * bits // 8 + 2 * (D // GS) * 2
        nbytes = decode_bytes(KV_LEN, True, bits=bits) + 4 * B * HKV * (row + D * 2)
        for mode in ("fused", "write"):
            calls, keep = make_decode_calls(torch, lib, dev, nsets, bits=bits, append=mode)
            label = "write in the step" if mode == "fused" else "write, then step"
            report(f"gda decode step + token write {cache} kv16000 ({label})",
                   time_calls(torch, calls, steps, warm), nbytes)
            del calls, keep
            torch.cuda.empty_cache()
    # verify slab: 5 rows over an fp16 cache of 32768 rows (16 + 4 columns)
    calls, keep = make_fp16_calls(torch, lib, dev, 6, kv_len=32768, cap=32768, s_q=5)
    report("verify slab f16 5 rows kv32768", time_calls(torch, calls, steps, warm),
           alg_bytes("f16", 32768, s_q=5))
    del calls, keep
    torch.cuda.empty_cache()
    # verify slab: 5 rows over a q8 cache of 32768 rows
    calls, keep = make_q_calls(torch, lib, dev, 8, 8, kv_len=32768, cap=32768, s_q=5)
    report("verify slab q8 5 rows kv32768", time_calls(torch, calls, steps, warm),
           alg_bytes("q8", 32768, s_q=5))
    del calls, keep
    torch.cuda.empty_cache()
    # prefill chunk: 512 query rows of 32 heads over a 3716-row fp16 cache
    # (bottom-right causal), the multi-row kernel with LDS-shared K/V tiles;
    # matrix-core bound, so reported as TFLOP/s of QK^T and both PV products
    # (and a 2048-row chunk over 4228 rows: blocks of 256 heads, no row split)
    for s_q, kvl, cap in ((512, 3716, 3840), (2048, 4228, 4352)):
        calls, keep = make_fp16_calls(torch, lib, dev, 4, kv_len=kvl, cap=cap, s_q=s_q)
        us = time_calls(torch, calls, steps if s_q == 512 else max(steps // 4, 1), warm)
        flops = 2 * HQ * s_q * kvl * D * 3
        log("EXTRA " + json.dumps({
            "workload": f"prefill chunk f16 {s_q} rows kv{kvl} (causal)",
            "us_per_call": round(us, 3), "tflops": round(flops / us / 1e6, 1),
            "pct_peak_f16_mfma": round(100 * flops / us / 1e6 / PEAK_F16_TFLOPS, 1)}))
        del calls, keep
        torch.cuda.empty_cache()
    # a 12.7B layer's prefill chunk from the projections: 512 rows at offset
    # 3204 (and a first chunk at offset 0), RoPE + cache write + origin
    # (32 heads) and noise (8 heads) passes in one launch, against
    # rope_split4 + two multi-row calls
    from mlx_motif.kernels import gda_prefill_attention_from_proj, rope_split4, sdpa_dual_v_rows
    g3 = torch.Generator(device=dev)
    g3.manual_seed(9)
    for off in (3204, 0):
        S = 512
        cap = (off + S + 255) // 256 * 256
        sets = []
        for _ in range(4):
            sets.append((torch.randn((B, S, 40 * D), generator=g3, device=dev).half(),
                         torch.randn((B, S, 16 * D), generator=g3, device=dev).half(),
                         torch.randn((B, S, 16 * D), generator=g3, device=dev).half(),
                         [torch.randn((B, HKV, cap, D), generator=g3, device=dev).half()
                          for _ in range(4)]))
        flops = 2 * (HQ + HKV) * D * 3 * sum(off + s + 1 for s in range(S))

        def fused(st):
            return lambda: gda_prefill_attention_from_proj(st[0], st[1], st[2], st[3], off, 8, 4,
                                                           8, D ** -0.5)

        def unfused(st):
            def call():
                q1, q2, k1, k2, v1, v2 = rope_split4(st[0], st[1], st[2], 8, 4, 8, 1, off,
                                                     caches=st[3])
                sdpa_dual_v_rows(q1, k1, v1, v2, D ** -0.5, kv_len=off + S, causal=True)
                sdpa_dual_v_rows(q2, k2, v1, v2, D ** -0.5, kv_len=off + S, causal=True)
            return call

        for name, mk in (("one launch", fused), ("rope_split4 + 2 calls", unfused)):
            us = time_calls(torch, [mk(st) for st in sets], steps, warm)
            log("EXTRA " + json.dumps({
                "workload": f"prefill layer chunk f16 512 rows at offset {off}, 32+8 heads ({name})",
                "us_per_call": round(us, 3), "tflops": round(flops / us / 1e6, 1),
                "pct_peak_f16_mfma": round(100 * flops / us / 1e6 / PEAK_F16_TFLOPS, 1)}))
        del sets
        torch.cuda.empty_cache()
    # gda_post_split prefill [1,16,3204,128]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    o = [torch.randn((1, 16, 3204, 128), generator=g, device=dev).half() for _ in range(8)]
    n = [torch.randn((1, 16, 3204, 128), generator=g, device=dev).half() for _ in range(8)]
    w = torch.rand(128, generator=g, device=dev).half()
    lam = torch.tensor([0.37], device=dev)
    calls = [lambda i=i: gda_post_split(o[i], n[i], w, lam, 0.2, 1, 1e-6) for i in range(8)]
    report("gda_post_split [1,16,3204,128]", time_calls(torch, calls, steps, warm),
           3 * 16 * 3204 * 128 * 2)
    del o, n, calls
    # PolyNorm [3204, 13824]
    xs = [torch.randn((3204, 13824), generator=g, device=dev).half() for _ in range(4)]
    pw = torch.rand(3, generator=g, device=dev).half()
    pb = torch.zeros(1, device=dev).half()
    calls = [lambda i=i: polynorm(xs[i], pw, pb, 1e-6) for i in range(4)]
    report("polynorm [3204,13824]", time_calls(torch, calls, steps, warm),
           2 * 3204 * 13824 * 2)
    del xs, calls
    # a layer's whole decode attention from the projections at kv_len 16000:
    # rope_split4 (q1/q2 roped, the token's k1/k2/v1/v2 rows into the cache)
    # then the fused step (attention + merge/epilogue): three launches
    from mlx_motif.kernels import gda_decode_attention, rope_split4 as _rope
    g2 = torch.Generator(device=dev)
    g2.manual_seed(5)
    layers = []
    for _ in range(6):
        slots = [torch.randn((B, HKV, CAP, D), generator=g2, device=dev).half() for _ in range(4)]
        layers.append(slots)
    qp1 = torch.randn((B, 1, 40 * D), generator=g2, device=dev).half()
    kp1 = torch.randn((B, 1, 16 * D), generator=g2, device=dev).half()
    vp1 = torch.randn((B, 1, 16 * D), generator=g2, device=dev).half()
    wsub = torch.rand(2 * D, generator=g2, device=dev).half()
    lam1 = torch.tensor([0.37], dtype=torch.float32, device=dev)

    def layer_step(slots):
        def call():
            q1, q2, *_ = _rope(qp1, kp1, vp1, 8, 4, 8, 1, KV_LEN - 1, caches=slots)
            gda_decode_attention(q1, q2, *slots, D ** -0.5, wsub, lam1, 0.2, 4, 1e-5,
                                 kv_len=KV_LEN)
        return call

    report("decode layer attention f16 kv16000 (rope_split4 + fused step)",
           time_calls(torch, [layer_step(sl) for sl in layers], steps, warm),
           decode_bytes(KV_LEN, True))
    from mlx_motif.kernels import gda_decode_attention_from_proj

    def layer_proj(slots):
        return lambda: gda_decode_attention_from_proj(qp1, kp1, vp1, *slots, D ** -0.5, wsub,
                                                      lam1, 0.2, 4, KV_LEN - 1)

    report("decode layer attention f16 kv16000 (from projections, RoPE in the step)",
           time_calls(torch, [layer_proj(sl) for sl in layers], steps, warm),
           decode_bytes(KV_LEN, True))
    from mlx_motif.kernels import gda_decode_attention_q4_from_proj, quantize as _quant
    qlayers = [[_quant(t, GS, 4) for t in sl] for sl in layers]
    del layers
    torch.cuda.synchronize()

    def layer_q_proj(slots):
        return lambda: gda_decode_attention_q4_from_proj(qp1, kp1, vp1, *slots, D ** -0.5, wsub,
                                                         lam1, 0.2, 4, KV_LEN - 1, GS, 4)

    report("decode layer attention q4 kv16000 (from projections, RoPE in the step)",
           time_calls(torch, [layer_q_proj(sl) for sl in qlayers], steps, warm),
           decode_bytes(KV_LEN, True, bits=4))
    layers = qlayers
    del layers
    torch.cuda.empty_cache()
    # RoPE + head split + 4-slot write of a 512-row prefill chunk (12.7B
    # heads: 40 q, 16 k, 16 v heads of 128) into an fp16 cache at offset 3204
    from mlx_motif.kernels import rope_split4
    qp = torch.randn((1, 512, 40 * 128), device=dev).half()
    kp = torch.randn((1, 512, 16 * 128), device=dev).half()
    vp = torch.randn((1, 512, 16 * 128), device=dev).half()
    slots = [torch.zeros((1, 8, 3840, 128), device=dev).half() for _ in range(4)]
    report("rope_split4 512 rows into the 4-slot cache",
           time_calls(torch, [lambda: rope_split4(qp, kp, vp, 8, 4, 8, 1, 3204, caches=slots)],
                      steps, warm), 2 * 512 * 72 * 128 * 2)
    del qp, kp, vp, slots
    # decode write of one token into four q4 slots at row 15999
    cache = MotifGroupedQuantizedKVCache(group_size=64, bits=4)
    big = torch.randn((1, 8, 15999, 128), device=dev).half()
    cache.update_and_fetch_4_quantized(big, big, big, big)
    tok = torch.randn((1, 8, 1, 128), device=dev).half()

    def write():
        cache.offset = 15999
        cache.update_and_fetch_4_quantized(tok, tok, tok, tok)

    report("quant_write4 q4 1 token", time_calls(torch, [write], steps, warm),
           4 * 8 * 128 * 2 + 4 * 8 * (64 + 8))


if __name__ == "__main__":
    sys.exit(main())
