"""ctypes binding of the C restatement (oracle/_build/libmotif_oracle.so).

TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg).  Arrays are
numpy: fp16 data as float16 arrays (passed as their uint16 bits), packed
words as uint32, outputs float32.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = _DIR / "_build" / "libmotif_oracle.so"
# The same source built -O3 -march=x86-64-v3 -ffast-math: a vectorised CPU
# baseline for bench.py, never a checker.
FAST_LIB_PATH = _DIR / "_build" / "libmotif_oracle_fast.so"
_libs = {}


def build() -> None:
    subprocess.run(["make", "-B", "-C", str(_DIR)], check=True, capture_output=True)


def lib(fast: bool = False) -> ctypes.CDLL:
    path = FAST_LIB_PATH if fast else LIB_PATH
    if path not in _libs:
        if not path.is_file():
            build()
        handle = ctypes.CDLL(str(path))
        handle.motif_oracle_max_threads.restype = ctypes.c_int
        _libs[path] = handle
    return _libs[path]


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def max_threads() -> int:
    return lib().motif_oracle_max_threads()


def sdpa_dual_v_f16(q, k, v1, v2, scale, kv_len=None, causal=False, nthreads=0, fast=False):
    q, k, v1, v2 = (np.ascontiguousarray(t, dtype=np.float16) for t in (q, k, v1, v2))
    B, Hq, S, D = q.shape
    _, Hkv, cap, _ = k.shape
    kv_len = cap if kv_len is None else kv_len
    y = np.empty((B, Hq, S, 2 * D), dtype=np.float32)
    f = lib(fast).motif_oracle_sdpa_dual_v_f16
    f.restype = None
    f(_p(q), _p(k), _p(v1), _p(v2), _p(y), ctypes.c_int(B), ctypes.c_int(Hq), ctypes.c_int(Hkv),
      ctypes.c_int(S), ctypes.c_int(D), ctypes.c_int(cap), ctypes.c_int(kv_len),
      ctypes.c_int(int(causal)), ctypes.c_float(scale), ctypes.c_int(nthreads))
    return y


def sdpa_dual_v_q_f16(q, k_q, v1_q, v2_q, scale, group_size=64, bits=4, kv_len=None,
                      causal=False, nthreads=0, fast=False):
    q = np.ascontiguousarray(q, dtype=np.float16)
    trip = []
    for t in (k_q, v1_q, v2_q):
        trip.append(np.ascontiguousarray(t[0], dtype=np.uint32))
        trip.append(np.ascontiguousarray(t[1], dtype=np.float16))
        trip.append(np.ascontiguousarray(t[2], dtype=np.float16))
    B, Hq, S, D = q.shape
    _, Hkv, cap, _ = trip[0].shape
    kv_len = cap if kv_len is None else kv_len
    y = np.empty((B, Hq, S, 2 * D), dtype=np.float32)
    f = lib(fast).motif_oracle_sdpa_dual_v_q_f16
    f.restype = None
    f(_p(q), *[_p(a) for a in trip], _p(y), ctypes.c_int(B), ctypes.c_int(Hq),
      ctypes.c_int(Hkv), ctypes.c_int(S), ctypes.c_int(D), ctypes.c_int(cap),
      ctypes.c_int(kv_len), ctypes.c_int(int(causal)), ctypes.c_int(bits),
      ctypes.c_int(group_size), ctypes.c_float(scale), ctypes.c_int(nthreads))
    return y


def quantize_f16(x, group_size=64, bits=4):
    x = np.ascontiguousarray(x, dtype=np.float16)
    *lead, D = x.shape
    rows = x.size // D
    data = np.empty((*lead, D * bits // 32), dtype=np.uint32)
    scales = np.empty((*lead, D // group_size), dtype=np.float16)
    biases = np.empty_like(scales)
    f = lib().motif_oracle_quantize_f16
    f.restype = None
    f(_p(x), _p(data), _p(scales), _p(biases), ctypes.c_long(rows), ctypes.c_int(D),
      ctypes.c_int(bits), ctypes.c_int(group_size))
    return data, scales, biases
