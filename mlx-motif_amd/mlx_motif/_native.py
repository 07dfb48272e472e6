"""ctypes binding of ``libmotif_hip.so`` (the C ABI in ``include/motif_hip.h``).

The shared library is built in-tree (``make -C mlx-motif_amd/csrc``) into
``mlx_motif/_lib/``.  There is no fallback: if the library is missing or a
tensor is not on a ROCm device, the call raises.  Tensors are torch tensors
used only as device memory; the ABI sees raw pointers, sizes and the current
torch stream.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().with_name("_lib") / "libmotif_hip.so"

MOTIF_OK = 0
MOTIF_ERR_CONTRACT = -1
MOTIF_ERR_UNSUPPORTED = -2
MOTIF_ERR_WORKSPACE = -3
MOTIF_ERR_HIP = -4
MOTIF_ERR_INTERNAL = -5

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f = ctypes.c_float
_c_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_VP4 = _vp * 4

# name -> (restype, argtypes); mirrors include/motif_hip.h
_SIGNATURES = {
    "motif_abi_version": (_c_int, []),
    "motif_last_error": (ctypes.c_char_p, []),
    "motif_sdpa_counter_bytes": (_c_sz, [_c_int] * 4),
    "motif_plan_selfcheck": (_c_int, []),
    "motif_sdpa_workspace_bytes": (_c_sz, [_c_int] * 6),
    "motif_sdpa_dual_v": (
        _c_int,
        [_vp] * 5 + [_c_int] * 7 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_noalloc": (
        _c_int,
        [_vp] * 5 + [_c_int] * 7 + [_c_f, _vp],
    ),
    "motif_sdpa_dual_v_rows": (
        _c_int,
        [_vp] * 5 + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_q": (
        _c_int,
        [_vp] * 11 + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_q_rows": (
        _c_int,
        [_vp] * 11 + [_c_int] * 11 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_q4": (
        _c_int,
        [_vp] * 11 + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_verify": (
        _c_int,
        [_vp] * 5 + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_sdpa_dual_v_q4_verify": (
        _c_int,
        [_vp] * 11 + [_c_int] * 11 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_quantize": (_c_int, [_vp] * 4 + [_c_int, _c_i64, _c_int, _c_int, _c_int, _vp]),
    "motif_dequantize": (_c_int, [_vp] * 4 + [_c_int, _c_i64, _c_int, _c_int, _c_int, _vp]),
    "motif_quant_write4": (
        _c_int,
        [_vp] * 4 + [_VP4, _VP4, _VP4] + [_c_int] * 9 + [_vp],
    ),
    "motif_gda_post_split": (
        _c_int,
        [_vp] * 4 + [_c_int] * 7 + [_vp, _c_f, _c_f, _vp],
    ),
    "motif_gda_post": (
        _c_int,
        [_vp] * 3 + [_c_int] * 6 + [_vp, _c_f, _c_f, _vp],
    ),
    "motif_gda_decode_workspace_bytes": (_c_sz, [_c_int] * 5),
    "motif_gda_decode": (
        _c_int,
        [_vp] * 8 + [_c_f, _c_f, _vp] + [_c_int] * 7 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_q": (
        _c_int,
        [_vp] * 16 + [_c_f, _c_f, _vp] + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_append": (
        _c_int,
        [_vp] * 12 + [_c_f, _c_f, _vp] + [_c_int] * 7 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_proj": (
        _c_int,
        [_vp] * 9 + [_c_f, _c_f, _vp] + [_c_int] * 7 + [_c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_q_proj": (
        _c_int,
        [_vp] * 17 + [_c_f, _c_f, _vp] + [_c_int] * 9
        + [_c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_proj_scaled": (
        _c_int,
        [_vp] * 9 + [_c_f, _c_f, _vp] + [_c_int] * 7 + [_c_f, _c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_q_proj_scaled": (
        _c_int,
        [_vp] * 17 + [_c_f, _c_f, _vp] + [_c_int] * 9
        + [_c_f, _c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_heads_workspace_bytes": (_c_sz, [_c_int] * 6),
    "motif_gda_decode_heads": (
        _c_int,
        [_vp] * 12 + [_c_f, _c_f, _vp] + [_c_int] * 8 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_q_heads": (
        _c_int,
        [_vp] * 20 + [_c_f, _c_f, _vp] + [_c_int] * 10 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_gda_decode_q_append": (
        _c_int,
        [_vp] * 20 + [_c_f, _c_f, _vp] + [_c_int] * 9 + [_c_f, _vp, _c_sz, _vp],
    ),
    "motif_polynorm": (_c_int, [_vp] * 4 + [_c_int, _c_i64, _c_int, _c_f, _vp]),
    "motif_rope_split4": (_c_int, [_vp] * 9 + [_c_int] * 11 + [_c_f, _c_int, _vp]),
    "motif_rope_split4_scaled": (_c_int, [_vp] * 9 + [_c_int] * 11 + [_c_f, _c_f, _c_int, _vp]),
    "motif_gda_prefill_workspace_bytes": (_c_sz, [_c_int] * 7),
    "motif_gda_prefill_proj": (
        _c_int,
        [_vp] * 9 + [_c_int] * 9 + [_c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_gda_prefill_proj_scaled": (
        _c_int,
        [_vp] * 9 + [_c_int] * 9 + [_c_f, _c_f, _c_f, _c_int, _vp, _c_sz, _vp],
    ),
    "motif_set_tuning": (_c_int, [ctypes.c_char_p, _c_int]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MotifNativeError(RuntimeError):
    """A non-OK status from libmotif_hip (message from motif_last_error())."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libmotif_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = pathlib.Path(os.environ.get("MOTIF_HIP_LIB", LIB_PATH))
            if not path.is_file():
                raise RuntimeError(
                    f"libmotif_hip.so not found at {path}: build it with "
                    "`make -C mlx-motif_amd/csrc -j8` (or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(str(path))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def exported_names() -> list[str]:
    return sorted(_SIGNATURES)


def check(status: int) -> None:
    if status != MOTIF_OK:
        msg = lib().motif_last_error().decode(errors="replace")
        raise MotifNativeError(status, msg)


def dtype_code(t: torch.dtype) -> int:
    try:
        return DTYPE_CODES[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}; expected float16, bfloat16 or float32") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it.  No CPU path exists."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "mlx_motif HIP kernels need tensors on a ROCm device "
                f"(got {t.device}); set MLX_MOTIF_DISABLE_KERNELS=1 for the reference path"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ------------------------------------------------------------ workspace ---
_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Buffers a larger call superseded.  A HIP graph captured earlier on that
# stream still holds their addresses, so they are kept (not returned to the
# allocator, where another tensor could take the memory a replay writes).
_retired: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per (device, stream) split-KV workspace; counters start at zero.

    Calls on one stream are ordered, so they can share it; the kernels leave
    the counters zero.  Growing allocates a fresh zeroed buffer of at least
    twice the old size and retires the old one without freeing it (graphs
    captured before the growth replay into it), so the retired memory stays
    below the live buffer's size.  ``release_retired_workspaces`` frees it
    once no such graph is alive.
    """
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream_of(device))
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 1 << 20, 2 * buf.numel() if buf is not None else 0)
            new = torch.zeros(size, dtype=torch.uint8, device=device)
            if buf is not None:
                _retired.append(buf)
            _workspaces[key] = buf = new
        return buf


def release_retired_workspaces() -> int:
    """Frees the workspaces that growth superseded; returns their bytes.
    Only safe when no HIP graph captured before a growth is still replayed."""
    with _ws_lock:
        n = sum(t.numel() for t in _retired)
        _retired.clear()
        return n


def set_tuning(key: str, value: int) -> None:
    check(lib().motif_set_tuning(key.encode(), int(value)))
