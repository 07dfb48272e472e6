"""The C ABI surface on the CPU: the library loads, exports exactly what
include/motif_hip.h declares (and what the ctypes binding binds), and
rejects out-of-contract arguments before touching the GPU.  No kernel runs.
"""

from __future__ import annotations

import pathlib
import re
import subprocess

import pytest

from mlx_motif import _native

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "motif_hip.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(motif_[a-z0-9_]+)\s*\(", text))


def test_header_symbols_are_exported_and_bound():
    lib = _native.lib()
    declared = _declared()
    assert declared == set(_native.exported_names()), declared ^ set(_native.exported_names())
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (motif_[a-z0-9_]+)$", out, flags=re.M))
    assert declared <= exported, declared - exported
    for name in declared:
        assert getattr(lib, name) is not None


def test_abi_version():
    assert _native.lib().motif_abi_version() == 1


def _err():
    return _native.lib().motif_last_error().decode()


def test_sdpa_contract_rejections_need_no_gpu():
    lib = _native.lib()
    st = lib.motif_sdpa_dual_v(None, None, None, None, None, 0, 1, 32, 8, 100, 256, 10, 0.1,
                               None, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "multiple of 32" in _err()
    st = lib.motif_sdpa_dual_v(None, None, None, None, None, 0, 1, 30, 8, 128, 256, 10, 0.1,
                               None, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "multiple of H_kv" in _err()
    st = lib.motif_sdpa_dual_v(None, None, None, None, None, 0, 1, 32, 8, 128, 256, 300, 0.1,
                               None, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "kv_len=300" in _err()
    st = lib.motif_sdpa_dual_v(None, None, None, None, None, 7, 1, 32, 8, 128, 256, 3, 0.1,
                               None, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "dtype" in _err()


@pytest.mark.parametrize("D,bits,fragment", [
    (256, 8, "D/32 <= 32/bits"), (512, 4, "qk_per_thread | EL_PER_INT"),
    (96, 8, "qk_per_thread | EL_PER_INT"), (160, 4, "qk_per_thread | EL_PER_INT"),
])
def test_packed_layout_contract_rejections(D, bits, fragment):
    lib = _native.lib()
    st = lib.motif_sdpa_dual_v_q(None, *[None] * 9, None, 0, 1, 4, 4, D, 64, 64, bits, 32, 0.1,
                                 None, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and fragment in _err()


def test_quant_and_epilogue_rejections():
    lib = _native.lib()
    assert lib.motif_quantize(None, None, None, None, 0, 4, 128, 3, 64, None) == -1
    assert "bits" in _err()
    assert lib.motif_quantize(None, None, None, None, 0, 4, 100, 4, 64, None) == -1
    assert lib.motif_quantize(None, None, None, None, 0, 4, 128, 4, 16, None) == -1
    vp4 = _native._VP4(None, None, None, None)
    st = lib.motif_quant_write4(None, None, None, None, vp4, vp4, vp4, 0, 1, 8, 2, 128, 256, 255,
                                4, 64, None)
    assert st == -1 and "exceed capacity" in _err()
    st = lib.motif_gda_post_split(None, None, None, None, 0, 1, 30, 8, 4, 1, 256, None, 0.8,
                                  1e-5, None)
    assert st == -1 and "q_origin=30 != q_groups(8) * gr(4)" in _err()
    assert lib.motif_polynorm(None, None, None, None, 5, 3, 16, 1e-6, None) == -1


@pytest.mark.parametrize("pscale", [0.0, -0.5, float("inf"), float("nan")])
def test_rope_position_scale_rejections(pscale):
    lib = _native.lib()
    st = lib.motif_rope_split4_scaled(*[None] * 9, 0, 1, 1, 8, 4, 8, 1, 128, 1, 0, 5, 1e4,
                                      pscale, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "position_scale" in _err()
    # a valid scale gets past the check to the null-pointer one
    st = lib.motif_rope_split4_scaled(*[None] * 9, 0, 1, 1, 8, 4, 8, 1, 128, 1, 0, 5, 1e4,
                                      0.5, 0, None)
    assert st == _native.MOTIF_ERR_CONTRACT and "null pointer" in _err()


def test_empty_work_is_a_no_op():
    lib = _native.lib()
    assert lib.motif_polynorm(None, None, None, None, 0, 0, 16, 1e-6, None) == 0
    assert lib.motif_quantize(None, None, None, None, 0, 0, 128, 4, 64, None) == 0
    assert lib.motif_gda_post_split(None, None, None, None, 0, 1, 0, 0, 4, 1, 256, None, 0.8,
                                    1e-5, None) == 0


def test_workspace_sizing_and_tuning():
    lib = _native.lib()
    counters = lib.motif_sdpa_counter_bytes(1, 32, 8, 1)
    assert counters == 256
    small = lib.motif_sdpa_workspace_bytes(1, 32, 8, 1, 16, 128)
    big = lib.motif_sdpa_workspace_bytes(1, 32, 8, 1, 16000, 128)
    assert counters <= small <= big
    # the split count is capped (256 per KV head), so the partials are bounded
    assert big <= counters + 32 * 256 * (2 * 128 + 2) * 4 + 512
    with pytest.raises(_native.MotifNativeError):
        _native.set_tuning("no_such_knob", 1)
    for key in ("qslab_ws", "merge_rows"):  # switches take 0 or 1 only
        for bad in (-1, 2):
            with pytest.raises(_native.MotifNativeError):
                _native.set_tuning(key, bad)
        _native.set_tuning(key, 1)
    for bad in (-1, 3):
        with pytest.raises(_native.MotifNativeError):
            _native.set_tuning("prefill_ncb", bad)
    _native.set_tuning("prefill_ncb", 0)
    for bad in (1, 4):
        with pytest.raises(_native.MotifNativeError):
            _native.set_tuning("qslab_sets", bad)
    _native.set_tuning("qslab_sets", 2)
    with pytest.raises(_native.MotifNativeError):
        _native.set_tuning("prefill_min_heads", -1)
    # the shared-tile kernel's workspace is covered from 17 heads over 2048+ rows
    lib = _native.lib()
    assert lib.motif_sdpa_workspace_bytes(1, 32, 8, 5, 32768, 128) > 0
    _native.set_tuning("rows_per_split", 64)
    forced = lib.motif_sdpa_workspace_bytes(1, 32, 8, 1, 16000, 128)
    _native.set_tuning("rows_per_split", 0)
    assert forced > big
    assert lib.motif_sdpa_workspace_bytes(1, 32, 8, 1, 16000, 128) == big
    # too-small workspace for a multi-split plan is refused before any launch
    st = lib.motif_sdpa_dual_v(1, 1, 1, 1, 1, 0, 1, 32, 8, 128, 16128, 16000, 0.1, None, 0, None)
    assert st == _native.MOTIF_ERR_WORKSPACE and "workspace" in _err()


def test_gda_decode_rejections_and_workspace():
    lib = _native.lib()
    args = lambda dtype, D, kv_cap, kv_len, ws, n: (  # noqa: E731
        1, 1, 1, 1, 1, 1, 1, 1, 0.8, 1e-5, 1, dtype, 1, 8, 4, D, kv_cap, kv_len, 0.1, ws, n, None)
    assert lib.motif_gda_decode(*args(7, 128, 256, 10, None, 0)) == -1 and "dtype" in _err()
    assert lib.motif_gda_decode(*args(0, 100, 256, 10, None, 0)) == -1
    assert "multiple of 32" in _err()
    assert lib.motif_gda_decode(*args(0, 128, 256, 300, None, 0)) == -1 and "kv_len" in _err()
    st = lib.motif_gda_decode(*args(0, 128, 16128, 16000, None, 0))
    assert st == _native.MOTIF_ERR_WORKSPACE and "workspace" in _err()
    # the fused path's partials (B*Hkv*(gr+1) rows) and the composed path's
    # attention outputs both fit the reported size, which grows with kv_len
    small = lib.motif_gda_decode_workspace_bytes(1, 8, 4, 16, 128)
    big = lib.motif_gda_decode_workspace_bytes(1, 8, 4, 16000, 128)
    assert 0 < small <= big
    assert big >= 8 * 5 * 32 * (2 * 128 + 2) * 4
    assert lib.motif_gda_decode_workspace_bytes(0, 8, 4, 16, 128) == 0


def test_gda_decode_heads_rejections_and_workspace():
    """The step for any noise-head count: q2's heads must be a multiple of
    H_kv and divide q1's (q_origin == q_groups * gr), and the new-row
    pointers come all null or all set; all refused before any HIP call."""
    lib = _native.lib()

    def args(Hq1, Hq2, Hkv, rows=(None,) * 4, dtype=0, kv_cap=1024, kv_len=1024, ws=None, n=0):
        return ((1, 1) + tuple(rows) + (1,) * 5 + (1, 0.8, 1e-5, 1, dtype, 1, Hq1, Hq2, Hkv, 128,
                kv_cap, kv_len, 0.1, ws, n, None))

    st = lib.motif_gda_decode_heads(*args(8, 6, 4))
    assert st == _native.MOTIF_ERR_CONTRACT and "H_q2=6 must be a multiple of H_kv=4" in _err()
    st = lib.motif_gda_decode_heads(*args(12, 8, 4))
    assert st == _native.MOTIF_ERR_CONTRACT and "H_q1=12 must be a multiple of H_q2=8" in _err()
    st = lib.motif_gda_decode_heads(*args(8, 8, 4, rows=(1, 1, None, 1)))
    assert st == _native.MOTIF_ERR_CONTRACT and "all null or all set" in _err()
    st = lib.motif_gda_decode_heads(*args(8, 8, 4, dtype=7))
    assert st == _native.MOTIF_ERR_CONTRACT and "dtype" in _err()
    st = lib.motif_gda_decode_heads(*args(8, 8, 4))
    assert st == _native.MOTIF_ERR_WORKSPACE and "workspace" in _err()
    qargs = ((1, 1) + (None,) * 4 + (1,) * 14 + (0.8, 1e-5, 1, 0, 1, 8, 6, 4, 128, 1024, 1024,
             4, 64, 0.1, None, 0, None))
    st = lib.motif_gda_decode_q_heads(*qargs)
    assert st == _native.MOTIF_ERR_CONTRACT and "multiple of H_kv" in _err()

    ws = lib.motif_gda_decode_heads_workspace_bytes
    assert ws(1, 8, 6, 4, 1024, 128) == 0 and ws(1, 12, 8, 4, 1024, 128) == 0
    assert ws(0, 8, 8, 4, 1024, 128) == 0
    # one noise head per KV head: the same layout as motif_gda_decode
    assert ws(1, 32, 8, 8, 16000, 128) == lib.motif_gda_decode_workspace_bytes(1, 8, 4, 16000, 128)
    # 8 origin + 8 noise heads over 4 KV heads: partial rows of 4 columns
    # per KV head, and the composed path's two (B, 8, 1, 2D) fp32 outputs
    n = ws(1, 8, 8, 4, 1024, 128)
    assert n >= 4 * 4 * (2 * 128 + 2) * 4 and n >= 2 * 8 * 2 * 128 * 4
    assert ws(1, 8, 8, 4, 16000, 128) >= n


def test_tuning_changes_while_other_threads_size_calls():
    """motif_set_tuning from one thread while others size calls: each call
    reads one snapshot of the knobs, so every size is the one of either
    setting (ctypes drops the GIL around the foreign calls, so the threads
    run in the library at once)."""
    import threading

    lib = _native.lib()
    args = (1, 32, 8, 1, 16000, 128)
    default = lib.motif_sdpa_workspace_bytes(*args)
    _native.set_tuning("rows_per_split", 64)
    forced = lib.motif_sdpa_workspace_bytes(*args)
    _native.set_tuning("rows_per_split", 0)
    seen, stop = set(), threading.Event()

    def size():
        while not stop.is_set():
            seen.add(lib.motif_sdpa_workspace_bytes(*args))

    threads = [threading.Thread(target=size) for _ in range(4)]
    for t in threads:
        t.start()
    try:
        for i in range(2000):
            _native.set_tuning("rows_per_split", 64 if i % 2 == 0 else 0)
    finally:
        _native.set_tuning("rows_per_split", 0)
        stop.set()
        for t in threads:
            t.join()
    assert seen <= {default, forced}, seen
    assert lib.motif_sdpa_workspace_bytes(*args) == default


def test_noalloc_refuses_calls_past_its_scratch_before_the_gpu():
    """motif_sdpa_dual_v_noalloc sizes the call on the host first: one that
    needs more than the static scratch is refused with no HIP call."""
    lib = _native.lib()
    _native.set_tuning("rows_per_split", 16)  # 256 splits per KV head, B=8: about 66 MB
    try:
        st = lib.motif_sdpa_dual_v_noalloc(1, 1, 1, 1, 1, 0, 8, 32, 8, 128, 16128, 16000, 0.1,
                                           None)
        msg = _err()
    finally:
        _native.set_tuning("rows_per_split", 0)
    assert st == _native.MOTIF_ERR_WORKSPACE and "static scratch holds 8388608" in msg
    # more B*Hq rows than counters the scratch clears
    st = lib.motif_sdpa_dual_v_noalloc(1, 1, 1, 1, 1, 0, 1024, 32, 8, 128, 64, 64, 0.1, None)
    assert st == _native.MOTIF_ERR_WORKSPACE and "counters" in _err()


def test_prefill_planner_choices_through_workspace_sizes():
    """The prefill planners' choices, read back through the workspace sizes
    (256 CUs without a device): a 12.7B layer's 512-row chunk at offset 3204
    takes two column blocks per wave (8 + 2 blocks of 256 heads per KV head)
    and 3 row splits; at offset 0 (512 rows) one block per wave and no split;
    a 512-row multi-row call over 3716 rows 4 splits of 256-head blocks."""
    lib = _native.lib()

    def parts(vrows, ns):
        r = lambda n: (n + 255) // 256 * 256  # noqa: E731
        return r(vrows * 4) + r(vrows * ns * 256 * 4) + r(vrows * ns * 2 * 4)

    vrows = 1 * 8 * (4 + 1) * 512
    assert lib.motif_gda_prefill_workspace_bytes(1, 512, 8, 4, 8, 128, 3716) == parts(vrows, 3)
    assert lib.motif_gda_prefill_workspace_bytes(1, 512, 8, 4, 8, 128, 512) == 0
    _native.set_tuning("prefill_ncb", 1)
    try:  # one block per wave: 160 blocks fit two rounds at 3 splits of 38 tiles
        assert lib.motif_gda_prefill_workspace_bytes(1, 512, 8, 4, 8, 128, 3716) == parts(vrows, 3)
    finally:
        _native.set_tuning("prefill_ncb", 0)
    assert lib.motif_sdpa_workspace_bytes(1, 32, 8, 512, 3716, 128) >= parts(32 * 512, 4)


def test_plan_selfcheck():
    """Every launch planner, walked on the host over decode, slab and prefill
    shapes: split plans get counters and partials inside their workspace,
    the pre-launch guard refuses a split plan without partial buffers (the
    fault class of a one-split slab staging partials through a null base),
    a missing workspace is refused, and the size query covers every plan.
    The no-alloc layout keeps partials past its fixed counter area."""
    from mlx_motif import _native

    lib = _native.lib()
    rc = lib.motif_plan_selfcheck()
    assert rc == _native.MOTIF_OK, lib.motif_last_error().decode()
