"""A GDA layer's prefill chunk from the projection outputs:
``gda_prefill_attention_from_proj``.

For a chunk of S tokens at cache offset ``offset`` the reference ropes q and
k (``src/mlx_motif/model.py:590-594``), splits k/v into the four slots and
writes them with ``update_and_fetch_4`` (``model.py:620-629``), splits q
into q1/q2 (``model.py:669-679``) and, on the k_ratio-1 fallback, runs four
``mx.fast.scaled_dot_product_attention`` calls with the causal mask whose
concatenated outputs are the origin and noise attention
(``model.py:769-797``), which then feed ``gda_post_split``.  Here that is one
attention launch (``motif_gda_prefill_proj``; a split merge follows when the
rows are split): q roped in registers, the chunk's K/V tiles taken from the
projections and roped in LDS, the chunk's rows written into the 4-slot cache.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common
from .attention import sdpa_dual_v_rows
from .rope import _heads, rope_position_scale, rope_split4, rope_split4_reference


def gda_prefill_attention_from_proj_reference(q_proj, k_proj, v_proj, caches, offset: int,
                                              q_groups: int, gr: int, k_groups: int,
                                              scale: float, theta: float = 10000.0,
                                              origin_first: bool = False,
                                              position_scale: float = 1.0):
    """Torch-op composition: ``rope_split4_reference`` into the cache, then
    the bottom-right causal dual-V attention of q1 over k1 and of q2 over k2
    (both over V1/V2)."""
    from .attention import _causal_mask, sdpa_dual_v_reference

    q1, q2, k1, k2, v1, v2 = rope_split4_reference(q_proj, k_proj, v_proj, q_groups, gr,
                                                   k_groups, 1, offset, theta, origin_first,
                                                   caches=caches, position_scale=position_scale)
    S = q_proj.shape[1]
    kv_len = offset + S
    mask = _causal_mask(S, kv_len, q_proj.device)
    cut = lambda t: t[..., :kv_len, :]  # noqa: E731
    y_o = sdpa_dual_v_reference(q1, cut(k1), cut(v1), cut(v2), scale, mask)
    y_n = sdpa_dual_v_reference(q2, cut(k2), cut(v1), cut(v2), scale, mask)
    return y_o, y_n


def gda_prefill_attention_from_proj(q_proj, k_proj, v_proj, caches, offset: int, q_groups: int,
                                    gr: int, k_groups: int, scale: float,
                                    theta: float = 10000.0, origin_first: bool = False,
                                    rope_scaling=None):
    """``q_proj`` (B, S, q_groups*(gr+1)*D), ``k_proj`` / ``v_proj`` (B, S,
    2*k_groups*D) (k_ratio 1); ``caches`` the full-capacity fp 4-slot cache
    ``(k1, k2, v1, v2)``, each (B, k_groups, cap, D), whose rows ``offset ..
    offset + S - 1`` are written (k roped at positions ``offset + s``).
    Returns ``(attn_origin, attn_noise)``: (B, q_groups*gr, S, 2D) and (B,
    q_groups, S, 2D), each ``[softmax(q k^T * scale) V1 || ... V2]`` with
    query row s seeing cache rows ``[0, offset + s]``.  One launch
    (``motif_gda_prefill_proj``) where the kernel takes the shape (fp16/bf16,
    D = 128), else ``rope_split4`` and two ``sdpa_dual_v_rows`` calls.
    ``rope_scaling``: None, or a default / linear config
    (``rope.rope_position_scale``)."""
    pscale = rope_position_scale(rope_scaling)
    if _common._DISABLE:
        return gda_prefill_attention_from_proj_reference(q_proj, k_proj, v_proj, caches, offset,
                                                         q_groups, gr, k_groups, scale, theta,
                                                         origin_first, position_scale=pscale)
    B, S, D = _heads(q_proj, k_proj, v_proj, q_groups, gr, k_groups, 1)
    assert q_groups % k_groups == 0, (
        f"q_groups={q_groups} must be a multiple of k_groups={k_groups}")
    if len(caches) != 4:
        raise ValueError("caches must be (k1, k2, v1, v2)")
    k1, k2, v1, v2 = caches
    cap = k1.shape[2]
    for c in caches:
        assert tuple(c.shape) == (B, k_groups, cap, D), (
            f"cache slot {tuple(c.shape)} must be {(B, k_groups, cap, D)}")
        if not c.is_contiguous():
            raise ValueError("the prefill writes the cache in place: it must be contiguous")
    assert 0 <= offset and offset + S <= cap, f"rows [{offset}, {offset + S}) exceed {cap}"
    dev = _native.require_device(q_proj, k_proj, v_proj, *caches)
    dt = q_proj.dtype
    for t in (k_proj, v_proj, *caches):
        if t.dtype != dt:
            raise TypeError(f"dtype {t.dtype} must match q dtype {dt}")
    q_proj, k_proj, v_proj = (_common.contiguous(t) for t in (q_proj, k_proj, v_proj))
    y_o = torch.empty((B, q_groups * gr, S, 2 * D), dtype=dt, device=dev)
    y_n = torch.empty((B, q_groups, S, 2 * D), dtype=dt, device=dev)
    lib = _native.lib()
    kv_len = offset + S
    nbytes = lib.motif_gda_prefill_workspace_bytes(B, S, q_groups, gr, k_groups, D, kv_len)
    ws = _native.workspace(dev, nbytes) if nbytes else None
    rc = lib.motif_gda_prefill_proj_scaled(
        q_proj.data_ptr(), k_proj.data_ptr(), v_proj.data_ptr(), *(c.data_ptr() for c in caches),
        y_o.data_ptr(), y_n.data_ptr(), _native.dtype_code(dt), B, S, q_groups, gr, k_groups, D,
        cap, int(offset), float(scale), float(theta), float(pscale), int(bool(origin_first)),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _native.stream_of(dev))
    if rc == _native.MOTIF_ERR_UNSUPPORTED:  # the separate native calls
        q1, q2, *_ = rope_split4(q_proj, k_proj, v_proj, q_groups, gr, k_groups, 1, offset, theta,
                                 origin_first, caches=caches, rope_scaling=rope_scaling)
        return (sdpa_dual_v_rows(q1, k1, v1, v2, scale, kv_len=kv_len, causal=True),
                sdpa_dual_v_rows(q2, k2, v1, v2, scale, kv_len=kv_len, causal=True))
    _native.check(rc)
    return y_o, y_n
