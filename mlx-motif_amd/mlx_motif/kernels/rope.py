"""RoPE + head split + 4-slot cache write of one attention step:
``rope_split4``.

The reference prepares a layer's attention inputs with two ``self.rope``
calls (``src/mlx_motif/model.py:590-594``; ``initialize_rope`` with
``traditional=False`` and no scaling), the k1/k2 and v1/v2 reshapes feeding
``update_and_fetch_4`` (``model.py:620-629``) and the q1/q2 split
(``model.py:669-679``).  ``rope_split4`` does all of it in one launch
(``motif_rope_split4``) from the projection outputs; with ``caches`` the
k1/k2/v1/v2 rows are written straight into the full-capacity 4-slot fp cache
at rows ``offset .. offset + S - 1``.

RoPE scaling: the reference builds its rope with
``initialize_rope(..., scaling_config=args.rope_scaling)`` (``model.py:414-419``,
mlx-lm 0.29.1).  ``None`` and the "default" type rope at positions
``offset + s``; the "linear" type of factor f ropes at ``(offset + s) / f``
(``nn.RoPE``'s ``scale = 1 / f``; the reference's grouped fixture uses f = 2),
which the kernels take as a position scale.  Other types (llama3, yarn,
longrope, ...) raise ``NotImplementedError`` rather than rope at the wrong
positions.
"""

from __future__ import annotations

import torch

from .. import _native
from . import _common


def _heads(q_proj, k_proj, v_proj, q_groups, gr, k_groups, kr):
    B, S, nq = q_proj.shape
    HQ = q_groups * (gr + 1)
    assert nq % HQ == 0, f"q width {nq} is not q_groups*(gr+1)={HQ} heads"
    D = nq // HQ
    assert k_proj.shape == (B, S, k_groups * (kr + 1) * D), "k must be (B, S, k_groups*(kr+1)*D)"
    assert v_proj.shape == (B, S, 2 * k_groups * D), "v must be (B, S, 2*k_groups*D)"
    return B, S, D


def rope_split4_reference(q_proj, k_proj, v_proj, q_groups: int, gr: int, k_groups: int,
                          kr: int, offset: int, theta: float = 10000.0,
                          origin_first: bool = False, caches=None, position_scale: float = 1.0):
    """Torch-op statement (fp32 angles and rotation, rounded once); positions
    are scaled by ``position_scale`` first."""
    B, S, D = _heads(q_proj, k_proj, v_proj, q_groups, gr, k_groups, kr)
    dev, dt = q_proj.device, q_proj.dtype
    half = D // 2
    inv = theta ** (-torch.arange(half, device=dev, dtype=torch.float32) * 2.0 / D)
    pos = (offset + torch.arange(S, device=dev, dtype=torch.float32)) * float(position_scale)
    ang = pos[:, None] * inv[None, :]
    cos, sin = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]

    def rot(x, H):
        x = x.reshape(B, S, H, D).float()
        x1, x2 = x[..., :half], x[..., half:]
        y = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
        return y.to(dt).transpose(1, 2)  # (B, H, S, D)

    HQ, HK = q_groups * (gr + 1), k_groups * (kr + 1)
    q, k = rot(q_proj, HQ), rot(k_proj, HK)
    v = v_proj.reshape(B, S, 2 * k_groups, D).transpose(1, 2)
    if origin_first:
        q1, q2 = q[:, : q_groups * gr], q[:, q_groups * gr:]
    else:
        q_ = q.reshape(B, q_groups, gr + 1, S, D)
        q1 = q_[:, :, :gr].reshape(B, q_groups * gr, S, D)
        q2 = q_[:, :, gr:].reshape(B, q_groups, S, D)
    k_ = k.reshape(B, k_groups, kr + 1, S, D)
    k1 = k_[:, :, :kr].reshape(B, k_groups * kr, S, D)
    k2 = k_[:, :, kr:].reshape(B, k_groups, S, D)
    v_ = v.reshape(B, k_groups, 2, S, D)
    rows = (k1, k2, v_[:, :, 0], v_[:, :, 1])
    if caches is None:
        return (q1.contiguous(), q2.contiguous(), *(t.contiguous() for t in rows))
    for c, r in zip(caches, rows):
        c[:, :, offset:offset + S] = r
    return (q1.contiguous(), q2.contiguous(), *caches)


def rope_position_scale(rope_scaling) -> float:
    """The position scale of a RoPE scaling config (``ModelArgs.rope_scaling``),
    read as mlx-lm's ``initialize_rope`` reads it: the type is ``"type"`` or
    else ``"rope_type"`` (default ``"default"``); ``None`` and "default" give
    1, "linear" gives ``1 / factor``.  Other types raise
    ``NotImplementedError``."""
    if rope_scaling is None:
        return 1.0
    kind = rope_scaling.get("type") or rope_scaling.get("rope_type", "default")
    if kind == "default":
        return 1.0
    if kind == "linear":
        factor = float(rope_scaling["factor"])
        if not factor > 0.0 or factor == float("inf"):
            raise ValueError(f"rope_scaling factor must be positive and finite, got {factor}")
        return 1.0 / factor
    raise NotImplementedError(
        f"rope_scaling={rope_scaling!r}: RoPE type {kind!r} is not built (default and linear "
        "are); it would otherwise be roped at the wrong positions")


def rope_split4(q_proj, k_proj, v_proj, q_groups: int, gr: int, k_groups: int, kr: int,
                offset: int, theta: float = 10000.0, origin_first: bool = False, caches=None,
                rope_scaling=None):
    """``q_proj`` (B, S, q_groups*(gr+1)*D), ``k_proj`` (B, S,
    k_groups*(kr+1)*D), ``v_proj`` (B, S, 2*k_groups*D): projection outputs.
    Returns ``(q1, q2, k1, k2, v1, v2)``: q1 (B, q_groups*gr, S, D) and q2
    (B, q_groups, S, D) roped at positions ``offset + s``; k1/k2 (roped) and
    v1/v2 either new (B, H, S, D) tensors or, with ``caches=(k1, k2, v1,
    v2)`` full-capacity (B, H, cap, D) buffers, those buffers with rows
    ``offset .. offset + S - 1`` written.  ``rope_scaling``: None, or a
    default / linear config (``rope_position_scale``)."""
    pscale = rope_position_scale(rope_scaling)
    if _common._DISABLE:
        return rope_split4_reference(q_proj, k_proj, v_proj, q_groups, gr, k_groups, kr, offset,
                                     theta, origin_first, caches, position_scale=pscale)
    B, S, D = _heads(q_proj, k_proj, v_proj, q_groups, gr, k_groups, kr)
    dev = _native.require_device(q_proj, k_proj, v_proj, *(caches or ()))
    dt = q_proj.dtype
    for t in (k_proj, v_proj, *(caches or ())):
        if t.dtype != dt:
            raise TypeError(f"dtype {t.dtype} must match q dtype {dt}")
    q_proj, k_proj, v_proj = (_common.contiguous(t) for t in (q_proj, k_proj, v_proj))
    new = lambda h, n: torch.empty((B, h, n, D), dtype=dt, device=dev)  # noqa: E731
    q1, q2 = new(q_groups * gr, S), new(q_groups, S)
    if caches is None:
        outs = (new(k_groups * kr, S), new(k_groups, S), new(k_groups, S), new(k_groups, S))
        cap, row0 = S, 0
    else:
        if len(caches) != 4:
            raise ValueError("caches must be (k1, k2, v1, v2)")
        cap = caches[0].shape[2]
        shapes = ((B, k_groups * kr, cap, D), (B, k_groups, cap, D), (B, k_groups, cap, D),
                  (B, k_groups, cap, D))
        for c, shp in zip(caches, shapes):
            assert tuple(c.shape) == shp, f"cache slot {tuple(c.shape)} must be {shp}"
            if not c.is_contiguous():
                raise ValueError("rope_split4 writes the cache in place: it must be contiguous")
        assert 0 <= offset and offset + S <= cap, f"rows [{offset}, {offset + S}) exceed {cap}"
        outs, row0 = tuple(caches), offset
    _native.check(
        _native.lib().motif_rope_split4_scaled(
            q_proj.data_ptr(), k_proj.data_ptr(), v_proj.data_ptr(), q1.data_ptr(), q2.data_ptr(),
            *(t.data_ptr() for t in outs), _native.dtype_code(dt), B, S, q_groups, gr, k_groups,
            kr, D, cap, row0, int(offset), float(theta), float(pscale), int(bool(origin_first)),
            _native.stream_of(dev),
        )
    )
    return (q1, q2, *outs)
