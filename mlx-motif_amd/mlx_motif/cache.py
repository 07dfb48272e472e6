"""4-slot KV caches of grouped differential attention, over torch device memory.

Mirror of the grouped caches of ``src/mlx_motif/cache.py:178-545``: four
separate slots k1, k2, v1, v2, capacity grown in steps of ``step = 256`` rows,
fetches that return the FULL row-contiguous capacity buffers (consumers bound
reads by ``offset``), trimming for speculative rollback, and ``state`` /
``meta_state`` that serialise only the live ``[:offset]`` rows.

The quantised cache stores each slot as an MLX-affine triple
``(data uint32, scales, biases)`` and writes the incoming rows of all four
slots with ONE kernel dispatch (``motif_quant_write4``); the reference does a
head-axis concat, one ``mx.quantize`` and 12 slice writes (``cache.py:485-512``).
"""

from __future__ import annotations

import torch

from . import _native
from .kernels import _common
from .kernels.quant import dequantize, quantize, quantize_reference


class MotifGroupedKVCacheBase:
    """Offset bookkeeping, trimming and growth shared by both 4-slot caches."""

    step = 256

    def update_and_fetch(self, keys, values):
        raise NotImplementedError(
            "MotifGroupedKVCacheBase subclasses require the model to call "
            "update_and_fetch_4 directly — the 1-slot path is intentionally unsupported."
        )

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    @property
    def state(self):
        raise NotImplementedError

    @state.setter
    def state(self, v):
        self.k1, self.k2, self.v1, self.v2 = v

    def _grow(self, B: int, H: int, S: int, D: int, dtype, device) -> None:
        """Ensure capacity for rows [offset, offset + S) (``cache.py:245-265``)."""
        prev = self.offset
        if self.k1 is None or (prev + S) > self._slot_capacity(self.k1):
            n_steps = (self.step + S - 1) // self.step
            new_len = n_steps * self.step
            if self.k1 is not None:
                if prev % self.step != 0:
                    self.k1 = self._trim_slot(self.k1, prev)
                    self.k2 = self._trim_slot(self.k2, prev)
                    self.v1 = self._trim_slot(self.v1, prev)
                    self.v2 = self._trim_slot(self.v2, prev)
                fresh = self._init_storage(B, H, new_len, D, dtype, device)
                self.k1 = self._expand_slot(self.k1, fresh)
                self.k2 = self._expand_slot(self.k2, fresh)
                self.v1 = self._expand_slot(self.v1, fresh)
                self.v2 = self._expand_slot(self.v2, fresh)
            else:
                self.k1 = self._init_storage(B, H, new_len, D, dtype, device)
                self.k2 = self._init_storage(B, H, new_len, D, dtype, device)
                self.v1 = self._init_storage(B, H, new_len, D, dtype, device)
                self.v2 = self._init_storage(B, H, new_len, D, dtype, device)

    def _slot_capacity(self, slot) -> int:
        raise NotImplementedError

    def _init_storage(self, B, H, n, D, dtype, device):
        raise NotImplementedError

    def _trim_slot(self, slot, prev: int):
        raise NotImplementedError

    def _expand_slot(self, slot, fresh):
        raise NotImplementedError

    @staticmethod
    def _assert_uniform_heads(k1, k2, v1, v2) -> None:
        h1 = k1.shape[1]
        if not (k2.shape[1] == v1.shape[1] == v2.shape[1] == h1):
            raise ValueError(
                "4-slot grouped KV cache requires k1/k2/v1/v2 to share a head "
                f"count; got k1={h1}, k2={k2.shape[1]}, v1={v1.shape[1]}, "
                f"v2={v2.shape[1]}. This happens with k_ratio > 1, which the "
                "4-slot cache does not support."
            )


class MotifGroupedKVCache(MotifGroupedKVCacheBase):
    """Unquantised 4-slot cache (fp16 / bf16 / fp32 slots)."""

    def __init__(self):
        self.k1 = self.k2 = self.v1 = self.v2 = None
        self.offset = 0

    def _slot_capacity(self, slot) -> int:
        return slot.shape[2]

    def _init_storage(self, B, H, n, D, dtype, device):
        return torch.zeros((B, H, n, D), dtype=dtype, device=device)

    def _trim_slot(self, slot, prev: int):
        return slot[..., :prev, :]

    def _expand_slot(self, slot, fresh):
        return torch.cat([slot, fresh], dim=2)

    def update_and_fetch_4(self, k1, k2, v1, v2):
        """Append the 4 incoming (B, H, S, D) slices; return the FULL capacity
        buffers (bound reads by ``offset``)."""
        self._assert_uniform_heads(k1, k2, v1, v2)
        B, H, S, D = k1.shape
        prev = self.offset
        self._grow(B, H, S, D, k1.dtype, k1.device)
        self.k1[..., prev : prev + S, :] = k1
        self.k2[..., prev : prev + S, :] = k2
        self.v1[..., prev : prev + S, :] = v1
        self.v2[..., prev : prev + S, :] = v2
        self.offset += S
        return self.k1, self.k2, self.v1, self.v2

    @property
    def state(self):
        if self.offset == 0 or self.k1 is None:
            return self.k1, self.k2, self.v1, self.v2
        o = self.offset
        return tuple(s[..., :o, :] for s in (self.k1, self.k2, self.v1, self.v2))

    @state.setter
    def state(self, v):
        self.k1, self.k2, self.v1, self.v2 = v

    @property
    def meta_state(self):
        return (str(self.offset),)

    @meta_state.setter
    def meta_state(self, v):
        self.offset = int(v[0])

    def to_quantized(self, group_size: int = 64, bits: int = 8) -> MotifGroupedQuantizedKVCache:
        """Quantise the live rows of the four slots into a quantised cache."""
        new = MotifGroupedQuantizedKVCache(group_size=group_size, bits=bits)
        if self.offset > 0:
            o = self.offset
            new.k1 = quantize(self.k1[..., :o, :], group_size=group_size, bits=bits)
            new.k2 = quantize(self.k2[..., :o, :], group_size=group_size, bits=bits)
            new.v1 = quantize(self.v1[..., :o, :], group_size=group_size, bits=bits)
            new.v2 = quantize(self.v2[..., :o, :], group_size=group_size, bits=bits)
            new.offset = self.offset
        return new


class MotifGroupedQuantizedKVCache(MotifGroupedKVCacheBase):
    """4-slot cache whose slots are MLX-affine triples ``(data, scales, biases)``."""

    def __init__(self, group_size: int = 64, bits: int = 8):
        self.k1 = self.k2 = self.v1 = self.v2 = None
        self.offset = 0
        self.group_size = group_size
        self.bits = bits

    def _slot_capacity(self, slot) -> int:
        return slot[0].shape[2]

    def _init_storage(self, B, H, n, D, dtype, device):
        el_per_int = 32 // self.bits
        return (
            torch.zeros((B, H, n, D // el_per_int), dtype=torch.uint32, device=device),
            torch.zeros((B, H, n, D // self.group_size), dtype=dtype, device=device),
            torch.zeros((B, H, n, D // self.group_size), dtype=dtype, device=device),
        )

    def _trim_slot(self, slot, prev: int):
        return tuple(x[..., :prev, :].contiguous() for x in slot)

    def _expand_slot(self, slot, fresh):
        return tuple(torch.cat([slot[i], fresh[i]], dim=-2) for i in range(3))

    def update_and_fetch_4(self, k1, k2, v1, v2):
        """Quantise + append, then return exact-length DEQUANTISED live slices
        (the dequant bridge of ``cache.py:448-465``)."""
        self._update_4(k1, k2, v1, v2)
        o = self.offset

        def _deq(slot):
            return dequantize(
                slot[0][..., :o, :], slot[1][..., :o, :], slot[2][..., :o, :],
                group_size=self.group_size, bits=self.bits,
            )

        return _deq(self.k1), _deq(self.k2), _deq(self.v1), _deq(self.v2)

    def update_and_fetch_4_quantized(self, k1, k2, v1, v2):
        """Quantise + append; return each slot's FULL capacity triple for
        ``sdpa_dual_v_q4`` (pass ``kv_len=offset``)."""
        self._update_4(k1, k2, v1, v2)
        return self.k1, self.k2, self.v1, self.v2

    def _update_4(self, k1, k2, v1, v2):
        self._assert_uniform_heads(k1, k2, v1, v2)
        B, H, S, D = k1.shape
        prev = self.offset
        self._grow(B, H, S, D, k1.dtype, k1.device)
        if _common._DISABLE:
            self._write_reference(k1, k2, v1, v2, prev)
        else:
            self._write_native(k1, k2, v1, v2, prev)
        self.offset += S

    def _write_reference(self, k1, k2, v1, v2, prev):
        """Reference structure: head-axis concat, one quantisation, 12 slice writes."""
        B, H, S, D = k1.shape
        fresh = torch.cat([k1, k2, v1, v2], dim=1)
        q_data, q_scales, q_biases = quantize_reference(fresh, self.group_size, self.bits)
        for i, slot in enumerate((self.k1, self.k2, self.v1, self.v2)):
            h0, h1 = i * H, (i + 1) * H
            slot[0][..., prev : prev + S, :] = q_data[:, h0:h1]
            slot[1][..., prev : prev + S, :] = q_scales[:, h0:h1]
            slot[2][..., prev : prev + S, :] = q_biases[:, h0:h1]

    def _write_native(self, k1, k2, v1, v2, prev):
        """All four slots in one ``motif_quant_write4`` dispatch."""
        B, H, S, D = k1.shape
        dev = _native.require_device(k1, k2, v1, v2, self.k1[0])
        dtype = k1.dtype
        srcs = []
        for t in (k1, k2, v1, v2):
            if t.dtype != dtype:
                raise TypeError("k1/k2/v1/v2 must share one dtype")
            srcs.append(_common.contiguous(t))
        slots = (self.k1, self.k2, self.v1, self.v2)
        vp4 = _native._VP4
        data = vp4(*[s[0].data_ptr() for s in slots])
        scales = vp4(*[s[1].data_ptr() for s in slots])
        biases = vp4(*[s[2].data_ptr() for s in slots])
        cap = self.k1[0].shape[2]
        _native.check(
            _native.lib().motif_quant_write4(
                *[t.data_ptr() for t in srcs], data, scales, biases, _native.dtype_code(dtype),
                B, H, S, D, cap, prev, self.bits, self.group_size, _native.stream_of(dev),
            )
        )

    @property
    def state(self):
        if self.offset == 0 or self.k1 is None:
            return self.k1, self.k2, self.v1, self.v2
        o = self.offset

        def _trim(slot):
            return tuple(x[..., :o, :] for x in slot)

        return _trim(self.k1), _trim(self.k2), _trim(self.v1), _trim(self.v2)

    @state.setter
    def state(self, v):
        self.k1, self.k2, self.v1, self.v2 = v

    @property
    def meta_state(self):
        return tuple(map(str, (self.offset, self.group_size, self.bits)))

    @meta_state.setter
    def meta_state(self, v):
        self.offset, self.group_size, self.bits = map(int, v)
