"""HIP kernels of the Motif decode-attention hot path (gfx950).

Mirror of ``src/mlx_motif/kernels/__init__.py``: the same public names with
the same signatures, each backed by ``libmotif_hip`` and paired with a
``*_reference`` in torch ops.  ``MLX_MOTIF_DISABLE_KERNELS=1`` (read once at
import) routes every wrapper to its reference.

    attention.py — sdpa_dual_v, sdpa_dual_v_q4 (+ multi-row *_rows variants)
    gda.py       — gda_post, gda_post_split
    decode.py    — gda_decode_attention(_q4) (both dual-V passes +
                   gda_post_split in one call; the reference composes three)
    mlp.py       — polynorm, _dequant_probe (test helper)
    quant.py     — quantize / dequantize (MLX affine format of the KV cache)
    rope.py      — rope_split4 (RoPE + q/k/v head split + 4-slot cache write
                   in one launch; the reference uses rope() and reshapes)
    prefill.py   — gda_prefill_attention_from_proj (a layer's prefill chunk:
                   RoPE, cache write and both dual-V passes in one launch)
"""

from .attention import (
    sdpa_dual_v,
    sdpa_dual_v_q4,
    sdpa_dual_v_q4_reference,
    sdpa_dual_v_q4_rows,
    sdpa_dual_v_reference,
    sdpa_dual_v_rows,
)
from .decode import (
    gda_decode_attention,
    gda_decode_attention_from_proj,
    gda_decode_attention_q4_from_proj,
    gda_decode_attention_q4,
    gda_decode_attention_q4_reference,
    gda_decode_attention_reference,
)
from .gda import (
    gda_post,
    gda_post_reference,
    gda_post_split,
    gda_post_split_reference,
)
from .mlp import (
    _dequant_probe,  # noqa: F401  — test helper, deliberately not in __all__
    polynorm,
    polynorm_reference,
)
from .quant import dequantize, dequantize_reference, quantize, quantize_reference
from .prefill import gda_prefill_attention_from_proj, gda_prefill_attention_from_proj_reference
from .rope import rope_split4, rope_split4_reference

__all__ = [
    "polynorm",
    "polynorm_reference",
    "gda_post",
    "gda_post_reference",
    "gda_post_split",
    "gda_post_split_reference",
    "gda_decode_attention",
    "gda_decode_attention_reference",
    "gda_decode_attention_from_proj",
    "gda_decode_attention_q4_from_proj",
    "gda_decode_attention_q4",
    "gda_decode_attention_q4_reference",
    "sdpa_dual_v",
    "sdpa_dual_v_reference",
    "sdpa_dual_v_q4",
    "sdpa_dual_v_q4_reference",
    "sdpa_dual_v_rows",
    "sdpa_dual_v_q4_rows",
    "quantize",
    "quantize_reference",
    "dequantize",
    "dequantize_reference",
    "rope_split4",
    "rope_split4_reference",
    "gda_prefill_attention_from_proj",
    "gda_prefill_attention_from_proj_reference",
]
