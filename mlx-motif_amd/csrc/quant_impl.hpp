// Per-group MLX-affine quantisation shared by the quantiser, the 4-slot
// cache write and the fused decode step's append (quant.hip,
// sdpa_mfma_q.hpp).
//
// Mapping: each lane owns 8 consecutive values (16 bytes of fp16), so a
// group spans gs/8 lanes (4, 8 or 16) and its min/max is a DPP reduction
// inside one 16-lane row.  A lane emits one packed word (q4) or two (q8).
//
// Bit-exactness: the per-group arithmetic is IEEE fp32 with correctly
// rounded division, round-half-even rint and no contraction, in the order
// of MLX's CPU quantizer (see group_scale_bias below).
#pragma once

#include "motif_common.hpp"

namespace motif {

template <int LPG>
__device__ inline float group_min_lanes(float x) {
  if constexpr (LPG >= 2) x = fminf(x, dpp<kDppQuadXor1>(x));
  if constexpr (LPG >= 4) x = fminf(x, dpp<kDppQuadXor2>(x));
  if constexpr (LPG >= 8) x = fminf(x, dpp<kDppHalfMirror>(x));
  if constexpr (LPG >= 16) x = fminf(x, dpp<kDppMirror>(x));
  return x;
}

// Scale and bias of one group from its min and max (fp32 math of
// mx.quantize, affine mode):
//   scale = max((max - min) / n_bins, 1e-7); the side with the larger
//   magnitude is the "edge"; scale takes the sign that maps the edge to a
//   non-positive code q0 = rint(edge / scale); when q0 != 0 the scale is
//   refit so the edge is exactly representable (scale = edge / q0) and the
//   bias is the edge, else bias = 0.
__device__ inline void group_scale_bias(float w_min, float w_max, float n_bins, float& scale,
                                        float& bias) {
#pragma clang fp contract(off)
  const float eps = 1e-7f;
  float s = fmaxf((w_max - w_min) / n_bins, eps);
  const bool side = fabsf(w_min) > fabsf(w_max);
  s = side ? s : -s;
  const float edge = side ? w_min : w_max;
  const float q0 = rintf(edge / s);
  float b = 0.f;
  if (q0 != 0.f) {
    s = edge / q0;
    b = edge;
  }
  scale = s;
  bias = b;
}

__device__ inline uint32_t quant_code(float w, float scale, float bias, float n_bins) {
#pragma clang fp contract(off)
  float q = rintf((w - bias) / scale);
  q = fminf(fmaxf(q, 0.f), n_bins);
  return (uint32_t)q;
}

// Load 8 consecutive values of type T as fp32.
template <typename T>
__device__ inline void load8(const void* base, long idx, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    uint4 w = *reinterpret_cast<const uint4*>((const uint16_t*)base + idx);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<T>::get(ws, i);
  } else {
    const float4* p = reinterpret_cast<const float4*>((const float*)base + idx);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

// Quantise the 8 values of this lane; every lane of the LPG-lane group
// computes the same scale/bias.  Packs into words[0] (q4) or words[0..1] (q8).
template <int BITS, int LPG>
__device__ inline void quantize8(const float (&v)[8], uint32_t (&words)[2], float& scale,
                                 float& bias) {
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
  mn = group_min_lanes<LPG>(mn);
  mx = group_max<LPG>(mx);
  const float n_bins = (float)((1 << BITS) - 1);
  group_scale_bias(mn, mx, n_bins, scale, bias);
  words[0] = 0u;
  words[1] = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t u = quant_code(v[i], scale, bias, n_bins);
    if constexpr (BITS == 4) {
      words[0] |= u << (4 * i);
    } else {
      words[i >> 2] |= u << (8 * (i & 3));
    }
  }
}

template <int BITS>
__device__ inline void store_words(uint32_t* dst, long widx, const uint32_t (&w)[2]) {
  if constexpr (BITS == 4) {
    dst[widx] = w[0];
  } else {
    *reinterpret_cast<uint2*>(dst + widx) = make_uint2(w[0], w[1]);
  }
}

}  // namespace motif
