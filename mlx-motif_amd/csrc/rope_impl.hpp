// Non-traditional RoPE of one channel pair (i, i + D/2), shared by the
// rope_split4 kernel and the decode step that ropes its own inputs, so both
// round identically: angle = (pos * pos_scale) * theta^(-2i/D) in fp32 (the
// position is scaled first, as mx.fast.rope scales it; pos_scale is 1 for
// unscaled RoPE and 1 / factor for linear scaling, and multiplying by 1
// leaves the position exact), rotation with explicit fmas (no contraction
// left to the compiler).
#pragma once

namespace motif {

__device__ inline float rope_inv_freq(int p, int D, float log2_theta) {
  return exp2f(-(2.f * (float)p / (float)D) * log2_theta);
}
__device__ inline void rope_angle_inv(float inv_freq, int pos, float pos_scale, float& cs,
                                      float& sn) {
  sincosf(((float)pos * pos_scale) * inv_freq, &sn, &cs);
}
__device__ inline void rope_angle(int p, int D, int pos, float log2_theta, float pos_scale,
                                  float& cs, float& sn) {
  rope_angle_inv(rope_inv_freq(p, D, log2_theta), pos, pos_scale, cs, sn);
}

__device__ inline void rope_rotate(float x1, float x2, float cs, float sn, float& y1, float& y2) {
  y1 = fmaf(x1, cs, -(x2 * sn));
  y2 = fmaf(x2, cs, x1 * sn);
}

}  // namespace motif
