// RoPE + head split + 4-slot cache write of one attention step, in one
// launch (src/mlx_motif/model.py:580-594 rope on q and k, 620-629 the k1/k2
// and v1/v2 split and update_and_fetch_4, 669-679 the q1/q2 split).
//
// Inputs are the projection outputs as the reference reshapes them:
// q (B, S, HQ*D), k (B, S, HK*D), v (B, S, HV*D), row-major.  RoPE is the
// non-traditional form (rotate halves), angle = (pos0 + s) * theta^(-2i/D)
// for channel pairs (i, i + D/2), computed in fp32 and rounded once to T.
// Outputs:
//   q1 (B, q_groups*gr, S, D), q2 (B, q_groups, S, D)         rows 0..S-1
//   k1 (B, k_groups*kr, cap, D), k2 (B, k_groups, cap, D),
//   v1, v2 (B, k_groups, cap, D)                              rows row0..row0+S-1
// so with cap = the cache capacity and row0 = its offset the new rows land
// in the 4-slot cache directly.  One 16-lane group per (b, s, head) row;
// lane l holds channel pairs l*PPL .. l*PPL + PPL - 1 of both halves
// (PPL = D/32), moved with 8-byte accesses when the pointers allow.  (Sharing
// a position's angles across its heads, one group per 8 heads, measured
// slower: 12.1 against 9.7 us for a 512-row chunk, fewer rows in flight.)
#include "motif_common.hpp"
#include "rope_impl.hpp"

namespace motif {

struct RopeArgs {
  const void* q;
  const void* k;
  const void* v;
  void* q1;
  void* q2;
  void* k1;
  void* k2;
  void* v1;
  void* v2;
  int B, S, D;
  int q_groups, gr, k_groups, kr;
  int cap, row0, pos0;
  int origin_first;
  float log2_theta;
  float pos_scale;  // RoPE position scale (1, or 1 / factor for linear scaling)
  long rows_q, rows_k, rows_v;  // B * S * heads of each projection
};

// Rotates (or, for v, copies) pairs p and p + D/2 in fp32.
__device__ inline void rope_pair(float x1, float x2, int p, int D, int pos, bool rotate,
                                 float log2_theta, float pos_scale, float& y1, float& y2) {
  y1 = x1;
  y2 = x2;
  if (rotate) {
    float cs, sn;
    rope_angle(p, D, pos, log2_theta, pos_scale, cs, sn);
    rope_rotate(x1, x2, cs, sn, y1, y2);
  }
}

// VEC (16-bit T, PPL a multiple of 4, 8-byte aligned rows): 8-byte loads and
// stores of 4 values from each half.
template <typename T, int PPL, bool VEC>
__device__ inline void rope_row(const RopeArgs& a, const void* src, long src_row, void* dst,
                                long dst_row, int pos, bool rotate, int l) {
  const int D = a.D;
  const int H = D / 2;
  const long si = src_row * D;
  const long di = dst_row * D;
  if constexpr (VEC) {
    static_assert(sizeof(T) == 2 && PPL % 4 == 0, "4 16-bit values per access");
    const uint16_t* sp = (const uint16_t*)src;
    uint16_t* dp = (uint16_t*)dst;
#pragma unroll
    for (int c = 0; c < PPL; c += 4) {
      const int p0 = l * PPL + c;
      const uint2 w1 = *reinterpret_cast<const uint2*>(sp + si + p0);
      const uint2 w2 = *reinterpret_cast<const uint2*>(sp + si + H + p0);
      const uint32_t in1[2] = {w1.x, w1.y}, in2[2] = {w2.x, w2.y};
      uint32_t o1[2], o2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float y1[2], y2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float x1 = Elem<T>::to_f32((uint16_t)(e ? in1[h] >> 16 : in1[h] & 0xFFFFu));
          const float x2 = Elem<T>::to_f32((uint16_t)(e ? in2[h] >> 16 : in2[h] & 0xFFFFu));
          rope_pair(x1, x2, p0 + 2 * h + e, D, pos, rotate, a.log2_theta, a.pos_scale, y1[e],
                    y2[e]);
        }
        o1[h] = (uint32_t)Elem<T>::from_f32(y1[0]) | ((uint32_t)Elem<T>::from_f32(y1[1]) << 16);
        o2[h] = (uint32_t)Elem<T>::from_f32(y2[0]) | ((uint32_t)Elem<T>::from_f32(y2[1]) << 16);
      }
      *reinterpret_cast<uint2*>(dp + di + p0) = make_uint2(o1[0], o1[1]);
      *reinterpret_cast<uint2*>(dp + di + H + p0) = make_uint2(o2[0], o2[1]);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < PPL; ++t) {
    const int p = l * PPL + t;
    const float x1 = Elem<T>::load(src, si + p);
    const float x2 = Elem<T>::load(src, si + H + p);
    float y1, y2;
    rope_pair(x1, x2, p, D, pos, rotate, a.log2_theta, a.pos_scale, y1, y2);
    Elem<T>::store(dst, di + p, y1);
    Elem<T>::store(dst, di + H + p, y2);
  }
}

// One 16-lane group per (b, s, head) row of the concatenated projections
// [q rows | k rows | v rows].
template <typename T, int PPL, bool VEC>
__global__ void __launch_bounds__(256) rope_split4_kernel(RopeArgs a) {
  const int l = threadIdx.x & 15;
  const long total = a.rows_q + a.rows_k + a.rows_v;
  const long stride = (long)gridDim.x * 16;
  for (long r = (long)blockIdx.x * 16 + (threadIdx.x >> 4); r < total; r += stride) {
    if (r < a.rows_q) {  // q: (b, s, h) of B x S x HQ
      const int HQ = a.q_groups * (a.gr + 1);
      const long bs = r / HQ;
      const int h = (int)(r - bs * HQ);
      const int b = (int)(bs / a.S);
      const int s = (int)(bs - (long)b * a.S);
      int g, j;
      if (a.origin_first) {
        const int no = a.q_groups * a.gr;
        g = h < no ? h / a.gr : h - no;
        j = h < no ? h % a.gr : a.gr;
      } else {
        g = h / (a.gr + 1);
        j = h % (a.gr + 1);
      }
      if (j < a.gr) {
        const long dst = ((long)b * a.q_groups * a.gr + g * a.gr + j) * a.S + s;
        rope_row<T, PPL, VEC>(a, a.q, r, a.q1, dst, a.pos0 + s, true, l);
      } else {
        const long dst = ((long)b * a.q_groups + g) * a.S + s;
        rope_row<T, PPL, VEC>(a, a.q, r, a.q2, dst, a.pos0 + s, true, l);
      }
    } else if (r < a.rows_q + a.rows_k) {  // k: (b, s, h) of B x S x HK
      const long rk = r - a.rows_q;
      const int HK = a.k_groups * (a.kr + 1);
      const long bs = rk / HK;
      const int h = (int)(rk - bs * HK);
      const int b = (int)(bs / a.S);
      const int s = (int)(bs - (long)b * a.S);
      const int g = h / (a.kr + 1);
      const int j = h % (a.kr + 1);
      if (j < a.kr) {
        const long dst = ((long)b * a.k_groups * a.kr + g * a.kr + j) * a.cap + a.row0 + s;
        rope_row<T, PPL, VEC>(a, a.k, rk, a.k1, dst, a.pos0 + s, true, l);
      } else {
        const long dst = ((long)b * a.k_groups + g) * a.cap + a.row0 + s;
        rope_row<T, PPL, VEC>(a, a.k, rk, a.k2, dst, a.pos0 + s, true, l);
      }
    } else {  // v: (b, s, h) of B x S x 2*k_groups; head 2n -> v1[n], 2n+1 -> v2[n]
      const long rv = r - a.rows_q - a.rows_k;
      const int HV = 2 * a.k_groups;
      const long bs = rv / HV;
      const int h = (int)(rv - bs * HV);
      const int b = (int)(bs / a.S);
      const int s = (int)(bs - (long)b * a.S);
      const long dst = ((long)b * a.k_groups + h / 2) * a.cap + a.row0 + s;
      rope_row<T, PPL, VEC>(a, a.v, rv, (h & 1) ? a.v2 : a.v1, dst, 0, false, l);
    }
  }
}

template <typename T, bool VEC>
static int launch_rope(const RopeArgs& a, hipStream_t s) {
  const long total = a.rows_q + a.rows_k + a.rows_v;
  long blocks = (total + 15) / 16;
  const long cap = (long)device_cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  switch (a.D / 32) {  // pairs per lane = D / 32
    case 1: hipLaunchKernelGGL((rope_split4_kernel<T, 1, VEC && 1 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((rope_split4_kernel<T, 2, VEC && 2 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((rope_split4_kernel<T, 3, VEC && 3 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((rope_split4_kernel<T, 4, VEC && 4 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 5: hipLaunchKernelGGL((rope_split4_kernel<T, 5, VEC && 5 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((rope_split4_kernel<T, 6, VEC && 6 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 7: hipLaunchKernelGGL((rope_split4_kernel<T, 7, VEC && 7 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((rope_split4_kernel<T, 8, VEC && 8 % 4 == 0>), dim3(blocks), dim3(256), 0, s, a); break;
    default:
      set_error("rope_split4: head dim D=%d has no compiled variant (32..256 step 32)", a.D);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("rope_split4");
}

}  // namespace motif

using namespace motif;

extern "C" {

int motif_rope_split4_scaled(const void* q, const void* k, const void* v, void* q1, void* q2,
                             void* k1, void* k2, void* v1, void* v2, int dtype, int B, int S,
                             int q_groups, int gr, int k_groups, int kr, int D, int cap,
                             int row0, int pos0, float theta, float position_scale,
                             int origin_first, void* stream) {
  CallScope scope;
  clear_error();
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "rope_split4: unknown dtype code %d", dtype);
  MOTIF_REQUIRE(B >= 0 && S >= 0, "rope_split4: B and S must be >= 0");
  MOTIF_REQUIRE(q_groups >= 1 && gr >= 1 && k_groups >= 1 && kr >= 1,
                "rope_split4: q_groups, gr, k_groups, kr must be >= 1");
  MOTIF_REQUIRE(D > 0 && D % 32 == 0 && D <= 256, "rope_split4: D=%d must be 32..256 step 32",
                D);
  MOTIF_REQUIRE(row0 >= 0 && (long)row0 + S <= cap,
                "rope_split4: rows [%d, %d) must fit the destination capacity %d", row0,
                row0 + S, cap);
  MOTIF_REQUIRE(pos0 >= 0, "rope_split4: pos0=%d must be >= 0", pos0);
  MOTIF_REQUIRE(theta > 1.f, "rope_split4: theta must be > 1");
  MOTIF_REQUIRE(position_scale > 0.f && position_scale <= 3.4028234663852886e38f,
                "rope_split4: position_scale must be positive and finite");
  if (B == 0 || S == 0) return MOTIF_OK;
  MOTIF_REQUIRE(q && k && v && q1 && q2 && k1 && k2 && v1 && v2, "rope_split4: null pointer");
  RopeArgs a{};
  a.q = q; a.k = k; a.v = v;
  a.q1 = q1; a.q2 = q2; a.k1 = k1; a.k2 = k2; a.v1 = v1; a.v2 = v2;
  a.B = B; a.S = S; a.D = D;
  a.q_groups = q_groups; a.gr = gr; a.k_groups = k_groups; a.kr = kr;
  a.cap = cap; a.row0 = row0; a.pos0 = pos0;
  a.origin_first = origin_first != 0;
  a.log2_theta = log2f(theta);
  a.pos_scale = position_scale;
  a.rows_q = (long)B * S * q_groups * (gr + 1);
  a.rows_k = (long)B * S * k_groups * (kr + 1);
  a.rows_v = (long)B * S * 2 * k_groups;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)q1 | (uintptr_t)q2 |
                    (uintptr_t)k1 | (uintptr_t)k2 | (uintptr_t)v1 | (uintptr_t)v2) % 8 == 0;
  switch (dtype) {
    case MOTIF_F16: return vec ? launch_rope<half_t, true>(a, s) : launch_rope<half_t, false>(a, s);
    case MOTIF_BF16: return vec ? launch_rope<bf16_t, true>(a, s) : launch_rope<bf16_t, false>(a, s);
    default: return launch_rope<float, false>(a, s);
  }
}

int motif_rope_split4(const void* q, const void* k, const void* v, void* q1, void* q2, void* k1,
                      void* k2, void* v1, void* v2, int dtype, int B, int S, int q_groups, int gr,
                      int k_groups, int kr, int D, int cap, int row0, int pos0, float theta,
                      int origin_first, void* stream) {
  return motif_rope_split4_scaled(q, k, v, q1, q2, k1, k2, v1, v2, dtype, B, S, q_groups, gr,
                                  k_groups, kr, D, cap, row0, pos0, theta, 1.f, origin_first,
                                  stream);
}

}  // extern "C"
