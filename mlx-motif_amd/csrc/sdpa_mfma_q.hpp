// Matrix-core formulation of split-KV dual-V decode over the packed
// MLX-affine cache (q4 / q8, head_dim 128, fp16 scales and biases).
//
// Dequantised value = s * u + b with u the unsigned code, (s, b) per row and
// group of gs channels.  Both products are split so that the matrix cores
// only ever see exact small integers u (as fp16):
//
//   score(h, r) = sum_g s_K(r,g) * [sum_{c in g} q_h[c] u_K(r,c)]
//                 + b_K(r,g) * [sum_{c in g} q_h[c]]
//     The bracket is one 16x16x32 MFMA sum per k-step with the groups kept
//     apart on the MFMA's spare columns: column n = h + GC*g holds q_h on
//     the channels of group g and zeros elsewhere.  The group scale and bias
//     are applied in the C layout (lane l: rows 4*(l/16)+r, column l%16) and
//     the group columns of one head are summed with DPP row rotations.
//   o(h, c) = sum_r u_V(r,c) * [p(h,r) s_V(r,g(c))] + sum_r p(h,r) b_V(r,g(c))
//     The bracket is the B operand of V^T . W^T (16x16x16 MFMA, column
//     h + GC*g carries p * s_V of group g); the bias term is a per-lane fp32
//     sum folded in at the end.
//
// Codes become fp16 with the exponent trick: a code placed in the mantissa
// of 1024.0 (0x6400) reads as 1024 + u (or 1024 + 16u for the high nibble of
// a byte), and one packed fp16 add or fma recovers u exactly.  V^T fragments
// (4 rows x 1 channel per lane) come from one code word per row, paired
// across rows with v_perm_b32.  Everything else (split plan, online softmax
// in log2 units, workgroup epilogue) matches the fp16-cache kernel.
#pragma once

#include "sdpa_mfma.hpp"

namespace motif {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ inline half2_t as_h2(uint32_t x) { return __builtin_bit_cast(half2_t, x); }

// 1024 + u  ->  u
__device__ inline half2_t sub1024(uint32_t x) {
  return as_h2(x) - half2_t{(_Float16)1024.f, (_Float16)1024.f};
}
// 1024 + 16u  ->  u
__device__ inline half2_t sub1024_hi(uint32_t x) {
  return as_h2(x) * half2_t{(_Float16)0.0625f, (_Float16)0.0625f} -
         half2_t{(_Float16)64.f, (_Float16)64.f};
}
__device__ inline uint32_t h2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// 8 channels of one q4 word as exact fp16 codes, in the order
// [0, 4, 1, 5, 2, 6, 3, 7] (q4_order): k-operand order of the K fragments.
__device__ inline half8_t q4_word_codes(uint32_t w) {
  const uint32_t w8 = w >> 8;
  const half2_t y0 = sub1024((w & 0x000F000Fu) | 0x64006400u);
  const half2_t y1 = sub1024_hi((w & 0x00F000F0u) | 0x64006400u);
  const half2_t y2 = sub1024((w8 & 0x000F000Fu) | 0x64006400u);
  const half2_t y3 = sub1024_hi((w8 & 0x00F000F0u) | 0x64006400u);
  return half8_t{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}
__host__ __device__ constexpr int q4_order(int j) { return (j & 1) ? 4 + (j >> 1) : (j >> 1); }

// 8 channels of two q8 words (4 each) as exact fp16 codes, natural order.
__device__ inline half8_t q8_words_codes(uint32_t w0, uint32_t w1) {
  const uint32_t magic = 0x64646464u;  // byte 0x64: high byte of 1024.0
  const half2_t y0 = sub1024(__builtin_amdgcn_perm(magic, w0, 0x04010400u));
  const half2_t y1 = sub1024(__builtin_amdgcn_perm(magic, w0, 0x04030402u));
  const half2_t y2 = sub1024(__builtin_amdgcn_perm(magic, w1, 0x04010400u));
  const half2_t y3 = sub1024(__builtin_amdgcn_perm(magic, w1, 0x04030402u));
  return half8_t{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}

// Byte k of words a (low half) and b (high half), zero-extended to 16 bits.
__device__ inline uint32_t pair_bytes(uint32_t a, uint32_t b, int k) {
  const uint32_t sel = (uint32_t)k | (0x0Cu << 8) | ((uint32_t)(4 + k) << 16) | (0x0Cu << 24);
  return __builtin_amdgcn_perm(b, a, sel);
}

// V^T fragment: code i of the lane's word in rows r0..r3, as exact fp16.
template <int BITS>
__device__ inline half4_t v_codes(const uint32_t (&w)[4], int i) {
  if constexpr (BITS == 4) {
    const int k = i >> 1;
    const uint32_t x01 = pair_bytes(w[0], w[1], k);
    const uint32_t x23 = pair_bytes(w[2], w[3], k);
    half2_t lo, hi;
    if (i & 1) {
      lo = sub1024_hi((x01 & 0x00F000F0u) | 0x64006400u);
      hi = sub1024_hi((x23 & 0x00F000F0u) | 0x64006400u);
    } else {
      lo = sub1024((x01 & 0x000F000Fu) | 0x64006400u);
      hi = sub1024((x23 & 0x000F000Fu) | 0x64006400u);
    }
    return half4_t{lo.x, lo.y, hi.x, hi.y};
  } else {
    const half2_t lo = sub1024(pair_bytes(w[0], w[1], i) | 0x64006400u);
    const half2_t hi = sub1024(pair_bytes(w[2], w[3], i) | 0x64006400u);
    return half4_t{lo.x, lo.y, hi.x, hi.y};
  }
}

// Rotate within 16-lane DPP rows.
template <int K>
__device__ inline float row_ror(float x) {
  return dpp<0x120 + K>(x);
}

// Sum over the columns n, n+GC, n+2GC, ... of one 16-lane row (the group
// columns of one head); every lane of the residue class gets the sum.
template <int GC>
__device__ inline float sum_group_columns(float x) {
  if constexpr (GC <= 8) x += row_ror<8>(x);
  if constexpr (GC <= 4) x += row_ror<4>(x);
  if constexpr (GC <= 2) x += row_ror<2>(x);
  if constexpr (GC <= 1) x += row_ror<1>(x);
  return x;
}

// fp16 scale/bias of rows row0..row0+3 (row0 % 4 == 0) for the lane's group
// gsel, NG groups per row.  The 4*NG halves of the four rows are contiguous
// (8, 16 or 32 bytes) and read with one or two vector loads; the lane's group
// is then picked with compile-time indexes only (selects, no dynamic register
// indexing).
template <int NG>
struct LaneScales {
  float v[4];
  __device__ inline void load(const uint16_t* base, long row0, bool full, int r_end, int gsel) {
    const uint16_t* p = base + row0 * NG;
    uint32_t w[2 * NG];
    if (full) {
      if constexpr (NG == 4) {
        const uint4 x = ld_stream4(p);
        const uint4 y = ld_stream4(p + 8);
        w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
        w[4] = y.x; w[5] = y.y; w[6] = y.z; w[7] = y.w;
      } else if constexpr (NG == 2) {
        const uint4 x = ld_stream4(p);
        w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
      } else {
        const uint2 x = ld_stream2(p);
        w[0] = x.x; w[1] = x.y;
      }
    } else {
      // Tail tile: only rows below r_end exist; the others read as 0.
#pragma unroll
      for (int i = 0; i < 2 * NG; ++i) {
        const int r0 = (2 * i) / NG, r1 = (2 * i + 1) / NG;
        const uint32_t lo = (row0 + r0 < r_end) ? p[2 * i] : 0u;
        const uint32_t hi = (row0 + r1 < r_end) ? p[2 * i + 1] : 0u;
        w[i] = lo | (hi << 16);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t bits = 0;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int idx = r * NG + g;
        const uint32_t hb = (idx & 1) ? (w[idx >> 1] >> 16) : (w[idx >> 1] & 0xFFFFu);
        bits = (g == gsel) ? hb : bits;
      }
      v[r] = Elem<half_t>::to_f32((uint16_t)bits);
    }
  }
};

template <int BITS, int GS, int GC, int NW, int U>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
sdpa_mfma_q_kernel(SdpaArgs a) {
  using T = half_t;
  constexpr int D = 128;
  constexpr int NG = D / GS;                    // scale groups per row
  constexpr int WPR = D * BITS / 32;            // code words per row
  constexpr int KW = WPR / 4;                   // K words per lane (32 channels)
  constexpr int VW = WPR / 16;                  // V words per lane per row (8 channels)
  static_assert(GC * NG <= 16, "heads x groups ride the 16 MFMA columns");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int blk = lane >> 4;

  const int units = a.B * a.Hkv * a.nchunk;
  const int unit = blockIdx.x % units;
  const int split = blockIdx.x / units;
  const int chunk = unit % a.nchunk;
  const int bk = unit / a.nchunk;
  const int b = bk / a.Hkv;
  const int kvh = bk % a.Hkv;
  const int vh0 = chunk * GC;
  const int nvh = min(GC, a.GV - vh0);
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q + vh0;

  const int h = col % GC;       // head of this column
  const int grp = col / GC;     // scale group of this column
  const bool col_used = grp < NG && h < nvh;
  const int gsel = grp < NG ? grp : 0;  // group whose scales this lane reads
  int max_lim = 0;
  for (int g = 0; g < nvh; ++g) max_lim = max(max_lim, vhead_limit(a, vh0 + g));
  const int lim = h < nvh ? vhead_limit(a, vh0 + h) : 0;
  const int r_begin = split * a.rows_per_split;
  const int r_end = min(r_begin + a.rows_per_split, max_lim);

  // Q^T (B of the K MFMA): lane (col, blk), k-step s covers channels
  // 32*blk + 8*s + order[j]; nonzero only where the channel's group is the
  // column's group.  qsum: sum of q_h over the column's group.
  half8_t qb[4];
  float qsum = 0.f;
  {
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (h < nvh ? h : 0)) * D + 32 * blk;
    const bool mine = col_used && (32 * blk) / GS == grp;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = 8 * s + (BITS == 4 ? q4_order(j) : j);
        const _Float16 v = mine ? __builtin_bit_cast(_Float16, qp[c]) : (_Float16)0.f;
        qb[s][j] = v;
        qsum += (float)v;
      }
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
  }

  const long hbase = (long)bk * a.kv_cap;  // first cache row of this KV head
  const uint32_t* kd = a.kd + hbase * WPR;
  const uint32_t* v1d = a.v1d + hbase * WPR;
  const uint32_t* v2d = a.v2d + hbase * WPR;
  const uint16_t* ks = (const uint16_t*)a.ks + hbase * NG;
  const uint16_t* kb = (const uint16_t*)a.kb + hbase * NG;
  const uint16_t* v1s = (const uint16_t*)a.v1s + hbase * NG;
  const uint16_t* v1b = (const uint16_t*)a.v1b + hbase * NG;
  const uint16_t* v2s = (const uint16_t*)a.v2s + hbase * NG;
  const uint16_t* v2b = (const uint16_t*)a.v2b + hbase * NG;

  floatx4 acc1[8], acc2[8], accl;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc1[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  accl = floatx4{0.f, 0.f, 0.f, 0.f};
  float beta1 = 0.f, beta2 = 0.f;  // sum_r p * b_V over this lane's rows
  float m_run = kNegSentinel;
  const half4_t ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};

  for (int base = r_begin + wave * 16; base < r_end; base += NW * 16 * U) {
    uint32_t kw[U][KW];
    uint32_t v1w[U][4][VW], v2w[U][4][VW];
    LaneScales<NG> sk[U], bk_[U], s1[U], b1[U], s2[U], b2[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t0 = base + u * NW * 16;
      const int krow = t0 + col;
      if (krow < r_end) {
        load_words_stream<KW>(kw[u], kd + (long)krow * WPR + KW * blk);
      } else {
#pragma unroll
        for (int i = 0; i < KW; ++i) kw[u][i] = 0u;
      }
      const int row0 = t0 + 4 * blk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + r;
        if (row < r_end) {
          load_words_stream<VW>(v1w[u][r], v1d + (long)row * WPR + VW * col);
          load_words_stream<VW>(v2w[u][r], v2d + (long)row * WPR + VW * col);
        } else {
#pragma unroll
          for (int i = 0; i < VW; ++i) { v1w[u][r][i] = 0u; v2w[u][r][i] = 0u; }
        }
      }
      const bool full = row0 + 3 < r_end;
      sk[u].load(ks, row0, full, r_end, gsel);
      bk_[u].load(kb, row0, full, r_end, gsel);
      s1[u].load(v1s, row0, full, r_end, gsel);
      b1[u].load(v1b, row0, full, r_end, gsel);
      s2[u].load(v2s, row0, full, r_end, gsel);
      b2[u].load(v2b, row0, full, r_end, gsel);
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t0 = base + u * NW * 16;
      floatx4 sacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        half8_t ka;
        if constexpr (BITS == 4) {
          ka = q4_word_codes(kw[u][s]);
        } else {
          ka = q8_words_codes(kw[u][2 * s], kw[u][2 * s + 1]);
        }
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[s], sacc, 0, 0, 0);
      }
      float sc[4];
      float mx = kNegSentinel;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = col_used ? fmaf(sk[u].v[r], sacc[r], bk_[u].v[r] * qsum) : 0.f;
        t = sum_group_columns<GC>(t);
        const int row = t0 + 4 * blk + r;
        const bool ok = row < r_end && row < lim;
        sc[r] = ok ? t * a.qscale : kNegSentinel;
        mx = fmaxf(mx, sc[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (__ballot(mx > m_run) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float fac = fast_exp2(m_run - m_new);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc1[j] *= fac;
          acc2[j] *= fac;
        }
        accl *= fac;
        beta1 *= fac;
        beta2 *= fac;
        m_run = m_new;
      }
      half4_t pb, w1, w2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (col_used && sc[r] > kNegSentinel) ? fast_exp2(sc[r] - m_run) : 0.f;
        pb[r] = (_Float16)p;
        w1[r] = (_Float16)(p * s1[u].v[r]);
        w2[r] = (_Float16)(p * s2[u].v[r]);
        beta1 = fmaf(p, b1[u].v[r], beta1);
        beta2 = fmaf(p, b2[u].v[r], beta2);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t x1[4], x2[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x1[r] = v1w[u][r][BITS == 4 ? 0 : (i >> 2)];
          x2[r] = v2w[u][r][BITS == 4 ? 0 : (i >> 2)];
        }
        const half4_t a1 = v_codes<BITS>(x1, BITS == 4 ? i : (i & 3));
        const half4_t a2 = v_codes<BITS>(x2, BITS == 4 ? i : (i & 3));
        acc1[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a1, w1, acc1[i], 0, 0, 0);
        acc2[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a2, w2, acc2[i], 0, 0, 0);
      }
      accl = __builtin_amdgcn_mfma_f32_16x16x16f16(ones, pb, accl, 0, 0, 0);
    }
  }

  // Bias terms: sum the four row blocks of each column.
  beta1 += __shfl_xor(beta1, 16);
  beta1 += __shfl_xor(beta1, 32);
  beta2 += __shfl_xor(beta2, 16);
  beta2 += __shfl_xor(beta2, 32);

  // acc[i][r] of lane (col, blk) is channel 8*(4*blk + r) + i for head h; it
  // is valid where that channel's group is the column's group, i.e. where
  // the row block's 32 channels belong to group grp.
  __shared__ __attribute__((aligned(16))) float lds_o[NW][GC][2 * D + kLdsPad];
  __shared__ float lds_m[NW][GC];
  __shared__ float lds_l[NW][GC];
  if (col_used && (32 * blk) / GS == grp) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ch = 8 * (4 * blk + r);
      *reinterpret_cast<float4*>(&lds_o[wave][h][ch]) =
          make_float4(acc1[0][r] + beta1, acc1[1][r] + beta1, acc1[2][r] + beta1,
                      acc1[3][r] + beta1);
      *reinterpret_cast<float4*>(&lds_o[wave][h][ch + 4]) =
          make_float4(acc1[4][r] + beta1, acc1[5][r] + beta1, acc1[6][r] + beta1,
                      acc1[7][r] + beta1);
      *reinterpret_cast<float4*>(&lds_o[wave][h][D + ch]) =
          make_float4(acc2[0][r] + beta2, acc2[1][r] + beta2, acc2[2][r] + beta2,
                      acc2[3][r] + beta2);
      *reinterpret_cast<float4*>(&lds_o[wave][h][D + ch + 4]) =
          make_float4(acc2[4][r] + beta2, acc2[5][r] + beta2, acc2[6][r] + beta2,
                      acc2[7][r] + beta2);
    }
  }
  if (col < GC && h < nvh && blk == 0) {
    lds_m[wave][h] = m_run;
    lds_l[wave][h] = accl[0];
  }
  __syncthreads();
  wg_epilogue<T, D, GC, NW>(a, lds_o, lds_m, lds_l, qrow0, nvh, split, unit);
}

// Packed cache, head_dim 128, fp16 scales: heads x groups <= 16 columns.
// Two tiles in flight per wave, except q8 with 32-channel groups, whose
// twelve scale vectors per tile would spill.
template <int BITS, int GS>
int launch_sdpa_mfma_q_gs(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t st) {
  constexpr int NG = 128 / GS;
  constexpr int U = (BITS == 8 && GS == 32) ? 1 : 2;
  switch (gc) {
    case 1:
      if (waves == 8) hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 1, 8, U>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 1, 4, U>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 2:
      if (waves == 8) hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 2, 8, U>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 2, 4, U>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 4:
      if (waves == 8) hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 4, 8, U>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 4, 4, U>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 8:
      if constexpr (8 * NG <= 16) {
        hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 8, 4, U>), dim3(nblocks), dim3(256), 0, st, a);
        break;
      }
      [[fallthrough]];
    default:
      set_error("sdpa_dual_v_q: no MFMA variant for %d heads per workgroup", gc);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("sdpa_dual_v_q (mfma)");
}

inline int launch_sdpa_mfma_q(const SdpaArgs& a, int bits, int gs, int gc, int waves, int nblocks,
                              hipStream_t st) {
  if (bits == 4) {
    if (gs == 32) return launch_sdpa_mfma_q_gs<4, 32>(a, gc, waves, nblocks, st);
    if (gs == 64) return launch_sdpa_mfma_q_gs<4, 64>(a, gc, waves, nblocks, st);
    return launch_sdpa_mfma_q_gs<4, 128>(a, gc, waves, nblocks, st);
  }
  if (gs == 32) return launch_sdpa_mfma_q_gs<8, 32>(a, gc, waves, nblocks, st);
  if (gs == 64) return launch_sdpa_mfma_q_gs<8, 64>(a, gc, waves, nblocks, st);
  return launch_sdpa_mfma_q_gs<8, 128>(a, gc, waves, nblocks, st);
}

}  // namespace motif
