// Packed-cache (q4 / q8 MLX-affine, head_dim 128, fp16 scales) split-KV
// dual-V decode on the matrix cores, processing 32 KV rows (two 16-row tiles)
// per step.
//
// Codes enter the MFMAs as fp16 subnormals.  A code u placed in the low
// mantissa bits of a zero-exponent half is the value u * 2^-24 (or
// 16u * 2^-24 for the high nibble of a byte), so one AND turns a packed word
// into two MFMA operands: no bias pattern to OR in and no subtraction.  The
// matrix cores take subnormal fp16 inputs at full precision (products are
// exact in fp32), and the 2^24 / 2^20 factors are folded into constants:
//
//   score(h, r) = sum_g s_K(r,g) * [sum_{c in g} q_h[c] u_K(r,c)] + b_K(r,g) * qsum_h(g)
//     q4: the low nibbles of the lane's four K words (channels in the order
//     lo_k) and the high nibbles (hi_k) form separate k-steps, accumulated in
//     two chains t_lo = sum q u 2^-24 and t_hi = sum q 16u 2^-24, so
//     sum q u = 2^24 (t_lo + t_hi / 16).  q8: bytes 0/2 and 1/3 of a word,
//     one chain.  Column n = NG*h + g holds q_h on the channels of scale
//     group g (zeros elsewhere); the group columns of a head meet through
//     DPP quad permutes.
//   o(h, c) = sum_r u_V(r,c) [p(h,r) s_V(r,g(c))] + sum_r p(h,r) b_V(r,g(c))
//     V^T . W^T on 16x16x32 MFMAs over a tile pair: k = 8*blk + j is row
//     4*blk + j of the first tile (j < 4) or row 4*blk + j - 4 of the second,
//     which is where the C layout of the two score tiles leaves each lane's
//     softmax weights, so P never moves between lanes.  The V^T operand of
//     channel 8*col + i takes code i of the lane's row words, paired across
//     rows with one v_perm_b32 (a byte per half).  q4: channel 2b (the low
//     nibble of byte b) masks it to u; channel 2b + 1 takes the whole byte
//     u + 16u' unmasked, and the epilogue recovers the high nibble's sum as
//     the difference of the two accumulators (one AND fewer per operand
//     dword; every product stays exact and the difference carries one fp32
//     rounding of a sum of similar size).
//
// Softmax: log2 units, one running-max update per pair (lazy rescaling with
// the packed kernel's slack), cross-row maxima with v_permlane16/32_swap,
// exp2 of fma(t, qscale', -m); rows past a column's limit are masked only
// in the pair that crosses it.  The workgroup epilogue is shared with the
// other split-KV kernels.
//
// bf16 activations (T = bf16_t: q, scales, biases and y in bf16) run the same
// fp16 matrix-core products: q is converted to fp16 once per workgroup after
// a power-of-two scaling per head that keeps its largest element below 2^15
// (exact; the factor is folded into that head's softmax scale), the V scales
// are converted to fp16 as they are staged in LDS (exact in fp16's normal
// range), and the K scale and both bias terms are taken in fp32.
#pragma once

#include "sdpa_mfma_q.hpp"

namespace motif {

// Sum over the NG adjacent group columns of a head (quad permutes); both
// partners add the same two operands, so every column gets the same bits.
template <int NG>
__device__ inline float sum_adjacent_groups(float x) {
  if constexpr (NG >= 2) x += dpp<kDppQuadXor1>(x);
  if constexpr (NG >= 4) x += dpp<kDppQuadXor2>(x);
  return x;
}

// Channel (within the lane's 32-channel block) of element j of k-step s of
// the K operand.  q4: steps 0/1 hold the low nibbles of words 0-1 / 2-3, steps
// 2/3 their high nibbles; a word w gives (w & 0x000F000F) = nibbles 0 and 4,
// ((w >> 8) & 0x000F000F) = nibbles 2 and 6.  q8: step s holds words 2s, 2s+1
// as bytes (0, 2), (1, 3) of each.
template <int BITS>
__host__ __device__ constexpr int qpair_k_channel(int s, int j) {
  if constexpr (BITS == 4) {
    const int lo[4] = {0, 4, 2, 6};
    return 16 * (s & 1) + 8 * (j / 4) + lo[j % 4] + (s >> 1);
  } else {
    const int b[4] = {0, 2, 1, 3};
    return 8 * s + 4 * (j / 4) + b[j % 4];
  }
}

// Raw loads of one 32-row pair as one lane needs them (nothing consumed at
// load time, so the whole pair is in flight together).
//   k[T][KW]         K words of row t_T + col, channels 32*blk .. 32*blk + 31
//   v1/v2[T][4][VW]  V words of rows t_T + 4*blk + r, channels 8*col .. +7
//   s[t]             word L of the pair's rows of tensor t (K scales, K
//                    biases, V1 scales, V1 biases, V2 scales, V2 biases) in
//                    lane L: rows r0 + L (NG = 2, L < 32) or r0 + 2L, +1
//                    (NG = 1, L < 16)
// Every lane of a 16-lane row needs the same scale rows, so each tensor's
// words for the pair arrive in one 32-bit load and reach the lanes through
// LDS at compute time, instead of sitting in registers 16 times over while
// the loads are in flight.
template <int BITS>
struct QPair {
  static constexpr int WPR = 128 * BITS / 32;
  static constexpr int KW = WPR / 4;
  static constexpr int VW = WPR / 16;
  uint32_t k[2][KW];
  uint32_t v1[2][4][VW];
  uint32_t v2[2][4][VW];
  uint32_t s[6];
};

// Packed cache, head_dim 128, fp16 scales; heads x groups <= 16 columns.
// GC heads per workgroup (column n = NG*h + g), NW waves, POL cache policy
// (cached when several head chunks read the same rows).
template <int BITS, int GS, int GC, int NW, int POL = kCachePolicyStream, typename E = half_t>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
sdpa_qpair_kernel(SdpaArgs a) {
  constexpr bool kBf16 = std::is_same<E, bf16_t>::value;
  constexpr int D = 128;
  constexpr int NG = D / GS;
  static_assert(GC * NG <= 16, "heads x groups ride the 16 MFMA columns");
  static_assert(NG == 1 || NG == 2, "group sizes 64 and 128");
  using Pair = QPair<BITS>;
  constexpr int SWT = 16 * NG;  // scale words of one tensor for a pair
  constexpr int SLANES = SWT;   // lanes that load them
  constexpr int WPR = Pair::WPR;
  constexpr int KW = Pair::KW;
  constexpr int VW = Pair::VW;
  constexpr float kSlack = BITS == 4 ? 2.f : 6.f;  // see sdpa_mfma_q_kernel
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int blk = lane >> 4;

  int unit, split;
  if (!sdpa_block_coords(a, blockIdx.x, unit, split)) return;  // grid padding
  const int chunk = unit % a.nchunk;
  const int bk = unit / a.nchunk;
  const int b = bk / a.Hkv;
  const int kvh = bk % a.Hkv;
  const int vh0 = chunk * GC;
  const int nvh = min(GC, a.GV - vh0);
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q + vh0;

  const int hh = col / NG;  // head of this column
  const int g = col % NG;   // scale group of this column
  const bool used = col < GC * NG && hh < nvh;
  const int lim = used ? vhead_limit(a, vh0 + hh) : 0;
  int max_lim, min_lim;
  vhead_limit_range(a, vh0, nvh, min_lim, max_lim);
  // v_perm selector keeping half g of two (row, group) words: NG = 2.
  const uint32_t sel = g ? 0x07060302u : 0x05040100u;

  // Rows are dealt to the splits in blocks of NW 32-row pairs, round robin:
  // pair k of wave w in split s is pair (k * nsplit + s) * NW + w of the KV
  // head.  Resources cover rows [0, max_lim): rows past them read 0 (codes,
  // scales and biases), and are masked in the pair that crosses the limit.
  const int ns = a.nsplit;
  auto pair_row = [&](int k) { return 32 * ((k * ns + split) * NW + wave); };
  const long hrow0 = (long)bk * a.kv_cap;
  const unsigned dbytes = (unsigned)(max_lim * WPR * 4);
  const auto rk = stream_rsrc(a.kd + hrow0 * WPR, dbytes);
  const auto rv1 = stream_rsrc(a.v1d + hrow0 * WPR, dbytes);
  const auto rv2 = stream_rsrc(a.v2d + hrow0 * WPR, dbytes);
  // Scale words: one row (NG = 2) or two rows (NG = 1) each, so the
  // resources end at max_lim, rounded up to even rows for NG = 1 (inside the
  // cache: cap % 4 == 0, checked on the host); the pair crossing max_lim
  // zeroes that odd row, which may be unwritten padding.
  const unsigned sbytes = (unsigned)((NG == 1 ? (max_lim + 1) & ~1 : max_lim) * NG * 2);
  // Lanes past SLANES read out of range (0, no memory access).
  const unsigned soff_lane = lane < SLANES ? 4u * (unsigned)lane : 0x80000000u;
  const __amdgpu_buffer_rsrc_t rs[6] = {
      stream_rsrc((const uint16_t*)a.ks + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.kb + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1b + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2b + hrow0 * NG, sbytes)};

  auto load_pair = [&](Pair& P, int k) {
    const unsigned r0 = (unsigned)pair_row(k);
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      const unsigned t0 = r0 + 16u * T;
      const unsigned koff = ((t0 + col) * WPR + KW * blk) * 4u;
#pragma unroll
      for (int i = 0; i < KW; i += 4) {
        const uint4 x = bload4<POL>(rk, koff + 4u * i);
        P.k[T][i] = x.x; P.k[T][i + 1] = x.y; P.k[T][i + 2] = x.z; P.k[T][i + 3] = x.w;
      }
      const unsigned vrow = t0 + 4u * blk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned voff = ((vrow + r) * WPR + VW * col) * 4u;
        if constexpr (VW == 1) {
          P.v1[T][r][0] = bload1<POL>(rv1, voff);
          P.v2[T][r][0] = bload1<POL>(rv2, voff);
        } else {
          const uint2 x1 = bload2<POL>(rv1, voff);
          const uint2 x2 = bload2<POL>(rv2, voff);
          P.v1[T][r][0] = x1.x; P.v1[T][r][1] = x1.y;
          P.v2[T][r][0] = x2.x; P.v2[T][r][1] = x2.y;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 6; ++t) P.s[t] = bload1<POL>(rs[t], r0 * NG * 2u + soff_lane);
  };

  // Q^T (B operand of the K MFMAs): lane (col, blk), k-step s, element j is
  // channel 32*blk + qpair_k_channel(s, j) of head hh, or 0 where that
  // channel is outside group g (or the column is unused).  qsum: sum of q
  // over the column's group, times 2^-24 (the codes' scale).
  int npair = 0;  // pairs of this wave
  while (pair_row(npair) < max_lim) ++npair;
  Pair P0, P1;
  load_pair(P0, 0);  // issued before q, so their latencies overlap
  half8_t qb[4];
  float qs;
  int q_exp = 0;  // bf16: this head's q was scaled by 2^-q_exp
  {
    const bool mine = used && (32 * blk) / GS == g;
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (used ? hh : 0)) * D + 32 * blk;
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 x = *reinterpret_cast<const uint4*>(qp + 8 * i);
      raw[4 * i] = x.x; raw[4 * i + 1] = x.y; raw[4 * i + 2] = x.z; raw[4 * i + 3] = x.w;
    }
    if constexpr (kBf16) {
      // Head scale 2^-e with e the smallest >= 0 that brings the head's
      // largest |q| below 2^15 (the four lanes of a column hold the head's
      // 128 channels), then q * 2^-e as fp16 pairs.
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        mx = fmaxf(mx, fmaxf(fabsf(pair_lo_f32<E>(raw[i])), fabsf(pair_hi_f32<E>(raw[i]))));
      mx = rows4_max(mx);
      const int ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFFu) - 127;
      q_exp = ex > 14 ? ex - 14 : 0;  // 0 for zero, subnormal and small heads
      const float f = __builtin_bit_cast(float, (uint32_t)(127 - q_exp) << 23);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        raw[i] = f16_pair(pair_lo_f32<E>(raw[i]) * f, pair_hi_f32<E>(raw[i]) * f);
    }
    float sum = 0.f;
    const half2_t one2 = half2_t{(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) sum = __builtin_amdgcn_fdot2(as_h2(raw[i]), one2, sum, false);
    qs = rows4_sum(mine ? sum : 0.f) * 0x1p-24f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint32_t w[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int c0 = qpair_k_channel<BITS>(s, 2 * v);
        const int c1 = qpair_k_channel<BITS>(s, 2 * v + 1);
        // half c0 % 2 of raw[c0 / 2] into the low half, half c1 % 2 of
        // raw[c1 / 2] into the high half
        const uint32_t sel_q = ((c0 & 1) ? 0x0302u : 0x0100u) | ((c1 & 1) ? 0x07060000u : 0x05040000u);
        const uint32_t x = __builtin_amdgcn_perm(raw[c1 / 2], raw[c0 / 2], sel_q);
        w[v] = mine ? x : 0u;
      }
      qb[s] = __builtin_bit_cast(half8_t, make_uint4(w[0], w[1], w[2], w[3]));
    }
  }
  // Scores are sums of q * u * 2^-24 (times 2^-q_exp for a scaled bf16 head).
  const float qscale = a.qscale * 0x1p24f * __builtin_bit_cast(float, (uint32_t)(127 + q_exp) << 23);

  floatx4 acc1[8], acc2[8], accl;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc1[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  accl = floatx4{0.f, 0.f, 0.f, 0.f};
  float beta1 = 0.f, beta2 = 0.f;  // sum_r p * b_V over this lane's rows
  float m_run = kNegSentinel;
  const _Float16 one = (_Float16)1.f;
  const half8_t ones = {one, one, one, one, one, one, one, one};

  // Per-wave LDS slots for one pair's scale words (two, used alternately:
  // the scores of pair k + 1 write one while pair k's V products read the
  // other; LDS operations of a wave run in order).
  __shared__ __attribute__((aligned(16))) uint32_t lds_s[NW][2][6 * SWT];

  // The lane's group halves of rows (4*blk, +1) in out[0] and (4*blk + 2,
  // +3) in out[1] of tile T, tensor t, pair slot k & 1.
  auto scales = [&](uint32_t (&out)[2], int t, int T, int k) {
    const uint32_t* sbuf = lds_s[wave][k & 1];
    if constexpr (NG == 2) {
      const uint4 w = *reinterpret_cast<const uint4*>(&sbuf[t * SWT + 16 * T + 4 * blk]);
      out[0] = __builtin_amdgcn_perm(w.y, w.x, sel);
      out[1] = __builtin_amdgcn_perm(w.w, w.z, sel);
    } else {
      const uint2 w = *reinterpret_cast<const uint2*>(&sbuf[t * SWT + 8 * T + 2 * blk]);
      out[0] = w.x;
      out[1] = w.y;
    }
  };

  // Scores of pair k, rows t_T + 4*blk + r of column col, in units of
  // 2^-24 / qscale' (unmasked).  Publishes the pair's scale words to LDS.
  auto score_pair = [&](const Pair& P, int k, float (&x)[8]) {
    uint32_t* sbuf = lds_s[wave][k & 1];
    if (lane < SLANES) {
      const int r0 = pair_row(k);
#pragma unroll
      for (int t = 0; t < 6; ++t) {
        uint32_t w = P.s[t];
        if constexpr (NG == 1) {  // rows past max_lim may be unwritten padding
          const int row = r0 + 2 * lane;
          w = row + 1 < max_lim ? w : (row < max_lim ? (w & 0xFFFFu) : 0u);
        }
        if constexpr (kBf16) {  // V scales as fp16 pairs for the weight products
          if (t == 2 || t == 4) w = f16_pair(pair_lo_f32<E>(w), pair_hi_f32<E>(w));
        }
        sbuf[t * SWT + lane] = w;
      }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      floatx4 t_lo = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 t_hi = floatx4{0.f, 0.f, 0.f, 0.f};
      if constexpr (BITS == 4) {
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t x0 = P.k[T][w], x8 = P.k[T][w] >> 8;
          lo[2 * w] = x0 & 0x000F000Fu;
          lo[2 * w + 1] = x8 & 0x000F000Fu;
          hi[2 * w] = x0 & 0x00F000F0u;
          hi[2 * w + 1] = x8 & 0x00F000F0u;
        }
        t_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(half8_t, make_uint4(lo[0], lo[1], lo[2], lo[3])), qb[0], t_lo, 0, 0, 0);
        t_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(half8_t, make_uint4(hi[0], hi[1], hi[2], hi[3])), qb[2], t_hi, 0, 0, 0);
        t_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(half8_t, make_uint4(lo[4], lo[5], lo[6], lo[7])), qb[1], t_lo, 0, 0, 0);
        t_hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(half8_t, make_uint4(hi[4], hi[5], hi[6], hi[7])), qb[3], t_hi, 0, 0, 0);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t w0 = P.k[T][2 * s], w1 = P.k[T][2 * s + 1];
          const uint4 e = make_uint4(w0 & 0x00FF00FFu, (w0 >> 8) & 0x00FF00FFu, w1 & 0x00FF00FFu,
                                     (w1 >> 8) & 0x00FF00FFu);
          t_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, e), qb[s],
                                                        t_lo, 0, 0, 0);
        }
      }
      uint32_t sk[2], sb[2];
      scales(sk, 0, T, k);
      scales(sb, 1, T, k);
      const float skr[4] = {pair_lo_f32<E>(sk[0]), pair_hi_f32<E>(sk[0]), pair_lo_f32<E>(sk[1]),
                            pair_hi_f32<E>(sk[1])};
      const float bkr[4] = {pair_lo_f32<E>(sb[0]), pair_hi_f32<E>(sb[0]), pair_lo_f32<E>(sb[1]),
                            pair_hi_f32<E>(sb[1])};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float tt = BITS == 4 ? fmaf(t_hi[r], 0.0625f, t_lo[r]) : t_lo[r];
        // Unused columns have q = 0 and qs = 0, so their score is 0.
        x[4 * T + r] = sum_adjacent_groups<NG>(fmaf(skr[r], tt, bkr[r] * qs));
      }
    }
  };

  // Mask, running-max update and fp16 softmax weights of pair k.  k order of
  // the weights: rows 0..3 of the first tile, then rows 0..3 of the second
  // (this lane's 4*blk + r).  p is rounded to fp16 once; the V weights, the
  // bias terms and l use the same values.
  auto softmax_pair = [&](float (&x)[8], int k, uint32_t (&pw)[4]) {
    const int r0 = pair_row(k);
    // Rows at or past the column's limit: only in a pair that crosses the
    // smallest limit of the workgroup's columns (a wave-uniform test).
    if (r0 + 32 > min_lim) {
      asm volatile("");  // keep this a branch: it runs in one pair per split
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = r0 + 16 * (i / 4) + 4 * blk + (i % 4);
        x[i] = row < lim ? x[i] : -__builtin_inff();
      }
    }
    float mx = vmax(vmax(vmax(x[0], x[1]), vmax(x[2], x[3])),
                    vmax(vmax(x[4], x[5]), vmax(x[6], x[7])));
    mx = rows4_max(mx) * qscale;
    if (__ballot(mx > m_run + kSlack) != 0) {
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
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float p0 = fast_exp2(fmaf(x[2 * v], qscale, -m_run));
      const float p1 = fast_exp2(fmaf(x[2 * v + 1], qscale, -m_run));
      pw[v] = h2_bits(half2_t{(_Float16)p0, (_Float16)p1});
    }
  };

  // Both V products (and l, and the bias terms) of pair k with weights pw.
  auto pv_pair = [&](const Pair& P, int k, const uint32_t (&pw)[4]) {
    uint32_t w1[4], w2[4];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      uint32_t s1[2], c1[2], s2[2], c2[2];
      scales(s1, 2, T, k);
      scales(c1, 3, T, k);
      scales(s2, 4, T, k);
      scales(c2, 5, T, k);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const half2_t p = as_h2(pw[2 * T + h]);
        w1[2 * T + h] = h2_bits(p * as_h2(s1[h]));
        w2[2 * T + h] = h2_bits(p * as_h2(s2[h]));
        if constexpr (kBf16) {  // bf16 biases: fp32 products of the same fp16 weights
          const float p0 = (float)p.x, p1 = (float)p.y;
          beta1 = fmaf(p1, pair_hi_f32<E>(c1[h]), fmaf(p0, pair_lo_f32<E>(c1[h]), beta1));
          beta2 = fmaf(p1, pair_hi_f32<E>(c2[h]), fmaf(p0, pair_lo_f32<E>(c2[h]), beta2));
        } else {
          beta1 = __builtin_amdgcn_fdot2(p, as_h2(c1[h]), beta1, false);
          beta2 = __builtin_amdgcn_fdot2(p, as_h2(c2[h]), beta2, false);
        }
      }
    }
    const half8_t W1 = __builtin_bit_cast(half8_t, make_uint4(w1[0], w1[1], w1[2], w1[3]));
    const half8_t W2 = __builtin_bit_cast(half8_t, make_uint4(w2[0], w2[1], w2[2], w2[3]));
    // V^T operands: channel 8*col + i, rows (first tile 0..3, second 0..3).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t a1[4], a2[4];
#pragma unroll
      for (int T = 0; T < 2; ++T) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int wi = BITS == 4 ? 0 : i / 4;
          const int by = BITS == 4 ? i / 2 : i % 4;
          const uint32_t x1 = pair_bytes(P.v1[T][2 * h][wi], P.v1[T][2 * h + 1][wi], by);
          const uint32_t x2 = pair_bytes(P.v2[T][2 * h][wi], P.v2[T][2 * h + 1][wi], by);
          if constexpr (BITS == 4) {  // even i: low nibbles; odd i: whole bytes
            a1[2 * T + h] = (i & 1) ? x1 : x1 & 0x000F000Fu;
            a2[2 * T + h] = (i & 1) ? x2 : x2 & 0x000F000Fu;
          } else {
            a1[2 * T + h] = x1;
            a2[2 * T + h] = x2;
          }
        }
      }
      acc1[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(half8_t, make_uint4(a1[0], a1[1], a1[2], a1[3])), W1, acc1[i], 0, 0, 0);
      acc2[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(half8_t, make_uint4(a2[0], a2[1], a2[2], a2[3])), W2, acc2[i], 0, 0, 0);
    }
    accl = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        ones, __builtin_bit_cast(half8_t, make_uint4(pw[0], pw[1], pw[2], pw[3])), accl, 0, 0, 0);
  };

  // Two pair sets in turn: the next pair's loads are in flight while the
  // current pair is computed.
  // (Loads past the wave's last pair are out of range: zeros, no traffic.)
  auto compute_pair = [&](const Pair& P, int k) {
    float x[8];
    uint32_t pw[4];
    score_pair(P, k, x);
    softmax_pair(x, k, pw);
    pv_pair(P, k, pw);
  };
  for (int k = 0; k < npair; k += 2) {
    load_pair(P1, k + 1);
    compute_pair(P0, k);
    if (k + 1 >= npair) break;
    load_pair(P0, k + 2);
    compute_pair(P1, k + 1);
  }

  // acc[i][r] of lane (col, blk) is channel 8*(4*blk + r) + i of head hh,
  // valid where that channel's group is g.  Codes were u * 2^-24 (q8, q4 low
  // nibbles: even i) or, for q4's odd i, whole bytes (u_lo + 16 u_hi) * 2^-24,
  // so acc[i] - acc[i - 1] is the high nibbles' 16 u_hi * 2^-24 sum.
  __shared__ __attribute__((aligned(16))) float lds_o[NW][GC][2 * D + kLdsPad];
  __shared__ float lds_m[NW][GC];
  __shared__ float lds_l[NW][GC];
  const float be1 = rows4_sum(beta1), be2 = rows4_sum(beta2);
  if (used && (32 * blk) / GS == g) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (BITS == 4 && (i & 1)) ? 0x1p20f : 0x1p24f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ch = 8 * (4 * blk + r);
      float o1[8], o2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool odd4 = BITS == 4 && (i & 1);
        o1[i] = fmaf(odd4 ? acc1[i][r] - acc1[i - 1][r] : acc1[i][r], f[i], be1);
        o2[i] = fmaf(odd4 ? acc2[i][r] - acc2[i - 1][r] : acc2[i][r], f[i], be2);
      }
      *reinterpret_cast<float4*>(&lds_o[wave][hh][ch]) = make_float4(o1[0], o1[1], o1[2], o1[3]);
      *reinterpret_cast<float4*>(&lds_o[wave][hh][ch + 4]) = make_float4(o1[4], o1[5], o1[6], o1[7]);
      *reinterpret_cast<float4*>(&lds_o[wave][hh][D + ch]) = make_float4(o2[0], o2[1], o2[2], o2[3]);
      *reinterpret_cast<float4*>(&lds_o[wave][hh][D + ch + 4]) =
          make_float4(o2[4], o2[5], o2[6], o2[7]);
    }
  }
  if (used && g == 0 && blk == 0) {
    lds_m[wave][hh] = m_run;
    lds_l[wave][hh] = accl[0];
  }
  __syncthreads();
  wg_epilogue<E, D, GC, NW, false, true>(a, lds_o, lds_m, lds_l, qrow0, nvh, split, unit);
}

// Heads per workgroup gc (a power of two, gc * 128 / gs <= 16), waves 4 or 8;
// E: element type of q, scales, biases and y (half_t or bf16_t).
template <int BITS, int GS, typename E>
int launch_sdpa_qpair_gs(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t st) {
  constexpr int NG = 128 / GS;
  constexpr int GCM = 16 / NG < 8 ? 16 / NG : 8;
  constexpr int S = kCachePolicyStream;
  if (a.nchunk > 1 && gc == GCM && waves == 4) {
    hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, GCM, 4, 0, E>), dim3(nblocks), dim3(256), 0,
                       st, a);
    return check_launch("sdpa_dual_v_q (pairs, chunks)");
  }
  switch (gc) {
    case 1:
      if (waves == 8) hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 1, 8, S, E>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 1, 4, S, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 2:
      if (waves == 8) hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 2, 8, S, E>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 2, 4, S, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 4:
      if (waves == 8) hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 4, 8, S, E>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 4, 4, S, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 8:
      if constexpr (8 * NG <= 16) {
        hipLaunchKernelGGL((sdpa_qpair_kernel<BITS, GS, 8, 4, S, E>), dim3(nblocks), dim3(256), 0, st, a);
        break;
      }
      [[fallthrough]];
    default:
      set_error("sdpa_dual_v_q: no paired MFMA variant for %d heads per workgroup", gc);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("sdpa_dual_v_q (pairs)");
}

}  // namespace motif
