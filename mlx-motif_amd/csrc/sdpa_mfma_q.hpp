// Matrix-core formulation of split-KV dual-V decode over the packed
// MLX-affine cache (q4 / q8, head_dim 128; fp16 or bf16 q, scales, biases
// and outputs, the products fp16 MFMAs either way).
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
// Codes enter the MFMAs as fp16 subnormals: a code u in the low mantissa
// bits of a zero-exponent half is the value u * 2^-24 (16u * 2^-24 for the
// high nibble of a byte), and the matrix cores multiply subnormal fp16
// inputs exactly, so a v_perm_b32 (q8: a byte per half) or one AND (q4: a
// nibble per half) makes an operand, with no bias to add or subtract.
//   K: q8 k-step s holds words 2s, 2s+1 in channel order.  q4 k-steps 0/1
//     hold the low nibbles of words 0-1 / 2-3 and steps 2/3 their high
//     nibbles (channel order qtile_k_channel), summed in two chains
//     t_lo = sum q u 2^-24 and t_hi = sum q 16u 2^-24; sum q u is
//     2^24 (t_lo + t_hi / 16).  The 2^24 rides on the softmax scale and
//     the bias term's qsum carries 2^-24 (powers of two: exact).
//   V^T fragments (4 rows x 1 channel per lane) take code i of one word per
//     row, paired across rows with v_perm_b32.  q4: channel 2b (the low
//     nibble of byte b) masks it to u; channel 2b + 1 takes the whole byte
//     u + 16u' and the epilogue recovers the high nibble's sum as the
//     difference of the two accumulators, times 2^20 (2^24 for the others).
// Everything else (split plan, online softmax in log2 units with lazy
// rescaling, workgroup epilogue) matches the fp16-cache kernel.
#pragma once

#include "quant_impl.hpp"
#include "rope_impl.hpp"
#include "sdpa_mfma.hpp"

namespace motif {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ inline half2_t as_h2(uint32_t x) { return __builtin_bit_cast(half2_t, x); }
__device__ inline uint32_t h2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Low / high 16-bit element of a packed pair as fp32 (fp16 or bf16).
template <typename T>
__device__ inline float pair_lo_f32(uint32_t w) {
  if constexpr (std::is_same<T, bf16_t>::value) return __builtin_bit_cast(float, w << 16);
  return (float)as_h2(w).x;
}
template <typename T>
__device__ inline float pair_hi_f32(uint32_t w) {
  if constexpr (std::is_same<T, bf16_t>::value) return __builtin_bit_cast(float, w & 0xFFFF0000u);
  return (float)as_h2(w).y;
}
// Two floats as an fp16 pair (round to nearest even).
__device__ inline uint32_t f16_pair(float lo, float hi) {
  return h2_bits(half2_t{(_Float16)lo, (_Float16)hi});
}
// Value of code 1 as an fp16 subnormal, and its inverse.
constexpr float kCodeUnit = 0x1p-24f;
constexpr float kCodeScale = 0x1p24f;

// Channel (within the lane's 32-channel block) of element j of k-step s of
// the K operand.  q4: steps 0/1 hold the low nibbles of words 0-1 / 2-3,
// steps 2/3 their high nibbles; a word w gives (w & 0x000F000F) = nibbles 0
// and 4, ((w >> 8) & 0x000F000F) = nibbles 2 and 6.  q8: step s holds words
// 2s, 2s+1, bytes in order.
template <int BITS>
__host__ __device__ constexpr int qtile_k_channel(int s, int j) {
  if constexpr (BITS == 4) {
    constexpr int lo[4] = {0, 4, 2, 6};
    return 16 * (s & 1) + 8 * (j / 4) + lo[j % 4] + (s >> 1);
  } else {
    return 8 * s + j;
  }
}

// K operand of k-step s from the lane's K words (order qtile_k_channel).
template <int BITS, int KW>
__device__ inline half8_t k_codes(const uint32_t (&k)[KW], int s) {
  uint32_t e[4];
  if constexpr (BITS == 4) {
    const uint32_t m = s < 2 ? 0x000F000Fu : 0x00F000F0u;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t x = k[2 * (s & 1) + w];
      e[2 * w] = x & m;
      e[2 * w + 1] = (x >> 8) & m;
    }
  } else {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t x = k[2 * s + w];
      e[2 * w] = __builtin_amdgcn_perm(x, x, 0x0C010C00u);
      e[2 * w + 1] = __builtin_amdgcn_perm(x, x, 0x0C030C02u);
    }
  }
  return __builtin_bit_cast(half8_t, make_uint4(e[0], e[1], e[2], e[3]));
}

// Byte k of words a (low half) and b (high half), zero-extended to 16 bits.
__device__ inline uint32_t pair_bytes(uint32_t a, uint32_t b, int k) {
  const uint32_t sel = (uint32_t)k | (0x0Cu << 8) | ((uint32_t)(4 + k) << 16) | (0x0Cu << 24);
  return __builtin_amdgcn_perm(b, a, sel);
}

// V^T fragment: code i of the lane's word in rows r0..r3 as fp16 subnormals
// (q4, odd i: the whole byte, u_lo + 16 u_hi).
template <int BITS>
__device__ inline half4_t v_codes(const uint32_t (&w)[4], int i) {
  const int k = BITS == 4 ? i >> 1 : i;
  uint32_t lo = pair_bytes(w[0], w[1], k);
  uint32_t hi = pair_bytes(w[2], w[3], k);
  if (BITS == 4 && !(i & 1)) {
    lo &= 0x000F000Fu;
    hi &= 0x000F000Fu;
  }
  return __builtin_bit_cast(half4_t, make_uint2(lo, hi));
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

// One 16-row tile of the packed cache as one lane loads it.
//   k[KW]      K codes of row t0 + col, channels 32*blk .. 32*blk+31
//   v1/v2[4][] V codes of rows t0 + 4*blk + r, channels 8*col .. 8*col+7
//   s[6][SW]   raw fp16 (scale, bias) words of K, V1, V2 for rows
//              t0 + 4*blk .. +3 that hold the lane's scale group
// Nothing is consumed at load time, so all loads of a tile are in flight
// together; scale_words() extracts the lane's halves when it is computed.
//   k2[KW], s[6..7]  (fused GDA decode step) the noise keys' codes and
//              their scale / bias words
template <int BITS, int NG, bool DUAL = false>
struct QTile {
  static constexpr int WPR = 128 * BITS / 32;
  static constexpr int KW = WPR / 4;
  static constexpr int VW = WPR / 16;
  static constexpr int SW = NG == 1 ? 2 : 4;
  static constexpr int NS = DUAL ? 8 : 6;
  uint32_t k[KW];
  uint32_t k2[DUAL ? KW : 1];
  uint32_t v1[4][VW];
  uint32_t v2[4][VW];
  uint32_t s[NS][SW];
};

// Raw scale / bias words of one tensor for rows row0 .. row0+3 (NG groups of
// fp16 per row).  NG = 1: the four halves, one 8-byte load; NG = 2: two
// 8-byte loads of two rows each; NG = 4: one 4-byte load per row holding
// groups (gsel & ~1, gsel | 1).  The resource covers whole 4-row groups, so
// no load straddles its end.
template <int NG, int POL>
__device__ inline void load_scales(uint32_t (&w)[NG == 1 ? 2 : 4], __amdgpu_buffer_rsrc_t r,
                                   unsigned row0, int gsel) {
  if constexpr (NG == 1) {
    const uint2 x = bload2<POL>(r, row0 * 2u);
    w[0] = x.x;
    w[1] = x.y;
  } else if constexpr (NG == 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint2 x = bload2<POL>(r, (row0 + 2u * p) * 4u);  // rows r, r+1: {g0,g1},{g0,g1}
      w[2 * p] = x.x;
      w[2 * p + 1] = x.y;
    }
  } else {
    const unsigned off = (row0 * 4u + (unsigned)(gsel & ~1)) * 2u;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = bload1<POL>(r, off + 8u * i);
  }
}

// The lane's halves of rows row0, row0+1 (word 0) and row0+2, row0+3
// (word 1); sel is the per-lane v_perm selector of half (gsel & 1).
template <int NG>
__device__ inline void scale_words(uint32_t (&out)[2], const uint32_t (&w)[NG == 1 ? 2 : 4],
                                   uint32_t sel) {
  if constexpr (NG == 1) {
    out[0] = w[0];
    out[1] = w[1];
  } else {
    out[0] = __builtin_amdgcn_perm(w[1], w[0], sel);
    out[1] = __builtin_amdgcn_perm(w[3], w[2], sel);
  }
}

// Rows at or past nrows (cache padding, possibly never written, read by a
// whole 4-row scale load) get zero scale and bias.
__device__ inline void drop_rows_past(uint32_t (&out)[2], unsigned row0, unsigned nrows) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const unsigned r0 = row0 + 2u * p;
    out[p] = r0 + 1u < nrows ? out[p] : (r0 < nrows ? (out[p] & 0xFFFFu) : 0u);
  }
}

// Packed rows: lane L quantises chunk L % 16 (8 values) of slot L / 16 (k1,
// k2, v1, v2) of the new token exactly as motif_quant_write4 does, and
// stores the codes, scale and bias at row kv_len - 1 of KV head bk.  E:
// element type of the new rows, scales and biases.
template <int BITS, int GS, typename E = half_t>
__device__ inline void append_rows_q(const SdpaArgs& a, long bk, int lane) {
  constexpr int D = 128;
  constexpr int LPG = GS / 8;
  constexpr int NG = D / GS;
  constexpr int WPR = D * BITS / 32;
  const int slot = lane / 16;
  const int chunk = lane % 16;
  const uint32_t* data = slot == 0 ? a.kd : slot == 1 ? a.k2d : slot == 2 ? a.v1d : a.v2d;
  const void* sc = slot == 0 ? a.ks : slot == 1 ? a.k2s : slot == 2 ? a.v1s : a.v2s;
  const void* bi = slot == 0 ? a.kb : slot == 1 ? a.k2b : slot == 2 ? a.v1b : a.v2b;
  float v[8];
  if (!a.from_proj) {
    const void* src =
        slot == 0 ? a.new_k1 : slot == 1 ? a.new_k2 : slot == 2 ? a.new_v1 : a.new_v2;
    load8<E>(src, bk * D + (long)chunk * 8, v);
  } else {
    // From the projections: head 2 * kvh + (slot & 1), row 2 * bk + (slot & 1);
    // k rows are roped (pair partner in lane L ^ 8) and rounded to E as
    // rope_split4 stores them, then quantised.
    load8<E>(slot < 2 ? a.new_k1 : a.new_v1, (2 * bk + (slot & 1)) * D + (long)chunk * 8, v);
    // Lane L computes the angle of pair L (0..63) once; the lanes read the
    // eight they need with __shfl (one slow-path sincosf per lane, not eight).
    const bool first = chunk < 8;
    float cs0, sn0;
    rope_angle(lane, D, a.kv_len - 1, a.rope_log2_theta, a.rope_pos_scale, cs0, sn0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float other = __shfl_xor(v[e], 8);
      const float cs = __shfl(cs0, 8 * (chunk & 7) + e);
      const float sn = __shfl(sn0, 8 * (chunk & 7) + e);
      float y1, y2;
      rope_rotate(first ? v[e] : other, first ? other : v[e], cs, sn, y1, y2);
      const float y = Elem<E>::to_f32(Elem<E>::from_f32(first ? y1 : y2));
      if (slot < 2) v[e] = y;
    }
  }
  uint32_t w[2];
  float scale, bias;
  quantize8<BITS, LPG>(v, w, scale, bias);
  const long crow = bk * a.kv_cap + a.kv_len - 1;
  store_words<BITS>(const_cast<uint32_t*>(data), crow * WPR + (long)chunk * (8 * BITS / 32), w);
  if (chunk % LPG == 0) {
    Elem<E>::store(const_cast<void*>(sc), crow * NG + chunk / LPG, scale);
    Elem<E>::store(const_cast<void*>(bi), crow * NG + chunk / LPG, bias);
  }
}

// POL: cache policy of the K/V/scale loads.  Launches with several head
// chunks (a.nchunk > 1: more virtual heads than one pass holds, e.g. a
// verify slab) read each row in several workgroups and use cached loads, so
// all but the first find the rows in L2 or the Infinity Cache.
// DUAL: fused GDA decode step, as in sdpa_mfma_kernel: head h < G of a
// column scores against k, heads G..G+G2-1 (the noise heads) against k2.
// NB: column blocks per wave.  Block bb holds heads bb*GC .. bb*GC+GC-1 of
// the workgroup's NB*GC; the K and V codes of a tile are unpacked once and
// feed every block's MFMAs, so a verify slab (e.g. 5 rows x GQA 4 = 20
// virtual heads) runs as one pass instead of one workgroup per 8 heads.
// The accumulators of NB > 1 blocks live in AGPRs at one wave per SIMD.
// E: element type of q, the scales and biases and y (fp16 or bf16).  bf16
// heads are scaled by a power of two and rounded to fp16 once (below); the
// products stay fp16 MFMAs over the codes, and the K scales and the bias
// terms are taken in fp32.  Those fp32 operands need more registers than two
// waves per SIMD leave, so bf16 variants run one wave per SIMD (4-wave
// workgroups, the planner's default).
template <int BITS, int GS, int GC, int NW, int U, int POL = kCachePolicyStream,
          bool DUAL = false, int NB = 1, typename E = half_t>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(NB > 1 || std::is_same<E, bf16_t>::value ? 1 : 2)))
sdpa_mfma_q_kernel(SdpaArgs a) {
  constexpr int D = 128;
  constexpr int NG = D / GS;  // scale groups per row
  constexpr int GCW = NB * GC;  // heads per workgroup
  using Tile = QTile<BITS, NG, DUAL>;
  constexpr int NS = Tile::NS;
  constexpr int WPR = Tile::WPR;
  constexpr int KW = Tile::KW;
  constexpr int VW = Tile::VW;
  static_assert(GC * NG <= 16, "heads x groups ride the 16 MFMA columns");
  static_assert(!DUAL || NB == 1, "the fused decode step uses one column block");
  constexpr bool kBf16 = std::is_same<E, bf16_t>::value;
  // Lazy-rescale slack (see kRescaleSlackF16): here p also multiplies the V
  // scale in fp16, so p * s must stay finite.  An fp16 cache row spans at
  // most 2 * 65504, so s <= 131008 / 15 (q4) or / 255 (q8), and 2^slack * s
  // stays below 65504 with slack 2 (q4) or 6 (q8).
  constexpr float kSlack = BITS == 4 ? 2.f : 6.f;
  const int lane = threadIdx.x & 63;
  // Wave index as a wave-uniform (scalar) value: tile rows and the tests on
  // them are then scalar, and so are the branches that depend on them.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int blk = lane >> 4;

  int unit, split;
  if (!sdpa_block_coords(a, blockIdx.x, unit, split)) return;  // grid padding
  const int chunk = unit % a.nchunk;
  const int bk = unit / a.nchunk;
  const int b = bk / a.Hkv;
  const int kvh = bk % a.Hkv;
  const int vh0 = chunk * GCW;
  const int nvh = min(GCW, a.GV - vh0);
  // First output row: y row (non-DUAL) or partial row (DUAL) of head 0.
  const long qrow0 = DUAL ? ((long)b * a.Hkv + kvh) * (a.G + a.G2)
                          : ((long)b * a.Hq + (long)kvh * a.G) * a.S_q + vh0;

  const int grp = col / GC;  // scale group of this column
  int hb[NB];                // head (within the workgroup) of this column, per block
  bool used[NB];
  int lim[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    hb[bb] = bb * GC + col % GC;
    used[bb] = grp < NG && hb[bb] < nvh;
    lim[bb] = hb[bb] < nvh ? vhead_limit(a, vh0 + hb[bb]) : 0;
  }
  const int h = hb[0];
  const int gsel = grp < NG ? grp : 0;  // group whose scales this lane reads
  // v_perm selector keeping half (gsel & 1) of two words: low word = row r.
  const uint32_t sel = (gsel & 1) ? 0x07060302u : 0x05040100u;
  // Rows below min_lim are visible to every column of the workgroup.
  int min_lim, max_lim;
  vhead_limit_range(a, vh0, nvh, min_lim, max_lim);
  // Rows are dealt to the splits in blocks of NW 16-row tiles, round robin,
  // as in sdpa_mfma_kernel: tile k of wave w in split s is tile
  // (k * nsplit + s) * NW + w of the KV head.  The resources cover rows
  // [0, max_lim) of the KV head (scales: whole 4-row groups, inside the
  // cache since kv_cap % 4 == 0); rows past them read 0.
  const int ns = a.nsplit;
  auto tile_row = [&](int k) { return 16 * ((k * ns + split) * NW + wave); };
  const long hrow0 = (long)bk * a.kv_cap;  // first cache row of this KV head
  const unsigned dbytes = (unsigned)(max_lim * WPR * 4);
  const auto rk = stream_rsrc(a.kd + hrow0 * WPR, dbytes);
  const auto rv1 = stream_rsrc(a.v1d + hrow0 * WPR, dbytes);
  const auto rv2 = stream_rsrc(a.v2d + hrow0 * WPR, dbytes);
  const unsigned sbytes = (unsigned)(((max_lim + 3) & ~3) * NG * 2);
  const __amdgpu_buffer_rsrc_t rs[8] = {
      stream_rsrc((const uint16_t*)a.ks + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.kb + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1b + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2b + hrow0 * NG, sbytes),
      stream_rsrc(DUAL ? (const uint16_t*)a.k2s + hrow0 * NG : nullptr, DUAL ? sbytes : 0u),
      stream_rsrc(DUAL ? (const uint16_t*)a.k2b + hrow0 * NG : nullptr, DUAL ? sbytes : 0u)};
  const auto rk2 = stream_rsrc(DUAL ? a.k2d + hrow0 * WPR : nullptr, DUAL ? dbytes : 0u);

  // Append: the owner quantises and stores the new rows first, and waits for
  // the stores before it loads the tile that holds row kv_len - 1.
  // (If that tile is not among the first U, the store is issued after the
  // first tiles' loads instead, so that it does not delay them.)
  bool owner = false;
  bool append_early = false;
  const int append_tile = (a.kv_len - 1) / 16 * 16;  // first row of that tile
  if constexpr (DUAL) {
    owner = append_owner<NW>(a, split, wave);
#pragma unroll
    for (int u = 0; u < U; ++u) append_early |= tile_row(u) == append_tile;
    if (owner && append_early) append_rows_q<BITS, GS, E>(a, bk, lane);
  }

  // All loads of this wave's tiles k0 .. k0 + U - 1 (rows past max_lim read 0).
  auto load_tiles = [&](Tile (&T)[U], int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (DUAL) {
        if (owner && tile_row(k0 + u) == append_tile)
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the new rows are stored
      }
      const unsigned r0 = (unsigned)tile_row(k0 + u);
      const unsigned koff = ((r0 + col) * WPR + KW * blk) * 4u;
#pragma unroll
      for (int i = 0; i < KW; i += 4) {
        const uint4 x = bload4<POL>(rk, koff + 4u * i);
        T[u].k[i] = x.x; T[u].k[i + 1] = x.y; T[u].k[i + 2] = x.z; T[u].k[i + 3] = x.w;
      }
      if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < KW; i += 4) {
          const uint4 x = bload4<POL>(rk2, koff + 4u * i);
          T[u].k2[i] = x.x; T[u].k2[i + 1] = x.y; T[u].k2[i + 2] = x.z; T[u].k2[i + 3] = x.w;
        }
      }
      const unsigned vrow = r0 + 4u * blk;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned voff = ((vrow + r) * WPR + VW * col) * 4u;
        if constexpr (VW == 1) {
          T[u].v1[r][0] = bload1<POL>(rv1, voff);
          T[u].v2[r][0] = bload1<POL>(rv2, voff);
        } else {
          const uint2 x1 = bload2<POL>(rv1, voff);
          const uint2 x2 = bload2<POL>(rv2, voff);
          T[u].v1[r][0] = x1.x; T[u].v1[r][1] = x1.y;
          T[u].v2[r][0] = x2.x; T[u].v2[r][1] = x2.y;
        }
      }
#pragma unroll
      for (int t = 0; t < NS; ++t) load_scales<NG, POL>(T[u].s[t], rs[t], vrow, gsel);
    }
  };

  // The first tile set's loads are issued before q is consumed, so their
  // latency and q's overlap.
  Tile ta[U], tb[U];
  int k0 = 0;
  uint4 qraw[NB][4];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    const uint16_t* qp =
        (const uint16_t*)a.q + (qrow0 + (hb[bb] < nvh ? hb[bb] : 0)) * D + 32 * blk;
    if constexpr (DUAL) {
      const int hq = h < nvh ? h : 0;  // unused columns load head 0 (in bounds)
      if (a.from_proj) {  // q_proj heads (G2 == 1): stripe g*(G+1)+j, or origin-first
        const int head = a.q_origin_first ? (hq < a.G ? kvh * a.G + hq : a.Hkv * a.G + kvh)
                                          : kvh * (a.G + 1) + (hq < a.G ? hq : a.G);
        qp = (const uint16_t*)a.q + ((long)b * a.Hkv * (a.G + 1) + head) * D;
      } else {  // noise column G + i: q2 head kvh * G2 + i
        qp = hq < a.G
                 ? (const uint16_t*)a.q + ((long)b * a.Hq + (long)kvh * a.G + hq) * D
                 : (const uint16_t*)a.q2 + (((long)b * a.Hkv + kvh) * a.G2 + (hq - a.G)) * D;
      }
      qp += 32 * blk;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) qraw[bb][s] = *reinterpret_cast<const uint4*>(qp + 8 * s);
  }
  // Fused step: keep the q loads ahead of the tile loads, so the q RoPE below
  // waits for q alone, not for the first tiles too.
  if constexpr (DUAL) __builtin_amdgcn_sched_barrier(0);
  load_tiles(ta, k0);
  if constexpr (DUAL) {
    if (a.from_proj) {
      // RoPE at kv_len - 1, rounded to fp16 as rope_split4 does (after the
      // first tiles' loads are issued, so their latency covers it).  Lane (col,
      // blk) holds channels 32*blk + 8*s + e; the pair partner of blk is blk ^ 2
      // (lane L ^ 32).  Lane L computes the angle of pair L, which the
      // others read with __shfl.
      float cs0, sn0;
      rope_angle(lane, D, a.kv_len - 1, a.rope_log2_theta, a.rope_pos_scale, cs0, sn0);
      const bool first = blk < 2;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint32_t w[4] = {qraw[0][s].x, qraw[0][s].y, qraw[0][s].z, qraw[0][s].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t o = (uint32_t)__shfl_xor((int)w[i], 32);
          uint32_t r = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int p = 32 * (blk & 1) + 8 * s + 2 * i + e;
            const float cs = __shfl(cs0, p);
            const float sn = __shfl(sn0, p);
            const float mine = Elem<E>::to_f32((uint16_t)(e ? w[i] >> 16 : w[i] & 0xFFFFu));
            const float oth = Elem<E>::to_f32((uint16_t)(e ? o >> 16 : o & 0xFFFFu));
            float y1, y2;
            rope_rotate(first ? mine : oth, first ? oth : mine, cs, sn, y1, y2);
            r |= (uint32_t)Elem<E>::from_f32(first ? y1 : y2) << (16 * e);
          }
          w[i] = r;
        }
        qraw[0][s] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    // The deferred append comes after the q RoPE: its loads would otherwise
    // make every wave's RoPE wait for the first tiles (register reuse
    // across the branch).
    if (owner && !append_early) append_rows_q<BITS, GS, E>(a, bk, lane);
  }

  // bf16 activations: each head's q is scaled by 2^-e, e the smallest >= 0
  // that brings the head's largest |q| below 2^15 (the four lanes of a
  // column hold the head's 128 channels), and rounded to fp16; 2^e goes
  // into that head's softmax scale.
  int q_exp[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    q_exp[bb] = 0;
    if constexpr (kBf16) {
      uint32_t w[16];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        w[4 * s] = qraw[bb][s].x; w[4 * s + 1] = qraw[bb][s].y;
        w[4 * s + 2] = qraw[bb][s].z; w[4 * s + 3] = qraw[bb][s].w;
      }
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        mx = fmaxf(mx, fmaxf(fabsf(pair_lo_f32<E>(w[i])), fabsf(pair_hi_f32<E>(w[i]))));
      mx = rows4_max(mx);
      const int ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFFu) - 127;
      q_exp[bb] = ex > 14 ? ex - 14 : 0;  // 0 for zero, subnormal and small heads
      const float f = __builtin_bit_cast(float, (uint32_t)(127 - q_exp[bb]) << 23);
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] = f16_pair(pair_lo_f32<E>(w[i]) * f, pair_hi_f32<E>(w[i]) * f);
#pragma unroll
      for (int s = 0; s < 4; ++s)
        qraw[bb][s] = make_uint4(w[4 * s], w[4 * s + 1], w[4 * s + 2], w[4 * s + 3]);
    }
  }

  // Q^T (B of the K MFMA): lane (col, blk), element j of k-step s is channel
  // 32*blk + qtile_k_channel(s, j); nonzero only where the channel's group is
  // the column's group.  qsum: sum of q_h over the column's group, times
  // 2^-24 (the unit of the code sums it is added to).
  half8_t qb[NB][4];
  float qsum[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    const bool mine = used[bb] && (32 * blk) / GS == grp;
    half8_t raw[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) raw[s] = __builtin_bit_cast(half8_t, qraw[bb][s]);
    qsum[bb] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = qtile_k_channel<BITS>(s, j);
        const _Float16 v = mine ? raw[c / 8][c % 8] : (_Float16)0.f;
        qb[bb][s][j] = v;
        qsum[bb] += (float)v;
      }
    }
    qsum[bb] += __shfl_xor(qsum[bb], 16);
    qsum[bb] += __shfl_xor(qsum[bb], 32);
    qsum[bb] *= kCodeUnit;
  }
  // Scores are sums in units of 2^-24 (times 2^-q_exp for a scaled bf16 head).
  float qsc[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
    qsc[bb] = a.qscale * kCodeScale * __builtin_bit_cast(float, (uint32_t)(127 + q_exp[bb]) << 23);

  floatx4 acc1[NB][8], acc2[NB][8], accl[NB];
  float beta1[NB], beta2[NB];  // sum_r p * b_V over this lane's rows
  float m_run[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc1[bb][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      acc2[bb][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    accl[bb] = floatx4{0.f, 0.f, 0.f, 0.f};
    beta1[bb] = beta2[bb] = 0.f;
    m_run[bb] = kNegSentinel;
  }
  const half4_t ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};

  // Scores, online softmax and both V products of this wave's loaded tiles
  // k0 .. k0 + U - 1.
  auto compute_tiles = [&](const Tile (&T)[U], int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tr = tile_row(k0 + u);
      const int row0 = tr + 4 * blk;  // row of r = 0
      uint32_t sw[NS][2];
#pragma unroll
      for (int t = 0; t < NS; ++t) scale_words<NG>(sw[t], T[u].s[t], sel);
      // Only a tile reaching past max_lim holds rows whose scale words may be
      // stale cache contents; the test is uniform over the wave, so the
      // others branch around the masking.
      if (tr + 16 > max_lim) {
#pragma unroll
        for (int t = 0; t < NS; ++t) drop_rows_past(sw[t], (unsigned)row0, (unsigned)max_lim);
      }
      // Code sums in units of 2^-24: q4 in two chains (low nibbles, high
      // nibbles at 16x), q8 in one.
      floatx4 sacc[NB], shi[NB];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        sacc[bb] = floatx4{0.f, 0.f, 0.f, 0.f};
        shi[bb] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const half8_t ka = k_codes<BITS>(T[u].k, s);
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          if (BITS == 4 && s >= 2)
            shi[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[bb][s], shi[bb], 0, 0, 0);
          else
            sacc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[bb][s], sacc[bb], 0, 0, 0);
        }
      }
      if constexpr (BITS == 4) {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
          for (int r = 0; r < 4; ++r) sacc[bb][r] = fmaf(shi[bb][r], 0.0625f, sacc[bb][r]);
      }
      uint32_t skw[2] = {sw[0][0], sw[0][1]}, bkw[2] = {sw[1][0], sw[1][1]};
      if constexpr (DUAL) {  // the noise head's column: k2 codes and scales
        floatx4 s2 = floatx4{0.f, 0.f, 0.f, 0.f};
        floatx4 s2hi = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const half8_t ka = k_codes<BITS>(T[u].k2, s);
          if (BITS == 4 && s >= 2)
            s2hi = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[0][s], s2hi, 0, 0, 0);
          else
            s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[0][s], s2, 0, 0, 0);
        }
        if constexpr (BITS == 4) {
#pragma unroll
          for (int r = 0; r < 4; ++r) s2[r] = fmaf(s2hi[r], 0.0625f, s2[r]);
        }
        const bool noise = h >= a.G;
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[0][r] = noise ? s2[r] : sacc[0][r];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          skw[p] = noise ? sw[6][p] : skw[p];
          bkw[p] = noise ? sw[7][p] : bkw[p];
        }
      }
      float skr[4], bkr[4];
      if constexpr (kBf16) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          skr[2 * p] = pair_lo_f32<E>(skw[p]);
          skr[2 * p + 1] = pair_hi_f32<E>(skw[p]);
          bkr[2 * p] = pair_lo_f32<E>(bkw[p]);
          bkr[2 * p + 1] = pair_hi_f32<E>(bkw[p]);
        }
        // V scales as fp16 pairs for the weight products (exact in fp16's
        // normal range).
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          sw[2][p] = f16_pair(pair_lo_f32<E>(sw[2][p]), pair_hi_f32<E>(sw[2][p]));
          sw[4][p] = f16_pair(pair_lo_f32<E>(sw[4][p]), pair_hi_f32<E>(sw[4][p]));
        }
      } else {
        const half2_t sk01 = as_h2(skw[0]), sk23 = as_h2(skw[1]);
        const half2_t bk01 = as_h2(bkw[0]), bk23 = as_h2(bkw[1]);
        skr[0] = (float)sk01.x; skr[1] = (float)sk01.y; skr[2] = (float)sk23.x; skr[3] = (float)sk23.y;
        bkr[0] = (float)bk01.x; bkr[1] = (float)bk01.y; bkr[2] = (float)bk23.x; bkr[3] = (float)bk23.y;
      }
      half4_t w1[NB], w2[NB], pbb[NB];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // Unused columns have Q^T = 0 and qsum = 0, so t = 0 there without
          // a select (their scale words are finite cache values or 0).
          const float t = fmaf(skr[r], sacc[bb][r], bkr[r] * qsum[bb]);
          sc[r] = sum_group_columns<GC>(t) * qsc[bb];
        }
        // Rows at or past the column's limit score -inf, so their weight
        // exp2(-inf - m) is 0 with no select (m_run starts at the finite
        // sentinel and only grows); only a tile reaching min_lim holds such
        // rows (a wave-uniform test).
        if (tr + 16 > min_lim) {
          asm volatile("");  // keep this a branch: only tiles at a limit take it
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] = row0 + r < lim[bb] ? sc[r] : -__builtin_inff();
        }
        float mx = kNegSentinel;
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = vmax(mx, sc[r]);
        mx = rows4_max(mx);
        if (__ballot(mx > m_run[bb] + kSlack) != 0) {
          const float m_new = fmaxf(m_run[bb], mx);
          const float fac = fast_exp2(m_run[bb] - m_new);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            acc1[bb][j] *= fac;
            acc2[bb][j] *= fac;
          }
          accl[bb] *= fac;
          beta1[bb] *= fac;
          beta2[bb] *= fac;
          m_run[bb] = m_new;
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          p[r] = fast_exp2(sc[r] - m_run[bb]);
        // p rounded to fp16 once; the V weights, the bias terms and l all
        // use these same values.
        const half2_t p01 = half2_t{(_Float16)p[0], (_Float16)p[1]};
        const half2_t p23 = half2_t{(_Float16)p[2], (_Float16)p[3]};
        pbb[bb] = half4_t{p01.x, p01.y, p23.x, p23.y};
        const half2_t w1a = p01 * as_h2(sw[2][0]), w1b = p23 * as_h2(sw[2][1]);
        const half2_t w2a = p01 * as_h2(sw[4][0]), w2b = p23 * as_h2(sw[4][1]);
        w1[bb] = half4_t{w1a.x, w1a.y, w1b.x, w1b.y};
        w2[bb] = half4_t{w2a.x, w2a.y, w2b.x, w2b.y};
        if constexpr (kBf16) {  // the bias terms in fp32, with the same fp16 weights
          const float pf[4] = {(float)p01.x, (float)p01.y, (float)p23.x, (float)p23.y};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t b1 = sw[3][r / 2], b2 = sw[5][r / 2];
            beta1[bb] = fmaf(pf[r], (r & 1) ? pair_hi_f32<E>(b1) : pair_lo_f32<E>(b1), beta1[bb]);
            beta2[bb] = fmaf(pf[r], (r & 1) ? pair_hi_f32<E>(b2) : pair_lo_f32<E>(b2), beta2[bb]);
          }
        } else {
          beta1[bb] = __builtin_amdgcn_fdot2(p01, as_h2(sw[3][0]), beta1[bb], false);
          beta1[bb] = __builtin_amdgcn_fdot2(p23, as_h2(sw[3][1]), beta1[bb], false);
          beta2[bb] = __builtin_amdgcn_fdot2(p01, as_h2(sw[5][0]), beta2[bb], false);
          beta2[bb] = __builtin_amdgcn_fdot2(p23, as_h2(sw[5][1]), beta2[bb], false);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t x1[4], x2[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x1[r] = T[u].v1[r][BITS == 4 ? 0 : (i >> 2)];
          x2[r] = T[u].v2[r][BITS == 4 ? 0 : (i >> 2)];
        }
        const half4_t a1 = v_codes<BITS>(x1, BITS == 4 ? i : (i & 3));
        const half4_t a2 = v_codes<BITS>(x2, BITS == 4 ? i : (i & 3));
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          acc1[bb][i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a1, w1[bb], acc1[bb][i], 0, 0, 0);
          acc2[bb][i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a2, w2[bb], acc2[bb][i], 0, 0, 0);
        }
      }
#pragma unroll
      for (int bb = 0; bb < NB; ++bb)
        accl[bb] = __builtin_amdgcn_mfma_f32_16x16x16f16(ones, pbb[bb], accl[bb], 0, 0, 0);
    }
  };

  // Two register sets in turn: the loads of the next U tiles are in flight
  // while the current ones are computed, and each set is reloaded as soon as
  // it has been consumed.  (Loading the next set at the top of each
  // iteration instead made the compiler wait there on the set in flight:
  // q8 at 16k 15.05 against 14.85 us per call.  A third set, with two sets'
  // loads in flight, measured slower for q4.)  Sets past the wave's last
  // tile read zeros and cost no traffic.
  int nset = 0;  // tile sets of U tiles this wave visits
  while (tile_row(nset * U) < max_lim) ++nset;
  load_tiles(tb, U);
  for (int n = 0; n < nset; n += 2) {
    compute_tiles(ta, n * U);
    load_tiles(ta, (n + 2) * U);
    if (n + 1 >= nset) break;
    compute_tiles(tb, (n + 1) * U);
    load_tiles(tb, (n + 3) * U);
  }

  // acc[i][r] of lane (col, blk) is channel 8*(4*blk + r) + i for head h; it
  // is valid where that channel's group is the column's group, i.e. where
  // the row block's 32 channels belong to group grp.
  __shared__ __attribute__((aligned(16))) float lds_o[NW][GCW][2 * D + kLdsPad];
  __shared__ float lds_m[NW][GCW];
  __shared__ float lds_l[NW][GCW];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    // Bias terms: sum the four row blocks of each column.
    float be1 = beta1[bb], be2 = beta2[bb];
    be1 += __shfl_xor(be1, 16);
    be1 += __shfl_xor(be1, 32);
    be2 += __shfl_xor(be2, 16);
    be2 += __shfl_xor(be2, 32);
    const int hh = hb[bb];
    if (used[bb] && (32 * blk) / GS == grp) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // Code sums to values: 2^24, or for a q4 high nibble (odd channel)
        // (whole-byte sum - low-nibble sum) * 2^20.
        float o1[8], o2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bool odd4 = BITS == 4 && (i & 1);
          const float f = odd4 ? 0x1p20f : kCodeScale;
          o1[i] = fmaf(odd4 ? acc1[bb][i][r] - acc1[bb][i & ~1][r] : acc1[bb][i][r], f, be1);
          o2[i] = fmaf(odd4 ? acc2[bb][i][r] - acc2[bb][i & ~1][r] : acc2[bb][i][r], f, be2);
        }
        const int ch = 8 * (4 * blk + r);
        *reinterpret_cast<float4*>(&lds_o[wave][hh][ch]) = make_float4(o1[0], o1[1], o1[2], o1[3]);
        *reinterpret_cast<float4*>(&lds_o[wave][hh][ch + 4]) =
            make_float4(o1[4], o1[5], o1[6], o1[7]);
        *reinterpret_cast<float4*>(&lds_o[wave][hh][D + ch]) =
            make_float4(o2[0], o2[1], o2[2], o2[3]);
        *reinterpret_cast<float4*>(&lds_o[wave][hh][D + ch + 4]) =
            make_float4(o2[4], o2[5], o2[6], o2[7]);
      }
    }
    if (col < GC && hh < nvh && blk == 0) {
      lds_m[wave][hh] = m_run[bb];
      lds_l[wave][hh] = accl[bb][0];
    }
  }
  __syncthreads();
  // The in-kernel merge's LDS does not fit beside NB > 1 blocks' staging:
  // those launches always use the merge launch.
  wg_epilogue<E, D, GCW, NW, DUAL, NB == 1>(a, lds_o, lds_m, lds_l, qrow0, nvh, split,
                                                 unit);
}

// Packed cache, head_dim 128, fp16 scales: heads x groups <= 16 columns.
// One tile per register set: with the prefetched set, two tiles' loads are
// in flight per wave while one is computed.
template <int BITS, int GS, typename E = half_t>
int launch_sdpa_mfma_q_gs(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t st) {
  constexpr int NG = 128 / GS;
  constexpr int U = 1;
  constexpr int P = kCachePolicyStream;
  constexpr int GCM = 16 / NG < 8 ? 16 / NG : 8;  // widest pass
  // bf16 variants run one wave per SIMD: 4-wave workgroups only.
  constexpr bool k8 = !std::is_same<E, bf16_t>::value;
  if (a.nchunk > 1 && gc == GCM && (waves == 4 || !k8)) {
    hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, GCM, 4, U, 0, false, 1, E>), dim3(nblocks),
                       dim3(256), 0, st, a);
    return check_launch("sdpa_dual_v_q (mfma, chunks)");
  }
  const bool w8 = k8 && waves == 8;
  switch (gc) {
    case 1:
      if constexpr (k8) {
        if (w8) {
          hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 1, 8, U, P, false, 1, E>), dim3(nblocks), dim3(512), 0, st, a);
          break;
        }
      }
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 1, 4, U, P, false, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 2:
      if constexpr (k8) {
        if (w8) {
          hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 2, 8, U, P, false, 1, E>), dim3(nblocks), dim3(512), 0, st, a);
          break;
        }
      }
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 2, 4, U, P, false, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 4:
      if constexpr (k8) {
        if (w8) {
          hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 4, 8, U, P, false, 1, E>), dim3(nblocks), dim3(512), 0, st, a);
          break;
        }
      }
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 4, 4, U, P, false, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 8:
      if constexpr (8 * NG <= 16) {
        hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 8, 4, U, P, false, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
        break;
      }
      [[fallthrough]];
    default:
      set_error("sdpa_dual_v_q: no MFMA variant for %d heads per workgroup", gc);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("sdpa_dual_v_q (mfma)");
}

// Fused GDA decode step over the packed cache: gc columns per scale group
// (G + G2 rounded up to a power of two, gc * 128 / gs <= 16), 4 waves; E the
// element type of q, the new rows, the scales and biases and y.
template <int BITS, int GS, typename E = half_t>
int launch_gda_decode_mfma_q_gs(const SdpaArgs& a, int gc, int nblocks, hipStream_t st) {
  constexpr int NG = 128 / GS;
  constexpr int P = kCachePolicyStream;
  if (gc * NG > 16 || (gc != 2 && gc != 4 && gc != 8 && gc != 16)) {
    set_error("gda_decode_q: no fused variant for %d columns at group size %d", gc, GS);
    return MOTIF_ERR_UNSUPPORTED;
  }
  if (gc == 2) {
    hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 2, 4, 1, P, true, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
  } else if (gc == 4) {
    if constexpr (4 * NG <= 16)
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 4, 4, 1, P, true, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
  } else if (gc == 8) {
    if constexpr (8 * NG <= 16)
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 8, 4, 1, P, true, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
  } else {
    if constexpr (16 * NG <= 16)
      hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, 16, 4, 1, P, true, 1, E>), dim3(nblocks), dim3(256), 0, st, a);
  }
  return check_launch("gda_decode_q (mfma)");
}

template <typename E = half_t>
inline int launch_gda_decode_mfma_q(const SdpaArgs& a, int bits, int gs, int gc, int nblocks,
                                    hipStream_t st) {
  if (bits == 4) {
    if (gs == 32) return launch_gda_decode_mfma_q_gs<4, 32, E>(a, gc, nblocks, st);
    if (gs == 64) return launch_gda_decode_mfma_q_gs<4, 64, E>(a, gc, nblocks, st);
    return launch_gda_decode_mfma_q_gs<4, 128, E>(a, gc, nblocks, st);
  }
  if (gs == 32) return launch_gda_decode_mfma_q_gs<8, 32, E>(a, gc, nblocks, st);
  if (gs == 64) return launch_gda_decode_mfma_q_gs<8, 64, E>(a, gc, nblocks, st);
  return launch_gda_decode_mfma_q_gs<8, 128, E>(a, gc, nblocks, st);
}

// Two column blocks of GC = 16 / groups (at most 8) heads per wave, one
// head chunk (all virtual heads of the KV head in one workgroup).
template <int BITS, int GS>
int launch_sdpa_mfma_q_wide_gs(const SdpaArgs& a, int nb, int nblocks, hipStream_t st) {
  constexpr int NG = 128 / GS;
  constexpr int GC = 16 / NG < 8 ? 16 / NG : 8;
  if (nb != 2 || a.nchunk != 1) {
    set_error("sdpa_dual_v_q: no variant with %d column blocks and %d head chunks", nb,
              a.nchunk);
    return MOTIF_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((sdpa_mfma_q_kernel<BITS, GS, GC, 4, 1, kCachePolicyStream, false, 2>),
                     dim3(nblocks), dim3(256), 0, st, a);
  return check_launch("sdpa_dual_v_q (mfma, column blocks)");
}

inline int launch_sdpa_mfma_q_wide(const SdpaArgs& a, int bits, int gs, int nb, int nblocks,
                                   hipStream_t st) {
  if (bits == 4) {
    if (gs == 32) return launch_sdpa_mfma_q_wide_gs<4, 32>(a, nb, nblocks, st);
    if (gs == 64) return launch_sdpa_mfma_q_wide_gs<4, 64>(a, nb, nblocks, st);
    return launch_sdpa_mfma_q_wide_gs<4, 128>(a, nb, nblocks, st);
  }
  if (gs == 32) return launch_sdpa_mfma_q_wide_gs<8, 32>(a, nb, nblocks, st);
  if (gs == 64) return launch_sdpa_mfma_q_wide_gs<8, 64>(a, nb, nblocks, st);
  return launch_sdpa_mfma_q_wide_gs<8, 128>(a, nb, nblocks, st);
}

template <typename E = half_t>
inline int launch_sdpa_mfma_q(const SdpaArgs& a, int bits, int gs, int gc, int waves, int nblocks,
                              hipStream_t st) {
  if (bits == 4) {
    if (gs == 32) return launch_sdpa_mfma_q_gs<4, 32, E>(a, gc, waves, nblocks, st);
    if (gs == 64) return launch_sdpa_mfma_q_gs<4, 64, E>(a, gc, waves, nblocks, st);
    return launch_sdpa_mfma_q_gs<4, 128, E>(a, gc, waves, nblocks, st);
  }
  if (gs == 32) return launch_sdpa_mfma_q_gs<8, 32, E>(a, gc, waves, nblocks, st);
  if (gs == 64) return launch_sdpa_mfma_q_gs<8, 64, E>(a, gc, waves, nblocks, st);
  return launch_sdpa_mfma_q_gs<8, 128, E>(a, gc, waves, nblocks, st);
}

}  // namespace motif
