// Matrix-core (MFMA) formulation of split-KV dual-V decode for head_dim 128.
//
// The VALU formulation spends ~3k lane-instructions per KV row (dot products,
// DPP reductions, per-head FMAs into two value slabs), which caps it far
// below the HBM roofline.  Here one wave processes 16 KV rows per step with
// matrix instructions, the virtual heads (GQA heads x query rows) riding the
// 16 columns of the MFMA:
//
//   S^T (16 rows x 16 heads) = K (16 x 128) . Q^T (128 x 16)
//       4 x v_mfma_f32_16x16x32_f16; A = K rows exactly as stored (each lane
//       reads 16 contiguous bytes of one row per step), B = Q^T held in
//       registers for the whole split.
//   O^T (128 ch x 16 heads) += V^T (128 x 16 rows) . P^T (16 rows x 16 heads)
//       8 x v_mfma_f32_16x16x16_f16 per value slab.  The C layout of S^T
//       (lane l: rows 4*(l/16)+r, head l%16) is exactly the B layout P^T
//       needs, so softmax weights never move between lanes.  V^T fragments
//       (4 rows x 1 channel per lane) come from 16-byte row loads (8
//       channels of one row per lane, four whole rows per instruction)
//       paired across rows with one v_perm_b32 per 2 values.
//   l (16 heads) += ones . P^T: one extra MFMA sums the same fp16-rounded
//       weights that multiply V, so o/l is consistent.
//
// Softmax state per head (column): running max in log2 units, shared by
// the 4 lanes of the column; accumulators are rescaled only when some
// column's max grows (wave-uniform branch).  The workgroup epilogue
// (cross-wave LDS merge, split partials, last-arrival merge) is shared with
// the VALU kernel.
#pragma once

#include "rope_impl.hpp"
#include "sdpa_impl.hpp"

namespace motif {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Matrix-core operands of a 16-bit cache element type: the 8-element A/B
// vector of v_mfma_f32_16x16x32_{f16,bf16} and the rounding of the softmax
// weights p to that type (both MFMA operands share it).  K, V and q enter
// the MFMAs exactly as stored.
template <typename T>
struct MfmaOp;
template <>
struct MfmaOp<half_t> {
  typedef half8_t V8;
  typedef _Float16 S;
  __device__ static inline floatx4 mma(V8 a, V8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline S from_f32(float x) { return (S)x; }
};
template <>
struct MfmaOp<bf16_t> {
  typedef bf16x8_t V8;
  typedef __bf16 S;
  __device__ static inline floatx4 mma(V8 a, V8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline S from_f32(float x) { return (S)x; }  // round to nearest even
};

// Lazy rescaling.  The reference point m_run of the online softmax is raised
// only when a tile's max exceeds it by more than a slack (log2 units); until
// then p = exp2(s - m_run) may exceed 1, up to 2^slack.  o and l share the
// reference point, so o / l and the split partials (m_run, l, o) are the
// same quantities as with an exact running max, and most tiles skip the
// rescale of the 68 accumulator registers.  The slack only bounds p, which
// the matrix cores take as fp16 or bf16: 2^8 leaves p a wide margin.
constexpr float kRescaleSlackF16 = 8.f;

// Lane l receives its own value and lane l ^ 16's (in row order: rows 0/1
// hold (row 0, row 1) of the pair, rows 2/3 (row 2, row 3)); likewise l ^ 32
// for the 32-lane swap.  Issued as asm: at -O3 the compiler folds the second
// result of __builtin_amdgcn_permlane16_swap into the first, which breaks a
// swap of one value against itself.  The s_nops cover the VALU-write ->
// permlane-read and permlane-write -> VALU-read hazards.
__device__ inline void swap16(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline void swap32(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// Max over the four 16-lane rows (lanes l, l^16, l^32, l^48): every lane
// receives the same value.
__device__ inline float rows4_max(float x) {
  float a, b;
  swap16(x, a, b);
  swap32(vmax(a, b), a, b);
  return vmax(a, b);
}
// Sum over the four 16-lane rows; every lane receives the same bits (the
// operands of each add are the same pair, in the same order, on both
// partners).
__device__ inline float rows4_sum(float x) {
  float a, b;
  swap16(x, a, b);
  swap32(a + b, a, b);
  return a + b;
}

// Causal row limit of query row s (see sdpa_dual_v_kernel).
__device__ inline int row_limit(const SdpaArgs& a, int s) {
  int L = a.causal ? a.kv_len - a.S_q + s + 1 : a.kv_len;
  return L < 0 ? 0 : (L > a.kv_len ? a.kv_len : L);
}
// Causal row limit of virtual head vh (query row vh % S_q).
__device__ inline int vhead_limit(const SdpaArgs& a, int vh) { return row_limit(a, vh % a.S_q); }
// Largest (hi) and smallest (lo) vhead_limit over the virtual heads v0 ..
// v0 + n - 1 without a division per head: the limit grows with the query
// row, so the extremes sit at the range's first and last rows, or at rows
// S_q - 1 and 0 once the range crosses into the next head.  n <= 0: hi 0, lo
// kv_len (the empty maximum and minimum).
__device__ inline void vhead_limit_range(const SdpaArgs& a, int v0, int n, int& lo, int& hi) {
  if (n <= 0) {
    lo = a.kv_len;
    hi = 0;
    return;
  }
  const int s0 = v0 % a.S_q;
  const bool wraps = s0 + n > a.S_q;
  lo = row_limit(a, wraps ? 0 : s0);
  hi = row_limit(a, wraps ? a.S_q - 1 : s0 + n - 1);
}
__device__ inline int vhead_limit_max(const SdpaArgs& a, int v0, int n) {
  int lo, hi;
  vhead_limit_range(a, v0, n, lo, hi);
  return hi;
}

// Append (fused decode step): the wave whose tiles include row kv_len - 1
// of this KV head stores the new token's four slot rows there.  Tile T of a
// KV head is tile k of wave T % NW in split (T / NW) % nsplit.
template <int NW>
__device__ inline bool append_owner(const SdpaArgs& a, int split, int wave) {
  if (!a.append || a.kv_len < 1) return false;
  const int t = (a.kv_len - 1) / 16;
  return wave == t % NW && split == (t / NW) % a.nsplit;
}

// 16-bit rows of 128 values: lane L copies 16 bytes (chunk L % 16) of slot
// L / 16 (k1, k2, v1, v2) into row kv_len - 1 of KV head bk.  From the
// projections (a.from_proj), the k rows are roped first: chunk c < 8 holds
// the first halves of the pairs whose second halves are in chunk c + 8,
// i.e. in lane L ^ 8.  Called by a whole wave.
template <typename T>
__device__ inline void append_rows_16bit(const SdpaArgs& a, long bk, int lane) {
  const int slot = lane / 16;
  const int chunk = lane % 16;
  const void* dst = slot == 0 ? a.k : slot == 1 ? a.k2 : slot == 2 ? a.v1 : a.v2;
  uint4 w;
  if (!a.from_proj) {
    const void* src =
        slot == 0 ? a.new_k1 : slot == 1 ? a.new_k2 : slot == 2 ? a.new_v1 : a.new_v2;
    w = *reinterpret_cast<const uint4*>((const uint8_t*)src + bk * 256 + chunk * 16);
  } else {
    // head 2 * kvh + (slot & 1) of position b: row 2 * bk + (slot & 1)
    const void* src = slot < 2 ? a.new_k1 : a.new_v1;
    w = *reinterpret_cast<const uint4*>((const uint8_t*)src + (2 * bk + (slot & 1)) * 256 +
                                        chunk * 16);
    uint32_t x[4] = {w.x, w.y, w.z, w.w}, o[4];
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (uint32_t)__shfl_xor((int)x[i], 8);  // partner chunk
    const bool first = chunk < 8;
    const int pos = a.kv_len - 1;
    // Lane L computes the angle of pair L (0..63) once; the lanes read the
    // eight they need with __shfl (one slow-path sincosf per lane, not eight).
    float cs0, sn0;
    rope_angle((int)(threadIdx.x & 63u), 128, pos, a.rope_log2_theta, a.rope_pos_scale, cs0, sn0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t r = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint16_t mine = (uint16_t)(e ? x[i] >> 16 : x[i] & 0xFFFFu);
        const uint16_t other = (uint16_t)(e ? o[i] >> 16 : o[i] & 0xFFFFu);
        const float x1 = Elem<T>::to_f32(first ? mine : other);
        const float x2 = Elem<T>::to_f32(first ? other : mine);
        const float cs = __shfl(cs0, 8 * (chunk & 7) + 2 * i + e);
        const float sn = __shfl(sn0, 8 * (chunk & 7) + 2 * i + e);
        float y1, y2;
        rope_rotate(x1, x2, cs, sn, y1, y2);
        r |= (uint32_t)Elem<T>::from_f32(first ? y1 : y2) << (16 * e);
      }
      y[i] = slot < 2 ? r : x[i];  // v rows are copied
    }
    w = make_uint4(y[0], y[1], y[2], y[3]);
  }
  *reinterpret_cast<uint4*>((uint8_t*)const_cast<void*>(dst) +
                            (bk * a.kv_cap + a.kv_len - 1) * 256 + chunk * 16) = w;
}

// DUAL: fused GDA decode step.  Columns 0..G-1 are the origin heads of the
// KV head (scores from k), columns G..G+G2-1 its noise heads (scores from
// k2; G2 = a.G2, one in the 12.7B layout); all share the V1/V2 rows, and
// the partials go to the fused merge launch.
// T: half_t (fp16 cache, v_mfma_f32_16x16x32_f16) or bf16_t (bf16 cache,
// v_mfma_f32_16x16x32_bf16).  The 16-column single-pass variant keeps the
// in-kernel merge's LDS (104 KB): one workgroup, one wave per SIMD, per CU.
template <typename T, int GC, int NW, int U, bool DUAL = false, int D = 128>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(GC == 16 && !DUAL ? 1 : 2)))
sdpa_mfma_kernel(SdpaArgs a) {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
  // head_dim 128 or 64: NQ k-steps of 32 channels for S^T, and VT dwords
  // (2 VT channels) of each V row per lane, 2 VT MFMAs per V for O^T.
  static_assert(D == 128 || D == 64, "head_dim 128 or 64");
  static_assert(!DUAL || D == 128, "the fused decode step is built for head_dim 128");
  constexpr int NQ = D / 32;
  constexpr int VT = D / 32;
  static_assert(GC <= 16, "virtual heads ride the 16 MFMA columns");
  static_assert(U % 2 == 0, "tiles are computed in pairs");
  const int lane = threadIdx.x & 63;
  // Wave index as a wave-uniform (scalar) value: tile rows and the tests on
  // them are then scalar, and so are the branches that depend on them.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;  // MFMA column: virtual head (S^T, P^T, O^T)
  const int blk = lane >> 4;  // MFMA k/row block

  int unit, split;
  if (!sdpa_block_coords(a, blockIdx.x, unit, split)) return;  // grid padding
  const int chunk = unit % a.nchunk;
  const int bk = unit / a.nchunk;
  const int b = bk / a.Hkv;
  const int kvh = bk % a.Hkv;
  const int vh0 = chunk * GC;
  const int nvh = min(GC, a.GV - vh0);
  // First output row: y row (non-DUAL) or partial row (DUAL) of column 0.
  const long qrow0 = DUAL ? ((long)b * a.Hkv + kvh) * (a.G + a.G2)
                          : ((long)b * a.Hq + (long)kvh * a.G) * a.S_q + vh0;

  // Rows below min_lim are visible to every column of the workgroup.
  int min_lim, max_lim;
  vhead_limit_range(a, vh0, nvh, min_lim, max_lim);
  const bool col_ok = col < nvh;
  const int lim = col_ok ? vhead_limit(a, vh0 + col) : 0;  // <= max_lim

  // Append: issue the new rows' stores first; the owner waits for them
  // before the loads of the tile that holds row kv_len - 1.
  bool owner = false;
  if constexpr (DUAL) {
    owner = append_owner<NW>(a, split, wave);
    if (owner) append_rows_16bit<T>(a, bk, lane);
  }

  // Q^T, B operand of the 16x16x32 MFMA: lane (col, blk) holds head col,
  // channels 32*s + 8*blk .. +7 for k-step s.
  V8 qb[NQ];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (col_ok ? col : 0)) * D + 8 * blk;
    if constexpr (DUAL) {
      if (a.from_proj) {  // q_proj heads (G2 == 1): stripe g*(G+1)+j, or origin-first
        const int head = a.q_origin_first
                             ? (col < a.G ? kvh * a.G + col : a.Hkv * a.G + kvh)
                             : kvh * (a.G + 1) + (col < a.G ? col : a.G);
        qp = (const uint16_t*)a.q + ((long)b * a.Hkv * (a.G + 1) + head) * D;
      } else {  // noise column G + i: q2 head kvh * G2 + i
        qp = col < a.G
                 ? (const uint16_t*)a.q + ((long)b * a.Hq + (long)kvh * a.G + col) * D
                 : (const uint16_t*)a.q2 + (((long)b * a.Hkv + kvh) * a.G2 + (col - a.G)) * D;
      }
      qp += 8 * blk;
    }
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      const uint4 w = col_ok ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
      qb[s] = __builtin_bit_cast(V8, w);
    }
    if constexpr (DUAL) {
      if (a.from_proj) {  // RoPE at kv_len - 1: channel 32s + 8blk + j pairs with s + 2
        // The 16 angles of a row block are the same for its 16 columns: lane
        // (col, blk) computes angle (s, j) = (col / 8, col % 8) and the
        // others are read from the lanes of its block.
        float cs0, sn0;
        rope_angle(32 * (col >> 3) + 8 * blk + (col & 7), 128, a.kv_len - 1, a.rope_log2_theta,
                   a.rope_pos_scale, cs0, sn0);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float cs = __shfl(cs0, 16 * blk + 8 * s + j);
            const float sn = __shfl(sn0, 16 * blk + 8 * s + j);
            float y1, y2;
            rope_rotate((float)qb[s][j], (float)qb[s + 2][j], cs, sn, y1, y2);
            qb[s][j] = Op::from_f32(y1);
            qb[s + 2][j] = Op::from_f32(y2);
          }
        }
      }
    }
  }


  floatx4 acc1[2 * VT], acc2[2 * VT], accl;
#pragma unroll
  for (int j = 0; j < 2 * VT; ++j) {
    acc1[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  accl = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegSentinel;
  const typename Op::S one = Op::from_f32(1.f);
  const V8 ones = {one, one, one, one, one, one, one, one};

  // Rows are dealt to the splits in blocks of NW 16-row tiles, round robin:
  // tile k of wave w in split s is tile (k * nsplit + s) * NW + w of the KV
  // head.  At any moment the workgroups of a KV head then stream one
  // contiguous stretch of the cache together; contiguous per-split row
  // ranges measured ~2 us slower at 16k rows (the loads alone, 32 splits:
  // 17.8 vs 15.8 us).  The resources cover rows [0, max_lim) of the KV head,
  // so rows past it read 0; offsets stay 32-bit (kv_len <= kMfmaMaxRows,
  // checked on the host).
  const long hrow0 = (long)bk * a.kv_cap;  // first cache row of this KV head
  const unsigned nbytes = (unsigned)(max_lim * D * 2);
  const auto rk = stream_rsrc((const uint16_t*)a.k + hrow0 * D, nbytes);
  const auto rv1 = stream_rsrc((const uint16_t*)a.v1 + hrow0 * D, nbytes);
  const auto rv2 = stream_rsrc((const uint16_t*)a.v2 + hrow0 * D, nbytes);
  const auto rk2 = DUAL ? stream_rsrc((const uint16_t*)a.k2 + hrow0 * D, nbytes) : rk;
  const int ns = a.nsplit;
  auto tile_row = [&](int k) { return 16 * ((k * ns + split) * NW + wave); };

  // U tiles per wave per iteration: all of their loads are issued before
  // any of them is consumed, so a wave keeps U x 12 KB in flight.
  for (int k0 = 0; tile_row(k0) < max_lim; k0 += U) {
    if constexpr (DUAL) {
      if (owner) {
        bool has = false;
#pragma unroll
        for (int u = 0; u < U; ++u) has |= tile_row(k0 + u) == (a.kv_len - 1) / 16 * 16;
        if (has) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the new rows are stored
      }
    }
    V8 ka[U][NQ];
    V8 ka2[DUAL ? U : 1][NQ];
    uint32_t v1w[U][4][VT], v2w[U][4][VT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t0 = tile_row(k0 + u);
      // K rows for S^T: row t0 + col (A operand row = lane % 16).
      const unsigned koff = (unsigned)((t0 + col) * D * 2 + 16 * blk);
#pragma unroll
      for (int s = 0; s < NQ; ++s) ka[u][s] = __builtin_bit_cast(V8, bload4(rk, koff + 64u * s));
      if constexpr (DUAL) {
#pragma unroll
        for (int s = 0; s < NQ; ++s)
          ka2[u][s] = __builtin_bit_cast(V8, bload4(rk2, koff + 64u * s));
      }
      // V rows t0 + 4*blk + r: 4 VT bytes per lane, dwords VT*col ..
      // VT*col + VT - 1 (dword VT*col + t holds channels 2*VT*col + 2t, +1);
      // one instruction covers four whole rows.
      const unsigned voff = (unsigned)((t0 + 4 * blk) * D * 2 + 4 * VT * col);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (VT == 4) {
          const uint4 w1 = bload4(rv1, voff + (unsigned)(r * D * 2));
          const uint4 w2 = bload4(rv2, voff + (unsigned)(r * D * 2));
          v1w[u][r][0] = w1.x; v1w[u][r][1] = w1.y; v1w[u][r][2] = w1.z; v1w[u][r][3] = w1.w;
          v2w[u][r][0] = w2.x; v2w[u][r][1] = w2.y; v2w[u][r][2] = w2.z; v2w[u][r][3] = w2.w;
        } else {
          const uint2 w1 = bload2(rv1, voff + (unsigned)(r * D * 2));
          const uint2 w2 = bload2(rv2, voff + (unsigned)(r * D * 2));
          v1w[u][r][0] = w1.x; v1w[u][r][1] = w1.y;
          v2w[u][r][0] = w2.x; v2w[u][r][1] = w2.y;
        }
      }
    }

    // Every load of the U tiles is issued before the first product (the
    // scheduler would otherwise hold some back until the first K rows land).
    __builtin_amdgcn_sched_barrier(0);

    // Tiles in pairs: the PV products take both tiles' 32 rows in one
    // 16x16x32 MFMA (k = 8*blk + j is row 4*blk + j of the pair's first
    // tile for j < 4, row 4*blk + j - 4 of its second for j >= 4), with one
    // running-max update per pair.
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      floatx4 sacc[2];
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        sacc[v] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NQ; ++s)
          sacc[v] = Op::mma(ka[u + v][s], qb[s], sacc[v]);
        if constexpr (DUAL) {
          floatx4 s2 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < NQ; ++s)
            s2 = Op::mma(ka2[u + v][s], qb[s], s2);
          if (col >= a.G) sacc[v] = s2;
        }
      }

      // Scores of rows t_v + 4*blk + r for head col, log2 units.  Rows at or
      // past the column's limit score -inf, so their weight exp2(-inf - m)
      // is 0 with no select (m_run starts at the finite sentinel and only
      // grows); only a pair reaching min_lim holds such rows (a wave-uniform
      // test).
      float sc[8];
#pragma unroll
      for (int v = 0; v < 2; ++v) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[4 * v + r] = sacc[v][r] * a.qscale;
      }
      if (tile_row(k0 + u + 1) + 16 > min_lim) {
        asm volatile("");  // keep this a branch: only pairs at a limit take it
#pragma unroll
        for (int v = 0; v < 2; ++v) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = tile_row(k0 + u + v) + 4 * blk + r;
            sc[4 * v + r] = row < lim ? sc[4 * v + r] : -__builtin_inff();
          }
        }
      }
      float mx = kNegSentinel;
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = vmax(mx, sc[j]);
      mx = rows4_max(mx);
      if (__ballot(mx > m_run + kRescaleSlackF16) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float fac = fast_exp2(m_run - m_new);
#pragma unroll
        for (int j = 0; j < 2 * VT; ++j) {
          acc1[j] *= fac;
          acc2[j] *= fac;
        }
        accl *= fac;
        m_run = m_new;
      }
      V8 pb;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        pb[j] = Op::from_f32(fast_exp2(sc[j] - m_run));

#pragma unroll
      for (int t = 0; t < VT; ++t) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t sel = h ? 0x07060302u : 0x05040100u;  // hi or lo halves, row r in half r%2
          const V8 a1 = __builtin_bit_cast(
              V8, make_uint4(__builtin_amdgcn_perm(v1w[u][1][t], v1w[u][0][t], sel),
                                  __builtin_amdgcn_perm(v1w[u][3][t], v1w[u][2][t], sel),
                                  __builtin_amdgcn_perm(v1w[u + 1][1][t], v1w[u + 1][0][t], sel),
                                  __builtin_amdgcn_perm(v1w[u + 1][3][t], v1w[u + 1][2][t], sel)));
          const V8 a2 = __builtin_bit_cast(
              V8, make_uint4(__builtin_amdgcn_perm(v2w[u][1][t], v2w[u][0][t], sel),
                                  __builtin_amdgcn_perm(v2w[u][3][t], v2w[u][2][t], sel),
                                  __builtin_amdgcn_perm(v2w[u + 1][1][t], v2w[u + 1][0][t], sel),
                                  __builtin_amdgcn_perm(v2w[u + 1][3][t], v2w[u + 1][2][t], sel)));
          acc1[2 * t + h] = Op::mma(a1, pb, acc1[2 * t + h]);
          acc2[2 * t + h] = Op::mma(a2, pb, acc2[2 * t + h]);
        }
      }
      accl = Op::mma(ones, pb, accl);
    }
  }

  // O^T element (m = 4*blk + r, head col) of MFMA j = 2*t + h is channel
  // 2*VT*m + j.
  __shared__ __attribute__((aligned(16))) float lds_o[NW][GC][2 * D + kLdsPad];
  __shared__ float lds_m[NW][GC];
  __shared__ float lds_l[NW][GC];
  if (col < nvh) {
    // acc[j][r] is channel 2*VT*m + j with m = 4*blk + r: VT / 2 float4 per
    // row m.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ch = 2 * VT * (4 * blk + r);
#pragma unroll
      for (int f = 0; f < VT / 2; ++f) {
        *reinterpret_cast<float4*>(&lds_o[wave][col][ch + 4 * f]) =
            make_float4(acc1[4 * f][r], acc1[4 * f + 1][r], acc1[4 * f + 2][r], acc1[4 * f + 3][r]);
        *reinterpret_cast<float4*>(&lds_o[wave][col][D + ch + 4 * f]) =
            make_float4(acc2[4 * f][r], acc2[4 * f + 1][r], acc2[4 * f + 2][r], acc2[4 * f + 3][r]);
      }
    }
    if (blk == 0) {
      lds_m[wave][col] = m_run;
      lds_l[wave][col] = accl[0];
    }
  }
  __syncthreads();
  wg_epilogue<T, D, GC, NW, DUAL>(a, lds_o, lds_m, lds_l, qrow0, nvh, split, unit);
}

// 16-bit cache (T = half_t or bf16_t), head_dim D (128 or 64), <= 16
// virtual heads per workgroup (16: 4 waves, for the cross-wave LDS merge).
template <typename T, int D = 128>
inline int launch_sdpa_mfma_16(const SdpaArgs& a, int gc, int waves, int nblocks,
                               hipStream_t stream) {
  switch (gc) {
    case 1:
      if (waves == 8) {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 1, 8, 2, false, D>), dim3(nblocks), dim3(8 * 64), 0, stream, a);
      } else {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 1, 4, 2, false, D>), dim3(nblocks), dim3(4 * 64), 0, stream, a);
      }
      break;
    case 2:
      if (waves == 8) {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 2, 8, 2, false, D>), dim3(nblocks), dim3(8 * 64), 0, stream, a);
      } else {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 2, 4, 2, false, D>), dim3(nblocks), dim3(4 * 64), 0, stream, a);
      }
      break;
    case 4:
      if (waves == 8) {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 4, 8, 2, false, D>), dim3(nblocks), dim3(8 * 64), 0, stream, a);
      } else {
        hipLaunchKernelGGL((sdpa_mfma_kernel<T, 4, 4, 2, false, D>), dim3(nblocks), dim3(4 * 64), 0, stream, a);
      }
      break;
    case 8:
      hipLaunchKernelGGL((sdpa_mfma_kernel<T, 8, 4, 2, false, D>), dim3(nblocks), dim3(4 * 64), 0, stream, a);
      break;
    case 16:
      hipLaunchKernelGGL((sdpa_mfma_kernel<T, 16, 4, 2, false, D>), dim3(nblocks), dim3(4 * 64), 0, stream, a);
      break;
    default:
      set_error("sdpa_dual_v: no MFMA variant for %d heads per workgroup", gc);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("sdpa_dual_v (mfma)");
}

// Fused GDA decode step, 16-bit cache, head_dim 128: gc = columns (G + G2,
// rounded up to 2, 4, 8 or 16); waves 8, or 4 (short contexts: one
// workgroup per CU reaches its first tile sooner).  16 columns: always 4.
template <typename T>
inline int launch_gda_decode_mfma_16(const SdpaArgs& a, int gc, int waves, int nblocks,
                                     hipStream_t st) {
  const bool w8 = waves == 8;
  switch (gc) {
    case 2:
      if (w8) hipLaunchKernelGGL((sdpa_mfma_kernel<T, 2, 8, 2, true>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_kernel<T, 2, 4, 2, true>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 4:
      if (w8) hipLaunchKernelGGL((sdpa_mfma_kernel<T, 4, 8, 2, true>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_kernel<T, 4, 4, 2, true>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 8:
      if (w8) hipLaunchKernelGGL((sdpa_mfma_kernel<T, 8, 8, 2, true>), dim3(nblocks), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((sdpa_mfma_kernel<T, 8, 4, 2, true>), dim3(nblocks), dim3(256), 0, st, a);
      break;
    case 16: hipLaunchKernelGGL((sdpa_mfma_kernel<T, 16, 4, 2, true>), dim3(nblocks), dim3(256), 0, st, a); break;
    default:
      set_error("gda_decode: no fused variant for %d columns", gc);
      return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("gda_decode (mfma)");
}

}  // namespace motif
