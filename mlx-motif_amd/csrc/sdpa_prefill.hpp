// Multi-row (chunked-prefill / long verify) dual-V attention over the fp16
// cache at head_dim 128, on matrix cores with K/V tiles shared through LDS.
//
// The split-KV decode kernel gives each workgroup at most 16 virtual heads
// (query head x query row) and re-reads every KV row once per head chunk,
// which for S_q rows of a prefill means G*S_q/16 reads of the cache.  Here a
// workgroup holds NW waves x 16 virtual heads (consecutive query rows of one
// head), and every 32-row K/V tile is loaded from HBM once per workgroup into
// LDS and read by all of its waves:
//   - staging: tiles are copied from HBM straight into a ring of NS LDS
//     stages (buffer loads with the LDS-direct bit, no registers), NS - 1
//     tiles ahead of the one being computed; the waves share each tile's 24
//     1-KB copies, wait for their own copies, then meet at one barrier per
//     tile.  Within a 256-byte row, 16-byte chunk c sits at position
//     c ^ (row % 16), so the K reads (16 rows, one chunk) and the V reads
//     (one row, 16 chunks) are free of bank conflicts;
//   - per wave: S^T = K Q^T (16x16x32 MFMA, two 16-row halves), online
//     softmax in log2 units with lazy rescaling, O^T = V^T P^T over the 32
//     rows as 16x16x32 MFMAs, exactly as the decode kernel does in registers;
//   - rows are split over workgroups only when the query blocks alone do not
//     fill the GPU; splits publish (m, l, o) partials to the merge launch.
// The causal limit is per column (bottom-right alignment), and a workgroup
// streams only the rows its columns can see.
#pragma once

#include "sdpa_mfma_q.hpp"

namespace motif {

constexpr int kPrefillTileRows = 32;
constexpr int kPrefillStages = 4;  // LDS ring: 4 x 24 KB

// 16 bytes per lane from byte offset voff of the range-checked resource r
// (past its end: zeros) into LDS at lds_base + 16 * lane.  Issued as asm so
// that the compiler neither waits on these copies at barriers nor before LDS
// reads; the kernel waits with wait_vm<>() / wait_vm_groups<>().
__device__ inline void lds_copy16_rsrc(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(r)
               : "memory");
}
__device__ inline unsigned lds_byte_addr(const void* p) {
  return (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
// 4 16-bit values through ds_read_b64_tr_b16 (gfx950) from an 8-byte
// aligned LDS address: within each 16-lane group, lane i receives element
// i % 4 of the 8 bytes addressed by lane 4*k + i/4 in slot k (k = 0..3).
// Returned as their 64 bits (slot k in bits 16k .. 16k + 15).
__device__ inline uint2 lds_read_tr16(const void* p) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t* lds_s4_ptr;
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_ptr)(p));
  return __builtin_bit_cast(uint2, v);
}

// Waits on this wave's outstanding vector memory operations (at most N
// left); also a compiler barrier for memory accesses.
template <int N>
__device__ inline void prefill_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// prefill_wait_vm<n * L>() for a wave-uniform n in [0, NMAX].
template <int L, int NMAX>
__device__ inline void prefill_wait_vm_groups(int n) {
  if constexpr (NMAX > 0) {
    if (n >= NMAX) {
      prefill_wait_vm<NMAX * L>();
      return;
    }
    prefill_wait_vm_groups<L, NMAX - 1>(n);
  } else {
    prefill_wait_vm<0>();
  }
}

// Workgroup -> (query block, (b, KV head) unit, split), as sdpa_block_coords
// places head chunks: workgroups are dealt to the 8 XCDs round robin, and
// the query blocks of one (b, KV head, split) share an XCD, so its K/V
// tiles are fetched into that XCD's L2 once and read there by every query
// block.  Groups of 8 (unit, split) pairs are padded; padding blocks exit.
__device__ inline bool prefill_block_coords(const SdpaArgs& a, int bid, int& qblk, int& unit,
                                            int& split) {
  const int bh = a.B * a.Hkv;
  const int slot = bid >> 3;
  qblk = slot % a.nchunk;
  const int g = (slot / a.nchunk) * 8 + (bid & 7);  // g = split * bh + unit
  if (g >= bh * a.nsplit) return false;
  split = g / bh;
  unit = g % bh;
  return true;
}

// One column's online-softmax state over 32-row fp16/bf16 K/V tiles held in
// LDS with 16-byte chunk c of row r at byte r * 256 + (c ^ (r % 16)) * 16:
// S^T = K Q^T (16x16x32 MFMA, two 16-row halves), scores in log2 units with
// lazy rescaling, O^T = V^T P^T over the 32 rows.  Lane (col, blk) of a wave
// owns column col; acc[j][r] ends as channel 32*blk + 4*j + r.
template <typename T>
struct SwizzledTileAcc {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
  floatx4 acc1[8], acc2[8], accl;
  float m_run;

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc1[j] = floatx4{0.f, 0.f, 0.f, 0.f};
      acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    accl = floatx4{0.f, 0.f, 0.f, 0.f};
    m_run = kNegSentinel;
  }

  // S^T = K Q^T of a tile (unscaled): sacc[h][r] is the score of row
  // 16*h + 4*blk + r for column col.  Issued on its own so that a loop can
  // start the next tile's products before this tile's softmax.
  __device__ __forceinline__ static void scores(const uint8_t* Kt, const V8 (&qb)[4],
                                                floatx4 (&sacc)[2], int col, int blk) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sacc[h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kr = 16 * h + col;
        const V8 ka = __builtin_bit_cast(
            V8, *reinterpret_cast<const uint4*>(&Kt[kr * 256 + (((4 * s + blk) ^ (kr % 16)) * 16)]));
        sacc[h] = Op::mma(ka, qb[s], sacc[h]);
      }
    }
  }

  // Mask and online softmax of a tile with scores sacc: returns P^T, the B
  // operand of the PV products, after rescaling the accumulators when the
  // running maximum moved past the lazy-rescale slack.  Rows row0 + 16*h +
  // 4*blk + r of the tile hold k index 8*blk + 4*h + r of the PV products (as
  // in the decode kernel); rows at or past r_end or lim are masked.
  // Masked rows score -inf, so their weight exp2(-inf - m) is 0 with no
  // select (m_run starts at the finite sentinel and only grows).  The
  // maximum is taken over the unscaled scores (qscale > 0, so scaling it
  // gives the maximum of the scaled ones bit for bit) and each weight is
  // exp2(fma(s, qscale, -m)).  full (wave-uniform): every row of the tile is
  // visible to every column of the wave, so no row is masked.
  __device__ __forceinline__ V8 softmax(const floatx4 (&sacc)[2], int row0, int r_end, int lim,
                                        float qscale, int blk, bool full) {
    float sc[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 * h + r] = sacc[h][r];
    }
    if (!full) {
      asm volatile("");  // keep this a branch: only tiles at a limit take it
      // row 16*h + 4*blk + r of the tile is visible while 16*h + r < vis
      const int vis = min(r_end, lim) - row0 - 4 * blk;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sc[4 * h + r] = 16 * h + r < vis ? sc[4 * h + r] : -__builtin_inff();
      }
    }
    float mx = vmax(vmax(vmax(sc[0], sc[1]), vmax(sc[2], sc[3])),
                    vmax(vmax(sc[4], sc[5]), vmax(sc[6], sc[7])));
    mx = fmaxf(rows4_max(mx) * qscale, kNegSentinel);
    if (__ballot(mx > m_run + kRescaleSlackF16) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float fac = fast_exp2(m_run - m_new);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc1[j] *= fac;
        acc2[j] *= fac;
      }
      accl *= fac;
      m_run = m_new;
    }
    V8 pb;
#pragma unroll
    for (int j = 0; j < 8; ++j) pb[j] = Op::from_f32(fast_exp2(fmaf(sc[j], qscale, -m_run)));
    return pb;
  }

  // Both PV products and l of a tile with softmax weights pb.
  __device__ __forceinline__ void pv(const V8& pb, const uint8_t* V1t, const uint8_t* V2t, int col,
                                     int blk) {
    // V^T fragments straight from LDS with transposing reads
    // (ds_read_b64_tr_b16).  In the 16-lane group of lanes with one blk,
    // lane 4*jj + q points at 4 channels of row 16*h + 4*blk + jj, and group
    // lane i receives element i % 4 of the 4 channels lane 4*jj + i/4
    // pointed at, for jj = 0..3: four rows of one channel, the A fragment.
    // MFMA j takes channels 32*q + 4*j .. +3 from lane 4*jj + q, so A row m
    // is channel 32*(m/4) + 4*j + m%4 and a lane's results cover 32
    // consecutive channels.
    const int jj = col >> 2;
    const int qq = col & 3;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint2 f1[2], f2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int vr = 16 * h + 4 * blk + jj;
        const int o = vr * 256 + (((4 * qq + j / 2) ^ (vr % 16)) * 16) + (j % 2) * 8;
        f1[h] = lds_read_tr16(&V1t[o]);
        f2[h] = lds_read_tr16(&V2t[o]);
      }
      const V8 a1 = __builtin_bit_cast(V8, make_uint4(f1[0].x, f1[0].y, f1[1].x, f1[1].y));
      const V8 a2 = __builtin_bit_cast(V8, make_uint4(f2[0].x, f2[0].y, f2[1].x, f2[1].y));
      acc1[j] = Op::mma(a1, pb, acc1[j]);
      acc2[j] = Op::mma(a2, pb, acc2[j]);
    }
    const typename Op::S one = Op::from_f32(1.f);
    const V8 ones = {one, one, one, one, one, one, one, one};
    accl = Op::mma(ones, pb, accl);
  }

  // Mask, online softmax and both PV products of a tile with scores sacc.
  __device__ __forceinline__ void update(const floatx4 (&sacc)[2], const uint8_t* V1t,
                                         const uint8_t* V2t, int row0, int r_end, int lim,
                                         float qscale, int col, int blk, bool full) {
    const V8 pb = softmax(sacc, row0, r_end, lim, qscale, blk, full);
    pv(pb, V1t, V2t, col, blk);
  }

  // One tile: scores() then update().
  __device__ __forceinline__ void tile(const uint8_t* Kt, const uint8_t* V1t, const uint8_t* V2t,
                                       const V8 (&qb)[4], int row0, int r_end, int lim,
                                       float qscale, int col, int blk, bool full) {
    floatx4 sacc[2];
    scores(Kt, qb, sacc, col, blk);
    update(sacc, V1t, V2t, row0, r_end, lim, qscale, col, blk, full);
  }

  // Column vrow's result: y (normalised, nsplit == 1) or its split partial.
  __device__ __forceinline__ void store(const SdpaArgs& a, long vrow, int split, int blk) const {
    store_to(a.y, vrow, a.part_o, a.part_ml, vrow, a.nsplit, split, blk, a.part_f16);
  }
  // The same into row yrow of y (nsplit == 1) or partial row prow (fp32 o,
  // or fp16 o / l with f16).
  __device__ __forceinline__ void store_to(void* y, long yrow, float* part_o, float* part_ml,
                                           long prow, int nsplit, int split, int blk,
                                           bool f16) const {
    constexpr int D = 128;
    const float l = accl[0];
    if (nsplit == 1) {
      const float inv = l == 0.f ? 1.f : 1.f / l;  // o stays 0 when no key is visible
      uint16_t* yp = (uint16_t*)y + yrow * 2 * D + 32 * blk;
#pragma unroll
      for (int p = 0; p < 4; ++p) {  // channels 32*blk + 8*p .. +7
        uint32_t w1[4], w2[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int j = 2 * p + t / 2;
          const int r = 2 * (t % 2);
          w1[t] = (uint32_t)Elem<T>::from_f32(acc1[j][r] * inv) |
                  ((uint32_t)Elem<T>::from_f32(acc1[j][r + 1] * inv) << 16);
          w2[t] = (uint32_t)Elem<T>::from_f32(acc2[j][r] * inv) |
                  ((uint32_t)Elem<T>::from_f32(acc2[j][r + 1] * inv) << 16);
        }
        *reinterpret_cast<uint4*>(yp + 8 * p) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        *reinterpret_cast<uint4*>(yp + D + 8 * p) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
      }
    } else if (f16) {
      const int ns = nsplit;
      const float inv = l == 0.f ? 0.f : 1.f / l;
      uint16_t* po = (uint16_t*)part_o + (prow * ns + split) * 2 * D + 32 * blk;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        *reinterpret_cast<uint2*>(po + 4 * j) = half4_bits(
            make_float4(acc1[j][0] * inv, acc1[j][1] * inv, acc1[j][2] * inv, acc1[j][3] * inv));
        *reinterpret_cast<uint2*>(po + D + 4 * j) = half4_bits(
            make_float4(acc2[j][0] * inv, acc2[j][1] * inv, acc2[j][2] * inv, acc2[j][3] * inv));
      }
      if (blk == 0)
        *reinterpret_cast<float2*>(part_ml + (prow * ns + split) * 2) = make_float2(m_run, l);
    } else {
      const int ns = nsplit;
      float* po = part_o + (prow * ns + split) * 2 * D + 32 * blk;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        *reinterpret_cast<float4*>(po + 4 * j) =
            make_float4(acc1[j][0], acc1[j][1], acc1[j][2], acc1[j][3]);
        *reinterpret_cast<float4*>(po + D + 4 * j) =
            make_float4(acc2[j][0], acc2[j][1], acc2[j][2], acc2[j][3]);
      }
      if (blk == 0)
        *reinterpret_cast<float2*>(part_ml + (prow * ns + split) * 2) = make_float2(m_run, l);
    }
  }
};

// Split partials of a wave's 16 columns staged through LDS: lane (col, blk)
// holds channels 32*blk + 4*j .. +3 of its column, so direct stores write
// 16-byte pieces of 16 rows per instruction; staged, each store instruction
// writes two whole 512-byte halves of partial rows (f16: fp16 o / l, two
// 256-byte halves).  lds: this wave's 16 rows of 132 floats (16 bytes of
// padding per row put the 16 columns' writes in distinct bank groups; with
// f16 the padding's first float carries the column's 1 / l).  Column c's
// partial row is prow0 + c, stored for c < ncols.
constexpr int kStageRowFloats = 132;
constexpr int kStageWaveBytes = 16 * kStageRowFloats * 4;
template <typename T>
__device__ __forceinline__ void store_partials_staged(const SwizzledTileAcc<T>& acc, float* lds,
                                                      float* part_o, float* part_ml, long prow0,
                                                      int ncols, int nsplit, int split, int col,
                                                      int blk, bool f16 = false) {
  constexpr int D = 128;
  const int lane = col + 16 * blk;
  if (f16 && blk == 0) {
    const float l = acc.accl[0];
    lds[col * kStageRowFloats + 128] = l == 0.f ? 0.f : 1.f / l;
  }
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const floatx4* src = half ? acc.acc2 : acc.acc1;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<float4*>(lds + col * kStageRowFloats + 32 * blk + 4 * j) =
          make_float4(src[j][0], src[j][1], src[j][2], src[j][3]);
    // (a wave's LDS accesses complete in order: the reads below see these writes)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 2 * i + (lane >> 5);
      const int q = lane & 31;
      const float4 v = *reinterpret_cast<const float4*>(lds + row * kStageRowFloats + 4 * q);
      if (row >= ncols) continue;
      const long e = ((prow0 + row) * nsplit + split) * 2 * D + half * D + 4 * q;
      if (f16) {
        const float inv = lds[row * kStageRowFloats + 128];
        *reinterpret_cast<uint2*>((uint16_t*)part_o + e) =
            half4_bits(make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv));
      } else {
        *reinterpret_cast<float4*>(part_o + e) = v;
      }
    }
  }
  if (blk == 0 && col < ncols)
    *reinterpret_cast<float2*>(part_ml + ((prow0 + col) * nsplit + split) * 2) =
        make_float2(acc.m_run, acc.accl[0]);
}

// S^T = K Q^T of a tile for NCB column blocks (16 columns each) of one
// wave: each K fragment is read from LDS once and used by every block.
template <typename T, int NCB>
__device__ __forceinline__ void tile_scores_n(const uint8_t* Kt,
                                              const typename MfmaOp<T>::V8 (&qb)[NCB][4],
                                              floatx4 (&sacc)[NCB][2], int col, int blk) {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) sacc[cb][h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kr = 16 * h + col;
      const V8 ka = __builtin_bit_cast(
          V8, *reinterpret_cast<const uint4*>(&Kt[kr * 256 + (((4 * s + blk) ^ (kr % 16)) * 16)]));
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) sacc[cb][h] = Op::mma(ka, qb[cb][s], sacc[cb][h]);
    }
  }
}

// Both PV products and l of a tile for NCB column blocks: each V^T fragment
// (SwizzledTileAcc::pv's transposing reads) is read once for every block.
template <typename T, int NCB>
__device__ __forceinline__ void tile_pv_n(SwizzledTileAcc<T> (&acc)[NCB],
                                          const typename MfmaOp<T>::V8 (&pb)[NCB],
                                          const uint8_t* V1t, const uint8_t* V2t, int col,
                                          int blk) {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
  const int jj = col >> 2;
  const int qq = col & 3;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint2 f1[2], f2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int vr = 16 * h + 4 * blk + jj;
      const int o = vr * 256 + (((4 * qq + j / 2) ^ (vr % 16)) * 16) + (j % 2) * 8;
      f1[h] = lds_read_tr16(&V1t[o]);
      f2[h] = lds_read_tr16(&V2t[o]);
    }
    const V8 a1 = __builtin_bit_cast(V8, make_uint4(f1[0].x, f1[0].y, f1[1].x, f1[1].y));
    const V8 a2 = __builtin_bit_cast(V8, make_uint4(f2[0].x, f2[0].y, f2[1].x, f2[1].y));
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      acc[cb].acc1[j] = Op::mma(a1, pb[cb], acc[cb].acc1[j]);
      acc[cb].acc2[j] = Op::mma(a2, pb[cb], acc[cb].acc2[j]);
    }
  }
  const typename Op::S one = Op::from_f32(1.f);
  const V8 ones = {one, one, one, one, one, one, one, one};
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) acc[cb].accl = Op::mma(ones, pb[cb], acc[cb].accl);
}

// The ring's LDS holds one workgroup per CU: two waves per SIMD at 8 waves,
// one at 4.
// T: half_t (fp16 cache) or bf16_t (bf16 cache, bf16 matrix cores).
// NCB: column blocks of 16 virtual heads per wave (2: every K/V fragment
// read from LDS feeds two blocks' MFMAs, half the LDS reads per head).
template <typename T, int NW, int NS = kPrefillStages, int NCB = 1>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 2 : 1)))
sdpa_prefill_kernel(SdpaArgs a) {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
  constexpr int D = 128;
  constexpr int TR = kPrefillTileRows;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int blk = lane >> 4;

  int qblk, unit, split;
  if (!prefill_block_coords(a, blockIdx.x, qblk, unit, split)) return;  // grid padding
  const int b = unit / a.Hkv;
  const int kvh = unit % a.Hkv;
  const int wg_vh0 = qblk * NW * 16 * NCB;
  int vh[NCB], lim[NCB];
  bool col_ok[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    vh[cb] = wg_vh0 + (wave * NCB + cb) * 16 + col;  // this lane's virtual heads (columns)
    col_ok[cb] = vh[cb] < a.GV;
    lim[cb] = col_ok[cb] ? vhead_limit(a, vh[cb]) : 0;
  }
  // Smallest limit over the wave's valid columns of each block: tiles ending
  // at or before it (and before r_end) need no mask.
  int lim_lo[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int v0 = wg_vh0 + (wave * NCB + cb) * 16;
    int hi;
    vhead_limit_range(a, v0, min(16, a.GV - v0), lim_lo[cb], hi);
    lim_lo[cb] = __builtin_amdgcn_readfirstlane(lim_lo[cb]);
  }
  const int max_lim = vhead_limit_max(a, wg_vh0, min(NW * 16 * NCB, a.GV - wg_vh0));
  // The block's visible rows [0, max_lim) in 32-row tiles, dealt to the
  // splits round robin (a.tiles_rr: tile i of split s is tile i * nsplit +
  // s, so every split of a block gets the same tile count, +-1, whatever the
  // causal limit) or in contiguous ranges of rows_per_split rows (tile
  // i of split s is tile s * tps + i).  Rows at or past r_end = max_lim are
  // masked.
  const int ns = a.nsplit;
  const int r_end = max_lim;
  const int tps = a.rows_per_split / TR;  // tiles per contiguous range
  const int tstride = a.tiles_rr ? ns : 1;
  const int tbase = a.tiles_rr ? split : split * tps;
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q;  // row of virtual head 0

  // Q^T, B operand of the 16x16x32 MFMA: lane (col, blk) holds its column's
  // channels 32*s + 8*blk .. +7 for k-step s.
  V8 qb[NCB][4];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const uint16_t* qp =
        (const uint16_t*)a.q + (qrow0 + (col_ok[cb] ? vh[cb] : 0)) * D + 8 * blk;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 w =
          col_ok[cb] ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
      qb[cb][s] = __builtin_bit_cast(V8, w);
    }
    // q is waited for here, before the first tile copies are issued: the
    // compiler's own wait would otherwise sit inside the tile loop and, as
    // vmcnt(0), drain the copies in flight on every iteration.
    asm volatile("" ::"v"(qb[cb][0]), "v"(qb[cb][1]), "v"(qb[cb][2]), "v"(qb[cb][3]));
  }

  // Rows [0, r_end) of this KV head through range-checked resources (byte
  // offsets stay 32-bit: kv_len <= kMfmaMaxRows, checked on the host).
  const long hrow0 = (long)unit * a.kv_cap;
  const unsigned nbytes = (unsigned)(max(r_end, 0) * D * 2);
  const __amdgpu_buffer_rsrc_t rsrc[3] = {
      stream_rsrc((const uint16_t*)a.k + hrow0 * D, nbytes),
      stream_rsrc((const uint16_t*)a.v1 + hrow0 * D, nbytes),
      stream_rsrc((const uint16_t*)a.v2 + hrow0 * D, nbytes)};

  // Ring stage st, tensor t (K, V1, V2): 32 rows x 256 bytes, chunk c of row
  // r at byte r * 256 + (c ^ (r % 16)) * 16.
  __shared__ __attribute__((aligned(16))) uint8_t ring[NS][3][TR * D * 2];
  constexpr int CPW = 3 * TR * D * 2 / 1024 / NW;  // 1 KB copies per wave per tile
  static_assert(3 * TR * D * 2 / 1024 % NW == 0, "whole copies per wave");
  static_assert((NS - 1) * CPW <= 63, "vmcnt counts at most 63");
  // Copy j = wave + c * NW of a tile: tensor j / 8 (= c * NW / 8 for 4 or 8
  // waves), rows 4 g .. 4 g + 3 with g = j % 8; lane L fills row 4 g + L / 16
  // at chunk position L % 16 with chunk (L % 16) ^ row.
  static_assert(NW == 4 || NW == 8, "copies are dealt over 4 or 8 waves");
  auto issue = [&](int st, int tile) {
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int t = c * NW / 8;
      const int g = (wave + c * NW) % 8;
      const int r = 4 * g + lane / 16;
      const int chunk = (lane % 16) ^ (r % 16);
      const unsigned voff = (unsigned)(((tile * tstride + tbase) * TR + r) * D * 2 + chunk * 16);
      lds_copy16_rsrc(rsrc[t], voff, lds_byte_addr(&ring[st][t][g * 1024]));
    }
  };

  SwizzledTileAcc<T> st_acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) st_acc[cb].init();
  const int n_vis = (max(r_end, 0) + TR - 1) / TR;  // the block's tiles
  const int ntiles = a.tiles_rr ? (n_vis > split ? (n_vis - split + ns - 1) / ns : 0)
                                : max(0, min(tps, n_vis - tbase));

  // Every workgroup's tile count is uniform, so every barrier is reached by
  // all of its threads.  Software-pipelined over tiles: the S^T products of
  // tile i + 1 are issued before the softmax and PV products of tile i.
  // Tile i sits in stage i % NS.  Barrier i publishes tile i; at it every
  // wave has finished the PV products of tile i - 2, so stage (i - 2) % NS
  // is refilled with tile i + NS - 2 right after it (barrier 0 fills stage
  // NS - 1, unused until then): NS - 2 tiles in flight ahead of the two
  // being worked on.
  int inflight = 0;
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) {
    if (t < ntiles) {
      issue(t, t);
      ++inflight;
    }
  }
  auto publish = [&](int i) {
    prefill_wait_vm_groups<CPW, NS - 2>(inflight - 1);  // this wave's copies of tile i landed
    asm volatile("s_barrier" ::: "memory");             // every wave's copies landed
    --inflight;
    const int t = i == 0 ? NS - 1 : i + NS - 2;
    if (i != 1 && t < ntiles) {
      issue(t % NS, t);
      ++inflight;
    }
  };
  // A wave whose columns all lie past the last virtual head (a slab's
  // 20 heads in a 4-wave block) only copies its share of the tiles and
  // meets the others at the barriers.
  const bool wave_busy = __builtin_amdgcn_readfirstlane(wg_vh0 + wave * NCB * 16 < a.GV);
  if constexpr (NCB == 1) {
    floatx4 s_cur[2], s_nxt[2];
    if (ntiles > 0) {
      publish(0);
      if (wave_busy) SwizzledTileAcc<T>::scores(ring[0][0], qb[0], s_cur, col, blk);
    }
    for (int i = 0; i < ntiles; ++i) {
      if (i + 1 < ntiles) {
        publish(i + 1);
        if (wave_busy) SwizzledTileAcc<T>::scores(ring[(i + 1) % NS][0], qb[0], s_nxt, col, blk);
      }
      if (wave_busy) {
        const int t0 = (i * tstride + tbase) * TR;
        st_acc[0].update(s_cur, ring[i % NS][1], ring[i % NS][2], t0, r_end, lim[0], a.qscale,
                         col, blk, t0 + TR <= min(r_end, lim_lo[0]));
        s_cur[0] = s_nxt[0];
        s_cur[1] = s_nxt[1];
      }
    }
  } else {
    // One tile per barrier (publish(i) frees the stage of tile i - 2 as above).
    for (int i = 0; i < ntiles; ++i) {
      publish(i);
      floatx4 sacc[NCB][2];
      tile_scores_n<T, NCB>(ring[i % NS][0], qb, sacc, col, blk);
      V8 pb[NCB];
      const int t0 = (i * tstride + tbase) * TR;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
        pb[cb] = st_acc[cb].softmax(sacc[cb], t0, r_end, lim[cb], a.qscale, blk,
                                    t0 + TR <= min(r_end, lim_lo[cb]));
      tile_pv_n<T, NCB>(st_acc, pb, ring[i % NS][1], ring[i % NS][2], col, blk);
    }
  }

  // acc[j][r] of lane (col, blk) is channel 32*blk + 4*j + r of column col.
  if (a.nsplit > 1) {
    // Partials through the ring, once every wave is done with it.
    static_assert(NW * kStageWaveBytes <= (int)sizeof(ring), "staging fits the ring");
    __syncthreads();
    float* lds = reinterpret_cast<float*>(&ring[0][0][0]) + wave * (kStageWaveBytes / 4);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int c0 = vh[cb] - col;  // the block's first virtual head
      store_partials_staged<T>(st_acc[cb], lds, a.part_o, a.part_ml, qrow0 + c0,
                               min(16, a.GV - c0), a.nsplit, split, col, blk, a.part_f16);
    }
    return;
  }
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
    if (col_ok[cb]) st_acc[cb].store(a, qrow0 + vh[cb], split, blk);
}

template <typename T>
inline int launch_prefill_kernel_16(const SdpaArgs& a, int waves, int ncb, int nblocks,
                                   hipStream_t st) {
  if (waves == 8 && ncb == 2) {
    hipLaunchKernelGGL((sdpa_prefill_kernel<T, 8, kPrefillStages, 2>), dim3(nblocks), dim3(512),
                       0, st, a);
  } else if (waves == 8) {
    hipLaunchKernelGGL((sdpa_prefill_kernel<T, 8>), dim3(nblocks), dim3(512), 0, st, a);
  } else {
    hipLaunchKernelGGL((sdpa_prefill_kernel<T, 4>), dim3(nblocks), dim3(256), 0, st, a);
  }
  return check_launch("sdpa_dual_v_rows (prefill)");
}


// ------------------------------------------------- prefill chunk from the projections ---
// One launch for a GDA layer's prefill chunk (src/mlx_motif/model.py:590-594
// rope on q and k, :620-629 the 4-slot split and cache write, :769-807 the
// two dual-V passes with the bottom-right causal mask): query blocks of the
// origin pass (q1 x k1) and of the noise pass (q2 x k2) share the grid, each
// over V1/V2.  What differs from sdpa_prefill_kernel:
//   - q is read from q_proj and roped in registers: channel c of k-step s
//     (s < 2) pairs with channel c + 64 of k-step s + 2 in the same lane;
//   - the rows before the chunk (kv_len - S_q) come from the cache in
//     32-row tiles, the chunk's rows from k_proj / v_proj in 32-row tiles
//     from its first row; the tiles are dealt to the row splits round robin;
//     each wave ropes in place the K rows of a chunk tile it copied, once
//     its own copies have landed and before the tile's barrier;
//   - before its tile loop each block writes its share of its split's chunk
//     rows into the cache (roped k1 / k2, v1, v2): the origin blocks of a
//     (b, KV head, split) share the split's k1, v1 and v2 rows, the noise
//     blocks its k2 rows.  No block reads those cache rows (every block
//     takes the chunk from the projections), so no block waits for another.
// RoPE is rope_impl.hpp's, rounded once to T, so q, the cache rows and the
// K tiles carry the values motif_rope_split4 produces.

// stream_rsrc from a wave-uniform base and size, made explicitly scalar
// (readfirstlane) so that the resource always lands in SGPRs, as the
// LDS-direct copies' inline asm requires.
__device__ inline __amdgpu_buffer_rsrc_t uniform_stream_rsrc(const void* base, unsigned bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return stream_rsrc((const void*)(uintptr_t)(((uint64_t)hi << 32) | lo),
                     __builtin_amdgcn_readfirstlane(bytes));
}

// Roped or copied pairs (c, c + 64) of 16-bit channels: 4 values from each
// half as 8-byte words.
// (inv: the pairs' inverse frequencies, rope_inv_freq.)
template <typename T>
__device__ inline void rope_words_inv(uint2& lo, uint2& hi, const float (&inv)[4], int pos,
                                      float pos_scale) {
  uint32_t a[2] = {lo.x, lo.y}, b[2] = {hi.x, hi.y};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float y1[2], y2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float x1 = Elem<T>::to_f32((uint16_t)(e ? a[h] >> 16 : a[h] & 0xFFFFu));
      const float x2 = Elem<T>::to_f32((uint16_t)(e ? b[h] >> 16 : b[h] & 0xFFFFu));
      float cs, sn;
      rope_angle_inv(inv[2 * h + e], pos, pos_scale, cs, sn);
      rope_rotate(x1, x2, cs, sn, y1[e], y2[e]);
    }
    a[h] = (uint32_t)Elem<T>::from_f32(y1[0]) | ((uint32_t)Elem<T>::from_f32(y1[1]) << 16);
    b[h] = (uint32_t)Elem<T>::from_f32(y2[0]) | ((uint32_t)Elem<T>::from_f32(y2[1]) << 16);
  }
  lo = make_uint2(a[0], a[1]);
  hi = make_uint2(b[0], b[1]);
}
template <typename T>
__device__ inline void rope_words(uint2& lo, uint2& hi, int p0, int pos, float log2_theta,
                                  float pos_scale) {
  const float inv[4] = {rope_inv_freq(p0, 128, log2_theta), rope_inv_freq(p0 + 1, 128, log2_theta),
                        rope_inv_freq(p0 + 2, 128, log2_theta),
                        rope_inv_freq(p0 + 3, 128, log2_theta)};
  rope_words_inv<T>(lo, hi, inv, pos, pos_scale);
}

// NCB: column blocks of 16 virtual heads per wave, as in sdpa_prefill_kernel.
template <typename T, int NW, int NS = kPrefillStages, int NCB = 1>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 2 : 1)))
gda_prefill_proj_kernel(SdpaArgs a) {
  using Op = MfmaOp<T>;
  using V8 = typename Op::V8;
  constexpr int D = 128;
  constexpr int TR = kPrefillTileRows;
  constexpr int NT = NW * 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int blk = lane >> 4;

  int qblk, unit, split;
  if (!prefill_block_coords(a, blockIdx.x, qblk, unit, split)) return;  // grid padding
  const bool noise = qblk >= a.nqb_origin;
  const int qb = noise ? qblk - a.nqb_origin : qblk;
  const int nqb = noise ? a.nchunk - a.nqb_origin : a.nqb_origin;
  const int G = noise ? a.G2 : a.G;  // heads of this pass per KV head
  const int S = a.S_q;
  const int GV = G * S;
  const int b = unit / a.Hkv;
  const int kvh = unit % a.Hkv;
  const int wg_vh0 = qb * NW * 16 * NCB;
  int vh[NCB], lim[NCB];  // virtual heads (pass head vh / S, query row vh % S)
  bool col_ok[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    vh[cb] = wg_vh0 + (wave * NCB + cb) * 16 + col;
    col_ok[cb] = vh[cb] < GV;
    lim[cb] = col_ok[cb] ? vhead_limit(a, vh[cb]) : 0;
  }
  int lim_lo[NCB];  // as in sdpa_prefill_kernel
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int v0 = wg_vh0 + (wave * NCB + cb) * 16;
    int hi;
    vhead_limit_range(a, v0, min(16, GV - v0), lim_lo[cb], hi);
    lim_lo[cb] = __builtin_amdgcn_readfirstlane(lim_lo[cb]);
  }
  const int max_lim = vhead_limit_max(a, wg_vh0, min(NW * 16 * NCB, GV - wg_vh0));

  // The KV head's tiles: T_OLD over cache rows [0, row0) (the last one may
  // stop short of 32 rows), then T_NEW over the chunk's rows [row0, kv_len)
  // from the projections, tile n at row0 + 32 n.  They are dealt to the
  // splits round robin (global tile g to split g % nsplit), so every split
  // gets its share of the old rows, of the chunk tiles to rope and of the
  // rows the causal limit cuts off.  Tiles starting at or past max_lim are
  // not visited.
  const int row0 = a.kv_len - S;  // the chunk's first cache row
  const int ns = a.nsplit;
  const int T_OLD = (row0 + TR - 1) / TR;
  const int T_NEW = (S + TR - 1) / TR;
  const int n_vis = max_lim <= row0 ? (max_lim + TR - 1) / TR
                                    : T_OLD + (max_lim - row0 + TR - 1) / TR;
  const int ntiles = n_vis > split ? (n_vis - split + ns - 1) / ns : 0;
  auto gtile = [&](int i) { return split + i * ns; };
  auto is_new_tile = [&](int i) { return gtile(i) >= T_OLD; };
  auto first_row = [&](int i) {
    const int g = gtile(i);
    return g >= T_OLD ? row0 + (g - T_OLD) * TR : g * TR;
  };

  const int HK = 2 * a.Hkv;  // heads of k_proj and of v_proj
  const long pstride = (long)HK * D;
  const uint16_t* kproj = (const uint16_t*)a.new_k1;
  const uint16_t* vproj = (const uint16_t*)a.new_v1;
  uint16_t* kc = (uint16_t*)(noise ? a.k2 : a.k);  // this pass's K slot
  const long crow0 = (long)unit * a.kv_cap;       // cache row 0 of this KV head

  // ---- this block's share of the chunk's cache rows (written, not read) ----
  // The split's chunk tiles n = n_first, n_first + ns, ..; local row lr of
  // them is chunk row 32 (n_first + (lr / 32) ns) + lr % 32.  The split's
  // origin blocks share k1, v1, v2 of those rows, its noise blocks k2.
  {
    const int n_first = ((split - T_OLD) % ns + ns) % ns;
    const int nnew = T_NEW > n_first ? (T_NEW - n_first + ns - 1) / ns : 0;
    const int nrows = nnew * TR;
    const int per = (nrows + nqb - 1) / nqb;
    const int r_lo = qb * per;
    const int r_hi = min(r_lo + per, nrows);
    auto chunk_row = [&](int lr) { return row0 + (n_first + (lr / TR) * ns) * TR + lr % TR; };
    const int hk = 2 * kvh + (noise ? 1 : 0);
    // K: one (row, chunk pair, half) item per thread: 4 pairs (c, c + 64).
    for (int it = threadIdx.x; it < max(r_hi - r_lo, 0) * 16; it += NT) {
      const int r = chunk_row(r_lo + (it >> 4));
      if (r >= a.kv_len) continue;
      const int cp = (it >> 1) & 7;
      const int p0 = 8 * cp + 4 * (it & 1);
      const long src = ((long)b * S + (r - row0)) * pstride + (long)hk * D;
      uint2 lo = *reinterpret_cast<const uint2*>(kproj + src + p0);
      uint2 hi = *reinterpret_cast<const uint2*>(kproj + src + 64 + p0);
      rope_words<T>(lo, hi, p0, a.rope_pos0 + (r - row0), a.rope_log2_theta, a.rope_pos_scale);
      *reinterpret_cast<uint2*>(kc + (crow0 + r) * D + p0) = lo;
      *reinterpret_cast<uint2*>(kc + (crow0 + r) * D + 64 + p0) = hi;
    }
    if (!noise) {  // V1 and V2: 16-byte copies
      for (int it = threadIdx.x; it < max(r_hi - r_lo, 0) * 32; it += NT) {
        const int r = chunk_row(r_lo + (it >> 5));
        if (r >= a.kv_len) continue;
        const int t = (it >> 4) & 1;
        const int c = it & 15;
        const long src = ((long)b * S + (r - row0)) * pstride + (long)(2 * kvh + t) * D + 8 * c;
        const uint4 w = *reinterpret_cast<const uint4*>(vproj + src);
        *reinterpret_cast<uint4*>((uint16_t*)(t ? a.v2 : a.v1) + (crow0 + r) * D + 8 * c) = w;
      }
    }
  }

  // ---- Q^T from q_proj, roped: lane (col, blk) holds channels 32*s + 8*blk .. +7 ----
  V8 qbv[NCB][4];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int hp = kvh * G + (col_ok[cb] ? vh[cb] / S : 0);  // head within the pass
    const int srow = col_ok[cb] ? vh[cb] % S : 0;
    const int HQ = a.q_groups * (a.q_gr + 1);
    int qh;
    if (!noise)
      qh = a.q_origin_first ? hp : (hp / a.q_gr) * (a.q_gr + 1) + hp % a.q_gr;
    else
      qh = a.q_origin_first ? a.q_groups * a.q_gr + hp : hp * (a.q_gr + 1) + a.q_gr;
    const uint16_t* qp = (const uint16_t*)a.q + (((long)b * S + srow) * HQ + qh) * D + 8 * blk;
    uint4 w[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      w[s] = col_ok[cb] ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
    const int pos = a.rope_pos0 + srow;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint2 l0 = make_uint2(w[s].x, w[s].y), h0 = make_uint2(w[s + 2].x, w[s + 2].y);
      uint2 l1 = make_uint2(w[s].z, w[s].w), h1 = make_uint2(w[s + 2].z, w[s + 2].w);
      rope_words<T>(l0, h0, 32 * s + 8 * blk, pos, a.rope_log2_theta, a.rope_pos_scale);
      rope_words<T>(l1, h1, 32 * s + 8 * blk + 4, pos, a.rope_log2_theta, a.rope_pos_scale);
      w[s] = make_uint4(l0.x, l0.y, l1.x, l1.y);
      w[s + 2] = make_uint4(h0.x, h0.y, h1.x, h1.y);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) qbv[cb][s] = __builtin_bit_cast(V8, w[s]);
  }
  // q and this block's cache stores are waited for here, before the first
  // tile copies are issued (vmcnt also counts stores; the tile waits below
  // count only the copies).
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
    asm volatile("s_waitcnt vmcnt(0)" ::"v"(qbv[cb][0]), "v"(qbv[cb][1]), "v"(qbv[cb][2]),
                 "v"(qbv[cb][3])
                 : "memory");

  // Rows [0, row0) from the cache, the chunk's rows from the projections,
  // through range-checked resources (past the range: zeros).
  const unsigned obytes = (unsigned)(row0 * D * 2);
  const __amdgpu_buffer_rsrc_t r_old[3] = {
      uniform_stream_rsrc(kc + crow0 * D, obytes),
      uniform_stream_rsrc((const uint16_t*)a.v1 + crow0 * D, obytes),
      uniform_stream_rsrc((const uint16_t*)a.v2 + crow0 * D, obytes)};
  const long prow0 = (long)b * S * pstride;
  const unsigned nbytes = S > 0 ? (unsigned)(((long)(S - 1) * pstride + D) * 2) : 0u;
  const __amdgpu_buffer_rsrc_t r_new[3] = {
      uniform_stream_rsrc(kproj + prow0 + (long)(2 * kvh + (noise ? 1 : 0)) * D, nbytes),
      uniform_stream_rsrc(vproj + prow0 + (long)(2 * kvh) * D, nbytes),
      uniform_stream_rsrc(vproj + prow0 + (long)(2 * kvh + 1) * D, nbytes)};
  const unsigned pstride_b = (unsigned)(pstride * 2);

  __shared__ __attribute__((aligned(16))) uint8_t ring[NS][3][TR * D * 2];
  constexpr int CPW = 3 * TR * D * 2 / 1024 / NW;
  static_assert(3 * TR * D * 2 / 1024 % NW == 0, "whole copies per wave");
  static_assert((NS - 1) * CPW <= 63, "vmcnt counts at most 63");
  static_assert(NW == 4 || NW == 8, "copies are dealt over 4 or 8 waves");
  auto issue = [&](int st, int tile) {
    const bool is_new = is_new_tile(tile);  // wave-uniform
    const int tr = is_new ? gtile(tile) - T_OLD : gtile(tile);
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int t = c * NW / 8;
      const int g = (wave + c * NW) % 8;
      const int r = 4 * g + lane / 16;
      const int chunk = (lane % 16) ^ (r % 16);
      const unsigned lds = lds_byte_addr(&ring[st][t][g * 1024]);
      if (is_new)
        lds_copy16_rsrc(r_new[t], (unsigned)(tr * TR + r) * pstride_b + chunk * 16, lds);
      else
        lds_copy16_rsrc(r_old[t], (unsigned)((tr * TR + r) * D * 2 + chunk * 16), lds);
    }
  };

  // K rows of a chunk tile, roped in place by the wave that copied them
  // (copy `wave` of a tile holds K rows 4*wave .. 4*wave + 3, and with 4
  // waves copy `wave + 4` rows 4*wave + 16 .. + 19): lane (row rr = lane/16
  // of those four, channel pair block cp = lane/2 % 8, half h = lane % 2)
  // ropes channels 8*cp + 4*h .. +3 with their partners 64 on.
  const int rr = lane >> 4;
  const int rcp = (lane >> 1) & 7;
  const int rh = lane & 1;
  float rinv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) rinv[e] = rope_inv_freq(8 * rcp + 4 * rh + e, D, a.rope_log2_theta);
  auto rope_own_rows = [&](int st, int first_row, int nrows) {
    uint8_t* Kt = ring[st][0];
#pragma unroll
    for (int c = 0; c < 8 / NW; ++c) {
      const int r = 4 * (wave + c * NW) + rr;
      if (r < nrows) {
        uint2* plo = reinterpret_cast<uint2*>(&Kt[r * 256 + ((rcp ^ (r % 16)) * 16) + 8 * rh]);
        uint2* phi =
            reinterpret_cast<uint2*>(&Kt[r * 256 + (((rcp + 8) ^ (r % 16)) * 16) + 8 * rh]);
        uint2 lo = *plo, hi = *phi;
        rope_words_inv<T>(lo, hi, rinv, a.rope_pos0 + (first_row + r - row0), a.rope_pos_scale);
        *plo = lo;
        *phi = hi;
      }
    }
  };

  SwizzledTileAcc<T> st_acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) st_acc[cb].init();
  // Pipelined as sdpa_prefill_kernel: barrier i publishes tile i (a chunk
  // tile's K rows roped first by the waves that copied them); the scores of
  // tile i + 1 are issued before the softmax and PV products of tile i.
  int inflight = 0;
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) {
    if (t < ntiles) {
      issue(t, t);
      ++inflight;
    }
  }
  auto publish = [&](int i) {
    prefill_wait_vm_groups<CPW, NS - 2>(inflight - 1);  // this wave's copies of tile i landed
    if (is_new_tile(i)) {  // rope the K rows this wave copied, before the waves meet
      const int first = first_row(i);
      rope_own_rows(i % NS, first, min(TR, max_lim - first));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    asm volatile("s_barrier" ::: "memory");  // every wave's copies (and ropes) landed
    --inflight;
    const int t = i == 0 ? NS - 1 : i + NS - 2;
    if (i != 1 && t < ntiles) {
      issue(t % NS, t);
      ++inflight;
    }
  };
  if constexpr (NCB == 1) {
    floatx4 s_cur[2], s_nxt[2];
    if (ntiles > 0) {
      publish(0);
      SwizzledTileAcc<T>::scores(ring[0][0], qbv[0], s_cur, col, blk);
    }
    for (int i = 0; i < ntiles; ++i) {
      if (i + 1 < ntiles) {
        publish(i + 1);
        SwizzledTileAcc<T>::scores(ring[(i + 1) % NS][0], qbv[0], s_nxt, col, blk);
      }
      const int t0 = first_row(i);
      const int rl = is_new_tile(i) ? max_lim : min(row0, max_lim);
      st_acc[0].update(s_cur, ring[i % NS][1], ring[i % NS][2], t0, rl, lim[0], a.qscale, col,
                       blk, t0 + TR <= min(rl, lim_lo[0]));
      s_cur[0] = s_nxt[0];
      s_cur[1] = s_nxt[1];
    }
  } else {
    for (int i = 0; i < ntiles; ++i) {  // one tile per barrier
      publish(i);
      floatx4 sacc[NCB][2];
      tile_scores_n<T, NCB>(ring[i % NS][0], qbv, sacc, col, blk);
      V8 pb[NCB];
      const int rl = is_new_tile(i) ? max_lim : min(row0, max_lim);
      const int t0 = first_row(i);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
        pb[cb] = st_acc[cb].softmax(sacc[cb], t0, rl, lim[cb], a.qscale, blk,
                                    t0 + TR <= min(rl, lim_lo[cb]));
      tile_pv_n<T, NCB>(st_acc, pb, ring[i % NS][1], ring[i % NS][2], col, blk);
    }
  }

  // Output rows: origin (b, head, s) of y, noise (b, head, s) of y2; split
  // partials in one row space, the noise rows after y2_row0.
  const int Hp = a.Hkv * G;
  const long yrow0 = ((long)b * Hp + (long)kvh * G) * S;
  if (a.nsplit > 1) {
    // Partials through the ring, once every wave is done with it.
    static_assert(NW * kStageWaveBytes <= (int)sizeof(ring), "staging fits the ring");
    __syncthreads();
    float* lds = reinterpret_cast<float*>(&ring[0][0][0]) + wave * (kStageWaveBytes / 4);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int c0 = vh[cb] - col;
      store_partials_staged<T>(st_acc[cb], lds, a.part_o, a.part_ml,
                               (noise ? a.y2_row0 : 0) + yrow0 + c0, min(16, GV - c0), a.nsplit,
                               split, col, blk, a.part_f16);
    }
    return;
  }
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    if (!col_ok[cb]) continue;
    const long yrow = yrow0 + vh[cb];
    st_acc[cb].store_to(noise ? a.y2 : a.y, yrow, a.part_o, a.part_ml,
                        (noise ? a.y2_row0 : 0) + yrow, a.nsplit, split, blk, a.part_f16);
  }
}

template <typename T>
inline int launch_gda_prefill_proj_16(const SdpaArgs& a, int waves, int ncb, int nblocks,
                                      hipStream_t st) {
  if (waves == 8 && ncb == 2) {
    hipLaunchKernelGGL((gda_prefill_proj_kernel<T, 8, kPrefillStages, 2>), dim3(nblocks),
                       dim3(512), 0, st, a);
  } else if (waves == 8) {
    hipLaunchKernelGGL((gda_prefill_proj_kernel<T, 8>), dim3(nblocks), dim3(512), 0, st, a);
  } else {
    hipLaunchKernelGGL((gda_prefill_proj_kernel<T, 4>), dim3(nblocks), dim3(256), 0, st, a);
  }
  return check_launch("gda_prefill_proj");
}

}  // namespace motif
