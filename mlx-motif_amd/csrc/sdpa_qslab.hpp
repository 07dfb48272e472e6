// Multi-row (speculative-verify slab) dual-V attention over the packed q4/q8
// cache at head_dim 128: each packed K/V tile is read from HBM once per
// workgroup, dequantised once into an fp16 LDS ring, and read there by every
// wave of the workgroup.
//
// The decode kernels carry (virtual head x scale group) on the 16 MFMA
// columns, so a slab of 5 query rows x GQA 4 = 20 virtual heads at group size
// 64 needs three column blocks, and running them as three head chunks reads
// every packed row three times and unpacks it three times.  Here:
//   - the workgroup's threads load a step of NP 32-row tiles of K, V1 and
//     V2 (16 codes per thread and chunk, with the chunk's scale and bias) into
//     registers two steps ahead, and dequantise them to fp16 (the rounding
//     point of the reference path, whose mx.dequantize output feeds the
//     attention: src/mlx_motif/kernels/attention.py:497-499) into an LDS
//     ring in the fp16 prefill kernel's swizzled tile layout;
//   - wave w owns column block w % NCB (16 virtual heads, one column each: no
//     scale-group columns, the values are already dequantised) and tile w /
//     NCB of each step, and runs SwizzledTileAcc on it: S^T = K Q^T, online
//     softmax, O^T = V^T P^T on 16x16x32 fp16 MFMAs with fp32 accumulation;
//   - the NP waves of a column block merge their (m, l, o) through LDS at the
//     end; the workgroup's rows are one split, published as partials to the
//     merge launch when there are several.
// The causal limit is per column (bottom-right alignment, as the decode
// kernels), and a workgroup streams only the rows its columns can see.
#pragma once

#include "sdpa_prefill.hpp"

namespace motif {

// Floats per lane of the consumer waves' merge records in LDS: 64 of o,
// then m and l, padded to a multiple of four so that every lane's float4
// accesses are 16-byte aligned (68 dwords per lane also put the 16 lanes of
// one access phase in distinct bank groups).
constexpr int kQslabMergeFloats = 68;

// Workgroup barrier after this wave's LDS writes completed, without the
// vector-memory wait of __syncthreads' fence (the packed loads in flight
// stay in flight; the compiler waits for them where they are used).
// Smallest row limit over the valid columns of the 16-column block at
// virtual head v0 (wave-uniform): tiles ending at or before it need no mask.
__device__ inline int qslab_block_limit_lo(const SdpaArgs& a, int v0) {
  int lo, hi;
  vhead_limit_range(a, v0, min(16, a.GV - v0), lo, hi);
  return __builtin_amdgcn_readfirstlane(lo);
}

__device__ inline void qslab_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NCB column blocks of 16 virtual heads, NW waves (4: one per SIMD, two
// LDS stages; 8: two per SIMD, one stage); NP = NW / NCB tiles per step.
template <int BITS, int GS, int NCB, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
sdpa_qslab_kernel(SdpaArgs a) {
  using Acc = SwizzledTileAcc<half_t>;
  using V8 = Acc::V8;
  constexpr int D = 128;
  constexpr int TR = kPrefillTileRows;  // 32
  constexpr int NP = NW / NCB;
  constexpr int NS = NW == 4 ? 2 : 1;  // LDS stages of dequantised steps
  constexpr int NG = D / GS;
  constexpr int RB = D * BITS / 8;   // packed bytes per row
  constexpr int CB = 16 * BITS / 8;  // packed bytes per 16-code chunk
  constexpr int CPT = 12 * NP / NW;  // chunks per thread per step (768 per tile)
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(NW % NCB == 0, "whole tiles per step");
  static_assert(GS % 16 == 0, "a chunk sits in one scale group");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int blk = lane >> 4;
  const int cb = wave % NCB;  // column block
  const int tp = wave / NCB;  // tile of the step

  int qblk, unit, split;
  if (!prefill_block_coords(a, blockIdx.x, qblk, unit, split)) return;  // grid padding
  const int b = unit / a.Hkv;
  const int kvh = unit % a.Hkv;
  const int wg_vh0 = qblk * NCB * 16;
  const int vh = wg_vh0 + cb * 16 + col;  // this lane's virtual head (column)
  const bool col_ok = vh < a.GV;
  const int lim = col_ok ? vhead_limit(a, vh) : 0;
  const int lim_lo = qslab_block_limit_lo(a, wg_vh0 + cb * 16);
  const int max_lim = vhead_limit_max(a, wg_vh0, min(NCB * 16, a.GV - wg_vh0));
  const int r_begin = split * a.rows_per_split;
  const int r_end = min(r_begin + a.rows_per_split, max_lim);
  const int nrows = max(r_end - r_begin, 0);
  const int nsteps = (nrows + NP * TR - 1) / (NP * TR);
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q;  // row of virtual head 0

  // Q^T, B operand: lane (col, blk) holds its column's channels 32*s + 8*blk
  // .. +7 for k-step s.
  V8 qb[4];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (col_ok ? vh : 0)) * D + 8 * blk;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 w = col_ok ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
      qb[s] = __builtin_bit_cast(V8, w);
    }
    // q is waited for here, before the tiles' loads are issued: the
    // compiler's own wait for it would otherwise sit inside the step loop as
    // vmcnt(0) and drain the loads in flight on every step.
    asm volatile("" ::"v"(qb[0]), "v"(qb[1]), "v"(qb[2]), "v"(qb[3]));
  }

  // Rows [r_begin, r_end) of this KV head through range-checked resources
  // (past the end: zeros).
  const long hrow0 = (long)unit * a.kv_cap + r_begin;
  const unsigned dbytes = (unsigned)(nrows * RB);
  const unsigned sbytes = (unsigned)(nrows * NG * 2);
  const __amdgpu_buffer_rsrc_t rd[3] = {
      stream_rsrc((const uint8_t*)a.kd + hrow0 * RB, dbytes),
      stream_rsrc((const uint8_t*)a.v1d + hrow0 * RB, dbytes),
      stream_rsrc((const uint8_t*)a.v2d + hrow0 * RB, dbytes)};
  const __amdgpu_buffer_rsrc_t rsc[3] = {
      stream_rsrc((const uint16_t*)a.ks + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2s + hrow0 * NG, sbytes)};
  const __amdgpu_buffer_rsrc_t rbi[3] = {
      stream_rsrc((const uint16_t*)a.kb + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1b + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2b + hrow0 * NG, sbytes)};

  // Chunk k of a step (k < CPT) is chunk u = tid + 64 * NW * k of the step's
  // NP x 3 (tile, tensor) blocks of 256: block u / 256 (tile / 3, tensor % 3),
  // row (u % 256) / 8, codes 16 * (u % 8) .. +15 of that row.  Eight lanes
  // cover a row, so one load instruction reads a tensor's 32 rows
  // contiguously; the block index is wave-uniform.
  const int crow = (tid & 255) >> 3;
  const int cchunk = tid & 7;
  auto cblock = [&](int k) { return (tid >> 8) + (NW / 4) * k; };
  const int cgroup = 16 * cchunk / GS;
  // Packed step data as loaded (no arithmetic on it before its use, so the
  // compiler's waits for it sit at the dequantisation).
  struct Packed {
    uint32_t w[CPT][CB / 4];
    uint32_t s[CPT], b[CPT];  // scale and bias bits (low 16)
  };
  auto load = [&](Packed& P, int step) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int t = cblock(k) % 3;
      const unsigned row = (unsigned)((step * NP + cblock(k) / 3) * TR + crow);
      const unsigned off = row * RB + (unsigned)(cchunk * CB);
      if constexpr (CB == 16) {
        const uint4 x = bload4(rd[t], off);
        P.w[k][0] = x.x; P.w[k][1] = x.y; P.w[k][2] = x.z; P.w[k][3] = x.w;
      } else {
        const uint2 x = bload2(rd[t], off);
        P.w[k][0] = x.x; P.w[k][1] = x.y;
      }
      const unsigned soff = (row * NG + (unsigned)cgroup) * 2u;
      P.s[k] = __builtin_amdgcn_raw_buffer_load_b16(rsc[t], soff, 0, kCachePolicyStream);
      P.b[k] = __builtin_amdgcn_raw_buffer_load_b16(rbi[t], soff, 0, kCachePolicyStream);
    }
  };

  // Ring stage st, tile p, tensor t: 32 rows x 256 bytes of fp16, 16-byte
  // chunk c of row r at byte r * 256 + (c ^ (r % 16)) * 16.
  // The same LDS holds the merge of the column blocks' waves at the end; a
  // spare stage is added where the merge needs it.
  constexpr int STAGE_BYTES = NP * 3 * TR * D * 2;
  constexpr int MERGE_BYTES = NCB * (NP / 2) * 64 * kQslabMergeFloats * 4;
  constexpr int NSA = NS * STAGE_BYTES >= MERGE_BYTES ? NS : NS + 1;
  static_assert(NSA * STAGE_BYTES >= MERGE_BYTES, "merge fits the stages");
  __shared__ __attribute__((aligned(16))) uint8_t ring[NSA][NP][3][TR * D * 2];
  // Code i of a chunk (its bits within the chunk's words), dequantised; two
  // fp16 values per dword, written as two 16-byte chunks of the row.
  auto dequant_store = [&](const Packed& P, int st) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)P.s[k]);
      const float bi = (float)__builtin_bit_cast(_Float16, (uint16_t)P.b[k]);
      const uint32_t* cw = P.w[k];
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        uint32_t u0, u1;
        if constexpr (BITS == 8) {
          u0 = (cw[i / 4] >> (8 * (i % 4))) & 0xFFu;
          u1 = (cw[(i + 1) / 4] >> (8 * ((i + 1) % 4))) & 0xFFu;
        } else {
          u0 = (cw[i / 8] >> (4 * (i % 8))) & 0xFu;
          u1 = (cw[(i + 1) / 8] >> (4 * ((i + 1) % 8))) & 0xFu;
        }
        // One rounding, to fp16, of the exact scale * code + bias (one
        // v_fma_mixlo_f16); the oracle's fp32 multiply-then-add differs from
        // it by at most one fp16 ulp, in rare values.
        const _Float16 v0 = (_Float16)__builtin_fmaf(s, (float)u0, bi);
        const _Float16 v1 = (_Float16)__builtin_fmaf(s, (float)u1, bi);
        h[i / 2] = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
      }
      uint8_t* base = ring[st][cblock(k) / 3][cblock(k) % 3] + crow * 256;
      const int c0 = (2 * cchunk) ^ (crow % 16);
      const int c1 = (2 * cchunk + 1) ^ (crow % 16);
      *reinterpret_cast<uint4*>(base + c0 * 16) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(base + c1 * 16) = make_uint4(h[4], h[5], h[6], h[7]);
    }
  };

  Acc acc;
  acc.init();

  // NW = 4: two register sets and two stages.  Step j's packed data is
  // loaded two steps ahead into set j % 2; step j computes stage j % 2
  // (written in the step before), dequantises step j + 1 (its loads were
  // issued before step j + 2's) into the other stage (freed by the barrier
  // ending the step before) and ends with a barrier.  NW = 8 (two waves per
  // SIMD, whose interleaving hides the waits): one set and one stage;
  // compute, barrier, dequantise step j + 1, load step j + 2, barrier.
  // Loads and dequantisation are unconditional (steps past the last read
  // past the resources' ends: zeros, no memory access), so the loop body is
  // straight-line code for the compiler's waits; the step count is uniform
  // over the workgroup, so every barrier is reached by all of its threads.
  if constexpr (NW == 4) {
    Packed P0, P1;
    load(P0, 0);
    load(P1, 1);
    dequant_store(P0, 0);
    qslab_barrier();
    auto step = [&](int j, Packed& ld, Packed& nx) {
      load(ld, j + 2);  // ld held step j, dequantised in the step before
      const int t0 = r_begin + (j * NP + tp) * TR;
      acc.tile(ring[j & 1][tp][0], ring[j & 1][tp][1], ring[j & 1][tp][2], qb, t0, r_end, lim,
               a.qscale, col, blk, t0 + TR <= min(r_end, lim_lo));
      dequant_store(nx, (j + 1) & 1);
      qslab_barrier();
    };
    for (int j = 0; j < nsteps; j += 2) {
      step(j, P0, P1);
      if (j + 1 >= nsteps) break;
      step(j + 1, P1, P0);
    }
  } else {
    Packed P;
    load(P, 0);
    dequant_store(P, 0);
    load(P, 1);
    qslab_barrier();
    for (int j = 0; j < nsteps; ++j) {
      const int t0 = r_begin + (j * NP + tp) * TR;
      acc.tile(ring[0][tp][0], ring[0][tp][1], ring[0][tp][2], qb, t0, r_end, lim, a.qscale, col,
               blk, t0 + TR <= min(r_end, lim_lo));
      qslab_barrier();
      dequant_store(P, 0);  // step j + 1
      load(P, j + 2);
      qslab_barrier();
    }
  }

  // The NP waves of a column block merge their (m, l, o) through LDS (the
  // ring is free after the last barrier), halving the count each round: the
  // upper half of the waves writes, the lower half adds.
  if constexpr (NP > 1) {
    float* xo = reinterpret_cast<float*>(&ring[0][0][0][0]);  // [NCB][NP / 2][64 lanes][kQslabMergeFloats]
#pragma unroll
    for (int half = NP / 2; half >= 1; half /= 2) {
      if (tp >= half && tp < 2 * half) {
        float* p = xo + ((cb * (NP / 2) + tp - half) * 64 + lane) * kQslabMergeFloats;
#pragma unroll
        for (int jx = 0; jx < 8; ++jx) {
          *reinterpret_cast<float4*>(p + 4 * jx) =
              make_float4(acc.acc1[jx][0], acc.acc1[jx][1], acc.acc1[jx][2], acc.acc1[jx][3]);
          *reinterpret_cast<float4*>(p + 32 + 4 * jx) =
              make_float4(acc.acc2[jx][0], acc.acc2[jx][1], acc.acc2[jx][2], acc.acc2[jx][3]);
        }
        p[64] = acc.m_run;
        p[65] = acc.accl[0];
      }
      __syncthreads();
      if (tp < half) {
        const float* p = xo + ((cb * (NP / 2) + tp) * 64 + lane) * kQslabMergeFloats;
        const float m2 = p[64];
        const float m = fmaxf(acc.m_run, m2);
        const float f1 = fast_exp2(acc.m_run - m);
        const float f2 = fast_exp2(m2 - m);
#pragma unroll
        for (int jx = 0; jx < 8; ++jx) {
          const float4 o1 = *reinterpret_cast<const float4*>(p + 4 * jx);
          const float4 o2 = *reinterpret_cast<const float4*>(p + 32 + 4 * jx);
          acc.acc1[jx][0] = fmaf(acc.acc1[jx][0], f1, o1.x * f2);
          acc.acc1[jx][1] = fmaf(acc.acc1[jx][1], f1, o1.y * f2);
          acc.acc1[jx][2] = fmaf(acc.acc1[jx][2], f1, o1.z * f2);
          acc.acc1[jx][3] = fmaf(acc.acc1[jx][3], f1, o1.w * f2);
          acc.acc2[jx][0] = fmaf(acc.acc2[jx][0], f1, o2.x * f2);
          acc.acc2[jx][1] = fmaf(acc.acc2[jx][1], f1, o2.y * f2);
          acc.acc2[jx][2] = fmaf(acc.acc2[jx][2], f1, o2.z * f2);
          acc.acc2[jx][3] = fmaf(acc.acc2[jx][3], f1, o2.w * f2);
        }
        acc.accl[0] = fmaf(acc.accl[0], f1, p[65] * f2);
        acc.m_run = m;
      }
      __syncthreads();  // before the next round's writes
    }
    if (tp > 0) return;
    if constexpr (NW * kStageWaveBytes <= (int)sizeof(ring)) {
      // Partials (split rows only: one split writes y) through the ring,
      // free after the merge's last barrier.
      if (a.nsplit > 1) {
        const int c0 = vh - col;
        store_partials_staged<half_t>(acc, reinterpret_cast<float*>(&ring[0][0][0][0]) +
                                               wave * (kStageWaveBytes / 4),
                                      a.part_o, a.part_ml, qrow0 + c0, min(16, a.GV - c0),
                                      a.nsplit, split, col, blk);
        return;
      }
    }
  }
  if (!col_ok) return;
  acc.store(a, qrow0 + vh, split, blk);
}


// ---------------------------------------------------- producer / consumer ---
// The same slab with the waves split by role, so that dequantisation (VALU)
// and attention (matrix cores) run at the same time on every SIMD: waves
// 0..3 are consumers (column block w % NCB, tile w / NCB of a step of
// NP = 4 / NCB tiles), waves 4..7 producers, one of each per SIMD.  Two LDS
// stages: in step j the consumers attend stage j % 2 while the producers
// dequantise step j + 1 into the other stage from the registers its loads
// landed in (issued two steps ahead, two register sets) and issue step
// j + 3's loads; one barrier ends the step.  Dequantisation is packed fp16:
// two codes become 1024 + u in the halves of one word (their byte or nibble
// under an fp16 exponent), a packed subtract leaves u exactly, and a packed
// fma gives s * u + b rounded once to fp16 -- the value mx.dequantize feeds
// the reference path's attention (src/mlx_motif/kernels/attention.py:497-499).
// NSET: register sets of packed step data per producer thread (NSET - 1
// steps in flight beside the one being dequantised).
template <int BITS, int GS, int NCB, int NSET = 2>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
sdpa_qslab_ws_kernel(SdpaArgs a) {
  using Acc = SwizzledTileAcc<half_t>;
  using V8 = Acc::V8;
  constexpr int D = 128;
  constexpr int TR = kPrefillTileRows;  // 32
  constexpr int NC = 4;                 // consumer waves
  constexpr int NP = NC / NCB;          // tiles per step
  constexpr int NG = D / GS;
  constexpr int RB = D * BITS / 8;   // packed bytes per row
  constexpr int CB = 16 * BITS / 8;  // packed bytes per 16-code chunk
  constexpr int CPT = 3 * NP;        // chunks per producer thread per step
  static_assert(NCB == 2 || NCB == 4, "2 or 4 column blocks");
  static_assert(GS % 16 == 0, "a chunk sits in one scale group");
  static_assert(NSET == 2 || NSET == 3, "2 or 3 register sets");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= NC;
  const int col = lane & 15;
  const int blk = lane >> 4;
  const int cb = wave % NCB;  // consumers: column block
  const int tp = wave / NCB;  // consumers: tile of the step

  int qblk, unit, split;
  if (!prefill_block_coords(a, blockIdx.x, qblk, unit, split)) return;  // grid padding
  const int b = unit / a.Hkv;
  const int kvh = unit % a.Hkv;
  const int wg_vh0 = qblk * NCB * 16;
  const int vh = wg_vh0 + cb * 16 + col;
  const bool col_ok = !producer && vh < a.GV;
  const int lim = col_ok ? vhead_limit(a, vh) : 0;
  const int lim_lo = qslab_block_limit_lo(a, wg_vh0 + cb * 16);
  const int max_lim = vhead_limit_max(a, wg_vh0, min(NCB * 16, a.GV - wg_vh0));
  const int r_begin = split * a.rows_per_split;
  const int r_end = min(r_begin + a.rows_per_split, max_lim);
  const int nrows = max(r_end - r_begin, 0);
  const int nsteps = (nrows + NP * TR - 1) / (NP * TR);
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q;

  // Ring stage st, tile p, tensor t: 32 rows x 256 bytes of fp16, 16-byte
  // chunk c of row r at byte r * 256 + (c ^ (r % 16)) * 16.  Reused by the
  // consumers' merge at the end.
  constexpr int STAGE_BYTES = NP * 3 * TR * D * 2;
  constexpr int MERGE_BYTES = NCB * (NP / 2) * 64 * kQslabMergeFloats * 4;
  static_assert(2 * STAGE_BYTES >= MERGE_BYTES, "merge fits the stages");
  __shared__ __attribute__((aligned(16))) uint8_t ring[2][NP][3][TR * D * 2];

  // Producers: thread p = tid - 256 handles row p / 8, 16-code chunk p % 8 of
  // every (tile, tensor) block k = 0 .. CPT - 1 of a step (tile k / 3,
  // tensor k % 3); eight lanes cover a row, so one load reads a tensor's
  // 32 rows contiguously.
  const int ptid = tid - NC * 64;
  const int crow = (ptid & 255) >> 3;
  const int cchunk = ptid & 7;
  const int cgroup = 16 * cchunk / GS;
  const long hrow0 = (long)unit * a.kv_cap + r_begin;
  const unsigned dbytes = (unsigned)(nrows * RB);
  const unsigned sbytes = (unsigned)(nrows * NG * 2);
  const __amdgpu_buffer_rsrc_t rd[3] = {
      stream_rsrc((const uint8_t*)a.kd + hrow0 * RB, dbytes),
      stream_rsrc((const uint8_t*)a.v1d + hrow0 * RB, dbytes),
      stream_rsrc((const uint8_t*)a.v2d + hrow0 * RB, dbytes)};
  const __amdgpu_buffer_rsrc_t rsc[3] = {
      stream_rsrc((const uint16_t*)a.ks + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1s + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2s + hrow0 * NG, sbytes)};
  const __amdgpu_buffer_rsrc_t rbi[3] = {
      stream_rsrc((const uint16_t*)a.kb + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v1b + hrow0 * NG, sbytes),
      stream_rsrc((const uint16_t*)a.v2b + hrow0 * NG, sbytes)};
  struct Packed {
    uint32_t w[CPT][CB / 4];
    uint32_t s[CPT], b[CPT];
  };
  auto load = [&](Packed& P, int step) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int t = k % 3;
      const unsigned row = (unsigned)((step * NP + k / 3) * TR + crow);
      const unsigned off = row * RB + (unsigned)(cchunk * CB);
      if constexpr (CB == 16) {
        const uint4 x = bload4(rd[t], off);
        P.w[k][0] = x.x; P.w[k][1] = x.y; P.w[k][2] = x.z; P.w[k][3] = x.w;
      } else {
        const uint2 x = bload2(rd[t], off);
        P.w[k][0] = x.x; P.w[k][1] = x.y;
      }
      const unsigned soff = (row * NG + (unsigned)cgroup) * 2u;
      P.s[k] = __builtin_amdgcn_raw_buffer_load_b16(rsc[t], soff, 0, kCachePolicyStream);
      P.b[k] = __builtin_amdgcn_raw_buffer_load_b16(rbi[t], soff, 0, kCachePolicyStream);
    }
  };
  auto dequant_store = [&](const Packed& P, int st) {
    const half2_t k1024 = half2_t{(_Float16)1024.f, (_Float16)1024.f};
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const uint32_t s16 = P.s[k] & 0xFFFFu, b16 = P.b[k] & 0xFFFFu;
      const half2_t s2 = as_h2(s16 | (s16 << 16));
      const half2_t b2 = as_h2(b16 | (b16 << 16));
      const uint32_t* cw = P.w[k];
      uint32_t h[8];  // codes (2i, 2i + 1) of the chunk
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t x;  // 1024 + u for both codes, as fp16 halves
        if constexpr (BITS == 8) {
          // bytes 2i%4, 2i%4 + 1 of word i / 2 under the exponent byte 0x64
          x = __builtin_amdgcn_perm(0x64646464u, cw[i / 2], (i & 1) ? 0x04030402u : 0x04010400u);
        } else {
          // the two nibbles of byte k = i % 4 of word i / 4: the word's low
          // and high nibble planes (shared by its four pairs), then byte k
          // of each into the low byte of one half and the exponent bits
          const uint32_t w = cw[i / 4];
          const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
          const uint32_t k = (uint32_t)(i % 4);
          x = __builtin_amdgcn_perm(hi, lo, 0x0C000C00u | ((4u + k) << 16) | k) | 0x64006400u;
        }
        const half2_t u = as_h2(x) - k1024;
        h[i] = h2_bits(__builtin_elementwise_fma(u, s2, b2));
      }
      uint8_t* base = ring[st][k / 3][k % 3] + crow * 256;
      const int c0 = (2 * cchunk) ^ (crow % 16);
      const int c1 = (2 * cchunk + 1) ^ (crow % 16);
      *reinterpret_cast<uint4*>(base + c0 * 16) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(base + c1 * 16) = make_uint4(h[4], h[5], h[6], h[7]);
    }
  };

  // Producers: loads of steps past the last read past the resources' ends
  // (zeros, no memory access).  The two roles run separate loops with the
  // same barriers (one per step, then the merge's), so their registers do
  // not add up; the step count is uniform over the workgroup, so every
  // barrier is reached by all of its threads.
  constexpr int kMergeBarriers = NP == 4 ? 4 : NP == 2 ? 2 : 0;
  if (producer) {
    // Step s in set s % NSET, loaded NSET steps ahead; after step 0 (alone
    // first: it lands sooner with nothing queued behind it), one
    // dequantisation and one barrier per step s = 1 .. nsteps (the last is
    // past the end: zeros, never consumed), unrolled by NSET so that the
    // compiler's wait before each set's dequantisation counts the other
    // sets' loads as still in flight.  Step s goes to ring stage s & 1.
    // (The scheduling barriers keep the dequantisation of the set due after
    // a barrier from being hoisted above it, where its wait would also
    // drain the loads of the other sets.)
    Packed P[NSET];
    load(P[0], 0);
    dequant_store(P[0], 0);
#pragma unroll
    for (int u = 1; u < NSET; ++u) load(P[u], u);
    load(P[0], NSET);
    qslab_barrier();
    int st = 1;  // st % NSET == 1 at the top of every pass
    for (; st + NSET - 1 <= nsteps; st += NSET) {
#pragma unroll
      for (int u = 0; u < NSET; ++u) {
        dequant_store(P[(1 + u) % NSET], (st + u) & 1);
        load(P[(1 + u) % NSET], st + u + NSET);
        qslab_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int u = 0; u + 1 < NSET; ++u) {
      if (st + u <= nsteps) {
        dequant_store(P[(1 + u) % NSET], (st + u) & 1);
        qslab_barrier();
      }
    }
#pragma unroll
    for (int i = 0; i < kMergeBarriers; ++i) __syncthreads();
    return;
  }

  Acc acc;
  acc.init();
  V8 qb[4];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (col_ok ? vh : 0)) * D + 8 * blk;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 w = col_ok ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
      qb[s] = __builtin_bit_cast(V8, w);
    }
  }
  qslab_barrier();
  for (int j = 0; j < nsteps; ++j) {
    const int t0 = r_begin + (j * NP + tp) * TR;
    acc.tile(ring[j & 1][tp][0], ring[j & 1][tp][1], ring[j & 1][tp][2], qb, t0, r_end, lim,
             a.qscale, col, blk, t0 + TR <= min(r_end, lim_lo));
    qslab_barrier();
  }

  // The NP consumer waves of a column block merge their (m, l, o) through
  // LDS (the ring is free after the last barrier); every wave takes part in
  // the barriers.
  if constexpr (NP > 1) {
    float* xo = reinterpret_cast<float*>(&ring[0][0][0][0]);  // [NCB][NP / 2][64 lanes][kQslabMergeFloats]
#pragma unroll
    for (int half = NP / 2; half >= 1; half /= 2) {
      if (tp >= half && tp < 2 * half) {
        float* p = xo + ((cb * (NP / 2) + tp - half) * 64 + lane) * kQslabMergeFloats;
#pragma unroll
        for (int jx = 0; jx < 8; ++jx) {
          *reinterpret_cast<float4*>(p + 4 * jx) =
              make_float4(acc.acc1[jx][0], acc.acc1[jx][1], acc.acc1[jx][2], acc.acc1[jx][3]);
          *reinterpret_cast<float4*>(p + 32 + 4 * jx) =
              make_float4(acc.acc2[jx][0], acc.acc2[jx][1], acc.acc2[jx][2], acc.acc2[jx][3]);
        }
        p[64] = acc.m_run;
        p[65] = acc.accl[0];
      }
      __syncthreads();
      if (tp < half) {
        const float* p = xo + ((cb * (NP / 2) + tp) * 64 + lane) * kQslabMergeFloats;
        const float m2 = p[64];
        const float m = fmaxf(acc.m_run, m2);
        const float f1 = fast_exp2(acc.m_run - m);
        const float f2 = fast_exp2(m2 - m);
#pragma unroll
        for (int jx = 0; jx < 8; ++jx) {
          const float4 o1 = *reinterpret_cast<const float4*>(p + 4 * jx);
          const float4 o2 = *reinterpret_cast<const float4*>(p + 32 + 4 * jx);
          acc.acc1[jx][0] = fmaf(acc.acc1[jx][0], f1, o1.x * f2);
          acc.acc1[jx][1] = fmaf(acc.acc1[jx][1], f1, o1.y * f2);
          acc.acc1[jx][2] = fmaf(acc.acc1[jx][2], f1, o1.z * f2);
          acc.acc1[jx][3] = fmaf(acc.acc1[jx][3], f1, o1.w * f2);
          acc.acc2[jx][0] = fmaf(acc.acc2[jx][0], f1, o2.x * f2);
          acc.acc2[jx][1] = fmaf(acc.acc2[jx][1], f1, o2.y * f2);
          acc.acc2[jx][2] = fmaf(acc.acc2[jx][2], f1, o2.z * f2);
          acc.acc2[jx][3] = fmaf(acc.acc2[jx][3], f1, o2.w * f2);
        }
        acc.accl[0] = fmaf(acc.accl[0], f1, p[65] * f2);
        acc.m_run = m;
      }
      __syncthreads();
    }
  }
  if (tp > 0) return;
  if constexpr (NP > 1 && 8 * kStageWaveBytes <= (int)sizeof(ring)) {
    // Partials (split rows only: one split writes y) through the ring, free
    // after the merge's last barrier.
    if (a.nsplit > 1) {
      const int c0 = vh - col;
      store_partials_staged<half_t>(acc, reinterpret_cast<float*>(&ring[0][0][0][0]) +
                                             wave * (kStageWaveBytes / 4),
                                    a.part_o, a.part_ml, qrow0 + c0, min(16, a.GV - c0),
                                    a.nsplit, split, col, blk);
      return;
    }
  }
  if (!col_ok) return;
  acc.store(a, qrow0 + vh, split, blk);
}

}  // namespace motif
