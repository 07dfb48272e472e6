// Multi-row (chunked-prefill / long verify) dual-V attention over the fp16
// cache at head_dim 128, on matrix cores with K/V tiles shared through LDS.
//
// The split-KV decode kernel gives each workgroup at most 16 virtual heads
// (query head x query row) and re-reads every KV row once per head chunk,
// which for S_q rows of a prefill means G*S_q/16 reads of the cache.  Here a
// workgroup holds NW waves x 16 virtual heads (consecutive query rows of one
// head), and every 32-row K/V tile is loaded from HBM once per workgroup into
// LDS and read by all of its waves:
//   - staging: each thread loads its 16-byte pieces of the next tile into
//     registers while the current tile is computed, then writes them to the
//     other LDS buffer (double buffering, one barrier per tile);
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
constexpr int kPrefillRowHalves = 128 + 8;  // LDS row stride (halves): 16-byte pad

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

template <int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
sdpa_prefill_f16_kernel(SdpaArgs a) {
  constexpr int D = 128;
  constexpr int TR = kPrefillTileRows;
  constexpr int RS = kPrefillRowHalves;
  constexpr int NT = NW * 64;
  constexpr int CHUNKS = TR * D * 2 / 16;  // 16-byte pieces per tensor tile
  constexpr int CPT = CHUNKS / NT;           // pieces per thread per tensor
  static_assert(CHUNKS % NT == 0, "whole pieces per thread");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int blk = lane >> 4;

  int qblk, unit, split;
  if (!prefill_block_coords(a, blockIdx.x, qblk, unit, split)) return;  // grid padding
  const int b = unit / a.Hkv;
  const int kvh = unit % a.Hkv;
  const int wg_vh0 = qblk * NW * 16;
  const int vh = wg_vh0 + wave * 16 + col;  // this lane's virtual head (column)
  const bool col_ok = vh < a.GV;
  const int lim = col_ok ? vhead_limit(a, vh) : 0;
  int max_lim = 0;
  for (int g = wg_vh0; g < min(wg_vh0 + NW * 16, a.GV); ++g)
    max_lim = max(max_lim, vhead_limit(a, g));
  const int r_begin = split * a.rows_per_split;
  const int r_end = min(r_begin + a.rows_per_split, max_lim);
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q;  // row of virtual head 0

  // Q^T, B operand of the 16x16x32 MFMA: lane (col, blk) holds its column's
  // channels 32*s + 8*blk .. +7 for k-step s.
  half8_t qb[4];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (qrow0 + (col_ok ? vh : 0)) * D + 8 * blk;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 w = col_ok ? *reinterpret_cast<const uint4*>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
      qb[s] = __builtin_bit_cast(half8_t, w);
    }
  }

  // Rows [r_begin, r_end) of this KV head through range-checked resources.
  const long hrow0 = (long)unit * a.kv_cap + r_begin;
  const unsigned nbytes = (unsigned)(max(r_end - r_begin, 0) * D * 2);
  const __amdgpu_buffer_rsrc_t rsrc[3] = {
      stream_rsrc((const uint16_t*)a.k + hrow0 * D, nbytes),
      stream_rsrc((const uint16_t*)a.v1 + hrow0 * D, nbytes),
      stream_rsrc((const uint16_t*)a.v2 + hrow0 * D, nbytes)};

  __shared__ __attribute__((aligned(16))) uint16_t lds_kv[2][3][TR * RS];
  // Staged pieces of the next tile (registers), written to the idle LDS
  // buffer after the current tile is computed.  A second register set (two
  // tiles in flight) spills at this register budget.
  uint4 stage[3][CPT];
  auto load_stage = [&](int t0) {  // t0: split-relative first row of the tile
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int piece = threadIdx.x + c * NT;
      const unsigned off = (unsigned)((t0 + piece / 16) * D * 2 + (piece % 16) * 16);
#pragma unroll
      for (int t = 0; t < 3; ++t) stage[t][c] = bload4(rsrc[t], off);
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int piece = threadIdx.x + c * NT;
      const int o = (piece / 16) * RS + (piece % 16) * 8;
#pragma unroll
      for (int t = 0; t < 3; ++t) *reinterpret_cast<uint4*>(&lds_kv[buf][t][o]) = stage[t][c];
    }
  };

  floatx4 acc1[8], acc2[8], accl;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc1[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  accl = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegSentinel;
  const half8_t ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f,
                        (_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};

  // One 32-row tile from LDS buffer buf: rows t0 + 16*h + 4*blk + r hold
  // k index 8*blk + 4*h + r of the PV products (as in the decode kernel).
  auto compute = [&](int buf, int t0) {
    const uint16_t* Kt = lds_kv[buf][0];
    const uint16_t* V1t = lds_kv[buf][1];
    const uint16_t* V2t = lds_kv[buf][2];
    floatx4 sacc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sacc[h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const half8_t ka = __builtin_bit_cast(
            half8_t, *reinterpret_cast<const uint4*>(&Kt[(16 * h + col) * RS + 32 * s + 8 * blk]));
        sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[s], sacc[h], 0, 0, 0);
      }
    }
    float sc[8];
    float mx = kNegSentinel;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r_begin + t0 + 16 * h + 4 * blk + r;
        const bool ok = row < r_end && row < lim;
        sc[4 * h + r] = ok ? sacc[h][r] * a.qscale : kNegSentinel;
        mx = fmaxf(mx, sc[4 * h + r]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
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
    half8_t pb;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      pb[j] = (_Float16)(sc[j] > kNegSentinel ? fast_exp2(sc[j] - m_run) : 0.f);

    // V rows 16*h + 4*blk + r, channels 8*col .. 8*col+7 (dword t holds
    // channels 8*col + 2t, +1).
    uint32_t v1w[2][4][4], v2w[2][4][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = (16 * h + 4 * blk + r) * RS + 8 * col;
        const uint4 w1 = *reinterpret_cast<const uint4*>(&V1t[o]);
        const uint4 w2 = *reinterpret_cast<const uint4*>(&V2t[o]);
        v1w[h][r][0] = w1.x; v1w[h][r][1] = w1.y; v1w[h][r][2] = w1.z; v1w[h][r][3] = w1.w;
        v2w[h][r][0] = w2.x; v2w[h][r][1] = w2.y; v2w[h][r][2] = w2.z; v2w[h][r][3] = w2.w;
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint32_t sel = hh ? 0x07060302u : 0x05040100u;  // hi or lo halves
        const half8_t a1 = __builtin_bit_cast(
            half8_t, make_uint4(__builtin_amdgcn_perm(v1w[0][1][t], v1w[0][0][t], sel),
                                __builtin_amdgcn_perm(v1w[0][3][t], v1w[0][2][t], sel),
                                __builtin_amdgcn_perm(v1w[1][1][t], v1w[1][0][t], sel),
                                __builtin_amdgcn_perm(v1w[1][3][t], v1w[1][2][t], sel)));
        const half8_t a2 = __builtin_bit_cast(
            half8_t, make_uint4(__builtin_amdgcn_perm(v2w[0][1][t], v2w[0][0][t], sel),
                                __builtin_amdgcn_perm(v2w[0][3][t], v2w[0][2][t], sel),
                                __builtin_amdgcn_perm(v2w[1][1][t], v2w[1][0][t], sel),
                                __builtin_amdgcn_perm(v2w[1][3][t], v2w[1][2][t], sel)));
        acc1[2 * t + hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, pb, acc1[2 * t + hh], 0, 0, 0);
        acc2[2 * t + hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, pb, acc2[2 * t + hh], 0, 0, 0);
      }
    }
    accl = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb, accl, 0, 0, 0);
  };

  // Every workgroup's tile count is uniform, so every barrier is reached by
  // all of its threads.  Tile i sits in LDS buffer i % 2; the store into
  // buffer (i + 1) % 2 follows the barrier that ended tile i - 1's reads.
  const int nrows = max(r_end - r_begin, 0);
  const int ntiles = (nrows + TR - 1) / TR;
  if (ntiles > 0) {
    load_stage(0);
    store_stage(0);
  }
  __syncthreads();
  for (int i = 0; i < ntiles; ++i) {
    const int buf = i & 1;
    if (i + 1 < ntiles) load_stage((i + 1) * TR);
    compute(buf, i * TR);
    if (i + 1 < ntiles) store_stage(buf ^ 1);
    __syncthreads();
  }

  // acc[j][r] of lane (col, blk) is channel 8*(4*blk + r) + j of column col.
  if (!col_ok) return;
  const long vrow = qrow0 + vh;
  const float l = accl[0];
  if (a.nsplit == 1) {
    const float inv = l == 0.f ? 1.f : 1.f / l;  // o stays 0 when no key is visible
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ch = 8 * (4 * blk + r);
      uint32_t w1[4], w2[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const half2_t x1 = half2_t{(_Float16)(acc1[2 * p][r] * inv), (_Float16)(acc1[2 * p + 1][r] * inv)};
        const half2_t x2 = half2_t{(_Float16)(acc2[2 * p][r] * inv), (_Float16)(acc2[2 * p + 1][r] * inv)};
        w1[p] = __builtin_bit_cast(uint32_t, x1);
        w2[p] = __builtin_bit_cast(uint32_t, x2);
      }
      uint16_t* yp = (uint16_t*)a.y + vrow * 2 * D;
      *reinterpret_cast<uint4*>(yp + ch) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
      *reinterpret_cast<uint4*>(yp + D + ch) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    }
  } else {
    const int ns = a.nsplit;
    float* po = a.part_o + (vrow * ns + split) * 2 * D;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ch = 8 * (4 * blk + r);
      *reinterpret_cast<float4*>(po + ch) = make_float4(acc1[0][r], acc1[1][r], acc1[2][r], acc1[3][r]);
      *reinterpret_cast<float4*>(po + ch + 4) = make_float4(acc1[4][r], acc1[5][r], acc1[6][r], acc1[7][r]);
      *reinterpret_cast<float4*>(po + D + ch) = make_float4(acc2[0][r], acc2[1][r], acc2[2][r], acc2[3][r]);
      *reinterpret_cast<float4*>(po + D + ch + 4) = make_float4(acc2[4][r], acc2[5][r], acc2[6][r], acc2[7][r]);
    }
    if (blk == 0)
      *reinterpret_cast<float2*>(a.part_ml + (vrow * ns + split) * 2) = make_float2(m_run, l);
  }
}

inline int launch_prefill_kernel_f16(const SdpaArgs& a, int waves, int nblocks, hipStream_t st) {
  if (waves == 8) {
    hipLaunchKernelGGL((sdpa_prefill_f16_kernel<8>), dim3(nblocks), dim3(512), 0, st, a);
  } else {
    hipLaunchKernelGGL((sdpa_prefill_f16_kernel<4>), dim3(nblocks), dim3(256), 0, st, a);
  }
  return check_launch("sdpa_dual_v_rows (prefill)");
}

}  // namespace motif
