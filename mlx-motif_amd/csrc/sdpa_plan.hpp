// Host-side launch plan of the split-KV dual-V attention kernels: how the
// query heads of one KV head are chunked, how the live KV rows are split
// across workgroups, and where counters and partials sit in the workspace.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "motif_common.hpp"

namespace motif {

// Everything a split-KV launch needs, shared by every cache format.
struct SdpaArgs {
  const void* q;  // (B, Hq, S_q, D)
  // fp16/bf16/fp32 cache (B, Hkv, kv_cap, D)
  const void* k;
  const void* v1;
  const void* v2;
  // packed cache: data u32 (B,Hkv,kv_cap,D*bits/32), scales/biases (B,Hkv,kv_cap,D/gs)
  const uint32_t* kd;
  const void* ks;
  const void* kb;
  const uint32_t* v1d;
  const void* v1s;
  const void* v1b;
  const uint32_t* v2d;
  const void* v2s;
  const void* v2b;
  void* y;             // (B, Hq, S_q, 2D)
  float* part_o;       // [B*Hq*S_q][nsplit][2D]
  float* part_ml;      // [B*Hq*S_q][nsplit][2]  (running max in log2 units, sum)
  unsigned* counters;  // [B*Hkv*nchunk] arrival counters, zero between calls
  int B, Hq, Hkv, S_q;
  int G;       // Hq / Hkv
  int GV;      // virtual heads per KV head = G * S_q (one per (head, query row))
  int nchunk;  // ceil(GV / GC): workgroups per KV head and split
  int kv_cap, kv_len, causal;
  // Splits per (b, KV head, chunk).  The VALU and shared-tile kernels give
  // split s the contiguous rows [s * rows_per_split, (s + 1) * rows_per_split);
  // the matrix-core decode kernels deal blocks of (waves x 16) rows to the
  // splits round robin and ignore rows_per_split.
  int nsplit, rows_per_split;
  // Shared-tile multi-row kernel: its 32-row tiles dealt to the splits round
  // robin (1: tile i of split s is tile i * nsplit + s) or in contiguous
  // ranges of rows_per_split rows (0).
  int tiles_rr;
  int group_size;
  int fused_merge;  // 1: last-arriving workgroup merges; 0: sdpa_merge_kernel does
  // Split partial outputs stored as fp16 o / l (the shared-tile kernels of
  // prefill chunks, whose partials the row-per-wave merge reads) instead of
  // fp32 o: half the bytes written and read back.
  int part_f16;
  float qscale;     // softmax scale * log2(e)
  // Fused GDA decode step (origin and noise passes in one launch, then the
  // merge applies gda_post_split): q holds the origin queries (B, Hq, 1, D)
  // with Hq = Hkv * G, q2 the noise queries (B, Hkv * G2, 1, D), k the
  // origin keys, k2 the noise keys; partial rows are (b, KV head, column)
  // with columns 0..G-1 the origin heads and G..G+G2-1 the noise heads
  // (G2 below; one in the 12.7B layout, G / G2 origin heads per noise head).
  const void* q2;
  const void* k2;
  const uint32_t* k2d;  // packed noise keys (data, scales, biases)
  const void* k2s;
  const void* k2b;
  const void* gda_w;         // (2D) subln weight
  const float* gda_lambda;   // device pointer to lambda_full (fp32)
  float gda_scale;           // 1 - lambda_init
  float gda_eps;
  // Fused decode step with append (append != 0): the new token's rows of
  // the four slots (B, Hkv, 1, D), written at row kv_len - 1 of the cache
  // (quantised for the packed cache) by the one wave whose tiles include
  // that row, before it loads the row.
  const void* new_k1;
  const void* new_k2;
  const void* new_v1;
  const void* new_v2;
  int append;
  // Decode step from the projection outputs (from_proj != 0, with append):
  // q is q_proj (B, 1, Hkv*(G+1)*D), heads g*(G+1)+j (origin j < G, noise
  // j = G), or origin-first (q_origin_first); new_k1 is k_proj (B, 1,
  // 2*Hkv*D: k1[g] = head 2g, k2[g] = 2g+1) and new_v1 v_proj (same head
  // pairing for v1/v2).  q and the new k rows are roped at position
  // kv_len - 1 (rope_impl.hpp) before use.
  int from_proj;
  int q_origin_first;
  float rope_log2_theta;
  float rope_pos_scale = 1.f;  // RoPE position scale: 1, or 1 / factor (linear scaling)
  // Prefill chunk of a GDA layer from the projection outputs
  // (gda_prefill_proj_kernel): q is q_proj (B, S_q, q_groups*(q_gr+1)*D),
  // new_k1 k_proj and new_v1 v_proj (B, S_q, 2*Hkv*D; k1[g] = head 2g,
  // k2[g] = 2g+1, likewise v1/v2).  Query blocks [0, nqb_origin) of a
  // (b, KV head, split) run the origin pass (G heads per KV head: q1 x k1,
  // output y), the others the noise pass (G2 heads: q2 x k2, output y2,
  // whose split partials start at row y2_row0).  The chunk is cache rows
  // kv_len - S_q .. kv_len - 1, roped at positions rope_pos0 + s.
  void* y2;
  long y2_row0;
  int nqb_origin;
  int G2;  // noise heads per KV head (the prefill chunk and the fused decode step)
  int q_groups, q_gr;
  int rope_pos0;
};

struct SdpaPlan {
  int gc;              // virtual heads per workgroup (1, 2, 4 or 8)
  int nchunk;
  int nsplit;
  int rows_per_split;
  int waves;           // waves per workgroup
  size_t counter_bytes;
  size_t workspace_bytes;
};

// Grid of a split-KV launch: one workgroup per (b, KV head, chunk, split).
// With several chunks, groups of 8 (b, KV head, split) are padded so that
// sdpa_block_coords() can place the chunks of one group on one XCD.
inline int sdpa_grid_blocks(int bh, int nchunk, int nsplit) {
  const int groups = bh * nsplit;
  return nchunk == 1 ? groups : (groups + 7) / 8 * 8 * nchunk;
}

// Upper bound on splits per (b, KV head, chunk): the final merge keeps every
// split's (m, l) pair in LDS.
constexpr int kMaxSplits = 256;

// gc_max: the largest per-workgroup head count compiled for this head dim.
// waves_pref: waves per workgroup (0: 8 where the LDS merge fits, else 4);
// wgs_per_cu: workgroups one CU holds at once (0: 8 / waves).
// gc_fixed > 0: exactly that many heads per workgroup (the packed-cache
// kernel's multi-block launches, which also hold one workgroup per CU), in
// place of a power of two <= gc_max.
SdpaPlan plan_sdpa(int B, int Hq, int Hkv, int S_q, int kv_len, int D, int gc_max,
                   int waves_pref, int wgs_per_cu, int gc_fixed = 0);

// Plan of the multi-row kernel with LDS-shared K/V tiles (fp16 cache, head
// dim 128): query blocks of waves x 16 virtual heads, rows split over
// workgroups only when the query blocks do not fill the GPU.  Used when a KV
// head has at least kPrefillMinHeads virtual heads.
constexpr int kPrefillMinHeads = 64;
// Whether a multi-row fp16/bf16 call of GV virtual heads per KV head over
// kv_len rows takes the shared-tile kernel: from kPrefillMinHeads heads (or
// the "prefill_min_heads" tuning), and from 17 heads (two decode head
// chunks, each reading the cache) over 2048+ rows.  Measured, 32 q-heads
// over 8 KV heads, decode chunks / shared tiles: 5 rows over 1024 9.6 /
// 10.2 us, over 3204 17.6 / 12.3, over 16000 34.5 / 26.3, over 32768 59.2 /
// 45.5; 8 rows over 16000 38.3 / 28.2.
bool use_shared_tiles(int GV, int kv_len);
constexpr int kPrefillTileRowsHost = 32;  // KV rows per tile (kPrefillTileRows)
struct PrefillPlan {
  int waves;  // 4 or 8
  int ncb;    // column blocks of 16 virtual heads per wave (1 or 2)
  int nqb;    // query blocks per (b, KV head)
  int nsplit, rows_per_split;
  size_t workspace_bytes;  // counters + partials, 0 when nsplit == 1
};
PrefillPlan plan_prefill(int B, int Hq, int Hkv, int S_q, int kv_len, int D);

// Plan of a GDA layer's prefill chunk from the projections
// (gda_prefill_proj_kernel): per (b, KV head) nqb_origin query blocks of the
// origin pass (G_origin heads x S rows) and nqb_noise of the noise pass
// (G_noise heads x S rows) of waves x 16 virtual heads each; rows are split
// (to about one workgroup per CU) only when the blocks fill fewer than half
// the CUs.  Partial rows (nsplit > 1): the origin pass's B*Hkv*G_origin*S,
// then the noise pass's.
struct GdaPrefillPlan {
  int waves;
  int ncb;  // column blocks of 16 virtual heads per wave (1 or 2)
  int nqb_origin, nqb_noise;
  int nsplit, rows_per_split;
  size_t workspace_bytes;  // counters + partials, 0 when nsplit == 1
};
GdaPrefillPlan plan_gda_prefill(int B, int Hkv, int G_origin, int G_noise, int S, int kv_len);

// Plan of the packed-cache slab kernel (sdpa_qslab.hpp): ncb column blocks of
// 16 virtual heads per workgroup (2 when the heads of a KV head fit 32
// columns, else 4), nchunk head chunks of ncb * 16, and the rows of a KV head
// split so that about one workgroup per CU runs; each split is a whole
// number of steps (waves / ncb tiles of 32 rows).  Used for packed
// caches at head_dim 128 when a KV head has more than 16 and at most
// kQSlabMaxHeads virtual heads.
constexpr int kQSlabMinHeads = 17;
constexpr int kQSlabMaxHeads = 64;
struct QSlabPlan {
  int ncb, nchunk;
  int waves;  // 8 (two per SIMD, one LDS stage) or 4 (tuning waves_per_wg 4)
  int nsplit, rows_per_split;
  size_t workspace_bytes;  // counters + partials
};
QSlabPlan plan_qslab(int B, int Hq, int Hkv, int S_q, int kv_len, int D);

// The matrix-core decode kernels deal 16-row tiles of a whole KV head to
// their splits and address them with 32-bit byte offsets from the head's
// first row: they take kv_len <= kMfmaMaxRows (the VALU kernels take the
// rest).
constexpr int kMfmaMaxRows = 1 << 22;

// Partial rows (B * Hq * S_q) from which a split call's merge launch runs one
// wave per row (tuning merge_rows) instead of one wave per row slice.
constexpr int kMergeRowsMin = 2048;
// The shared-tile kernels store split partials as fp16 o / l (SdpaArgs::
// part_f16) when the row-per-wave merge will read them, over fp16 caches
// only: o / l is a convex combination of the V rows, within fp16 range for
// an fp16 cache but not for a bf16 one (those keep fp32 partials).
inline bool use_part_f16(long rows, int nsplit, bool f16_cache) {
  return nsplit > 1 && f16_cache && rows >= kMergeRowsMin && tuning().merge_rows &&
         tuning().part_f16;
}

// The tile-softmax kernels (shared-tile prefill and slab kernels, the packed
// slab kernel, the paired-tile q4 kernel and the fused prefill chunk) take
// each tile's running maximum over the unscaled scores and scale it after,
// which is the maximum of the scaled scores only for a positive, finite
// scale.  Calls with any other scale (the reference accepts every float)
// take the per-tile kernels, which scale every score before the maximum.
// qscale is the softmax scale times log2(e).
inline bool tile_softmax_scale_ok(float qscale) {
  return qscale > 0.f && qscale <= 3.4028234663852886e38f;
}
// Single-row fp16/bf16 decode calls over at most this many rows run 4-wave
// workgroups, one per CU, instead of 8-wave ones: with few rows per split
// the smaller blocks reach their first tile sooner (32 q-heads over 8 KV
// heads, D 128, µs per call 8 / 4 waves: 1024 rows 8.84 / 7.51, 2048 9.08 /
// 8.07, 3204 9.59 / 9.20, 4096 9.97 / 9.69, 6144 12.19 / 12.09, 8192 13.59 /
// 14.03).  The fused decode step (both passes over k1/k2/v1/v2, the
// token's row written inside the launch) follows the same rule: 1024 rows
// 12.58 / 10.25, 2048 12.74 / 11.03, 3204 13.92 / 13.47, 4096 14.32 / 13.96.
constexpr int kShortDecodeRows = 4096;

// Plan of the packed-cache matrix-core kernel (head_dim 128, fp16): 4-wave
// workgroups at one wave per SIMD, one per CU.
constexpr int kSdpaMfmaQD = 128;
constexpr int kSdpaMfmaQWaves = 4;
constexpr int kSdpaMfmaQWgsPerCu = 1;

// Largest head chunk compiled for head dim D (register budget).
inline int sdpa_gc_max(int D) { return D <= 128 ? 8 : 4; }

// Largest head chunk of the fp16/bf16 matrix-core kernel (head_dim 128):
// the 16 MFMA columns, with 4-wave workgroups for the cross-wave LDS merge.
constexpr int kSdpaMfmaGcMax = 16;
// Head dims of the single-pass fp16/bf16 matrix-core decode kernel: 128, or
// 64 with a 16-byte aligned K (its rows are read 16 bytes per lane).
inline bool mfma16_head_dim_ok(int D, const void* k) {
  return D == 128 || (D == 64 && ((uintptr_t)k & 15u) == 0);
}

// Largest head chunk for the packed cache's matrix-core kernel: heads times
// scale groups share the 16 MFMA columns.
inline int sdpa_gc_max_q(int D, int group_size) {
  const int ng = D / group_size;
  const int lim = 16 / (ng > 0 ? ng : 1);
  const int base = sdpa_gc_max(D);
  return lim < base ? lim : base;
}

// Column blocks per wave of the packed-cache kernel for GV virtual heads per
// KV head: 2 when they need more than one block of sdpa_gc_max_q(D, gs)
// heads but fit two (one pass over the cache instead of two head chunks),
// else 1.  Measured on a q8 slab at 32768 rows: 16 heads 41.9 -> 37.6 us; for
// 20 heads two chunks of two blocks were slower than three chunks of one
// (55.8 vs 52.9 us), and a third block's accumulators spill.
constexpr int kSdpaMfmaQMaxBlocks = 2;
inline int sdpa_q_blocks(int GV, int D, int group_size) {
  const int gcq = sdpa_gc_max_q(D, group_size);
  return GV > gcq && GV <= kSdpaMfmaQMaxBlocks * gcq ? kSdpaMfmaQMaxBlocks : 1;
}

}  // namespace motif
