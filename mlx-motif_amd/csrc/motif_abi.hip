// C-ABI plumbing shared by every entry point: thread-local error messages,
// tuning knobs, device queries and the split-KV launch plan.
#include <algorithm>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "motif_common.hpp"
#include "sdpa_plan.hpp"

namespace motif {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return MOTIF_ERR_HIP;
  }
  return MOTIF_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

static std::mutex g_tuning_mu;
static Tuning g_tuning;                    // written only under g_tuning_mu
static thread_local Tuning tl_tuning;      // this thread's snapshot
static thread_local int tl_scope_depth = 0;

static void snapshot_tuning() {
  std::lock_guard<std::mutex> lock(g_tuning_mu);
  tl_tuning = g_tuning;
}

const Tuning& tuning() {
  if (tl_scope_depth == 0) snapshot_tuning();
  return tl_tuning;
}

CallScope::CallScope() {
  if (tl_scope_depth++ == 0) snapshot_tuning();
}

CallScope::~CallScope() { --tl_scope_depth; }

// motif_set_tuning: applies f to the shared knobs under their lock.
template <typename F>
static void update_tuning(F f) {
  std::lock_guard<std::mutex> lock(g_tuning_mu);
  f(g_tuning);
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

SdpaPlan plan_sdpa(int B, int Hq, int Hkv, int S_q, int kv_len, int D, int gc_max,
                   int waves_pref, int wgs_per_cu, int gc_fixed) {
  SdpaPlan p{};
  const int G = Hkv > 0 ? Hq / Hkv : 1;
  const int GV = G * S_q;
  int gc = 1;
  while (gc < GV && gc < gc_max) gc *= 2;
  if (gc_fixed > 0) gc = gc_fixed;
  p.gc = gc;
  p.nchunk = (GV + gc - 1) / gc;
  // 8-wave workgroups when their cross-wave LDS merge fits (D * gc <= 512
  // floats per wave per slab), else 4.
  const int max_waves = (D * gc <= 512) ? 8 : 4;
  p.waves = tuning().waves_per_wg ? tuning().waves_per_wg
                                  : (waves_pref > 0 && waves_pref < max_waves ? waves_pref : max_waves);
  if (p.waves > max_waves) p.waves = max_waves;

  const int units = B * Hkv * p.nchunk;
  // Rows one block iteration of a workgroup consumes: waves x rows per wave
  // load (4 for 16 lanes per row) x unroll 4.  Splits are whole iterations.
  const int step = p.waves * 4 * 4;
  // Default: one round of workgroups over the CUs (an 8-wave workgroup
  // fills a CU at two waves per SIMD; a 4-wave one fills half of it, or all
  // of it for kernels that run one wave per SIMD: wgs_per_cu = 1).
  // With several head chunks per KV head (a verify slab), each chunk's
  // workgroups should still cover the CUs: up to 3x more workgroups.
  int per_cu = wgs_per_cu > 0 ? wgs_per_cu * (p.nchunk < 3 ? p.nchunk : 3) : 8 / p.waves;
  if (gc_fixed > 0) per_cu = 1;  // multi-block kernels run one wave per SIMD
  int min_wgs = tuning().min_wgs > 0 ? tuning().min_wgs : device_cu_count() * per_cu;
  int rows = kv_len > 0 ? kv_len : 1;
  int rps;
  if (tuning().rows_per_split > 0) {
    rps = (int)round_up((size_t)tuning().rows_per_split, 16);  // whole 16-row tiles
  } else {
    int nsplit = (min_wgs + units - 1) / units;
    int max_split = (rows + step - 1) / step;  // at least one iteration each
    if (nsplit > max_split) nsplit = max_split;
    if (nsplit < 1) nsplit = 1;
    rps = (int)round_up((size_t)((rows + nsplit - 1) / nsplit), (size_t)step);
  }
  // The merge holds every split's (m, l) in LDS: at most kMaxSplits splits.
  const int min_rps = (rows + kMaxSplits - 1) / kMaxSplits;
  if (rps < min_rps) rps = (int)round_up((size_t)min_rps, (size_t)step);
  p.rows_per_split = rps;
  p.nsplit = (rows + rps - 1) / rps;
  if (p.nsplit < 1) p.nsplit = 1;

  const size_t vrows = (size_t)B * Hq * S_q;
  p.counter_bytes = round_up(vrows * sizeof(unsigned), 256);
  size_t part = 0;
  if (p.nsplit > 1) {
    part = round_up(vrows * p.nsplit * 2 * D * sizeof(float), 256) +
           round_up(vrows * p.nsplit * 2 * sizeof(float), 256);
  }
  p.workspace_bytes = p.counter_bytes + part;
  return p;
}

bool use_shared_tiles(int GV, int kv_len) {
  const int t = tuning().prefill_min_heads;
  if (t > 0) return GV >= t;
  return GV >= kPrefillMinHeads || (GV > 16 && kv_len >= 2048);
}

PrefillPlan plan_prefill(int B, int Hq, int Hkv, int S_q, int kv_len, int D) {
  PrefillPlan p{};
  const int G = Hkv > 0 ? Hq / Hkv : 1;
  const int GV = G * S_q;
  const int cus = device_cu_count();
  const int bh = B * Hkv;
  // 8 waves (128 virtual heads per block, two waves per SIMD) from 512
  // virtual heads per KV head on, even if the row splits that fill the GPU
  // then need the merge launch; 4 below (measured, 32 q-heads over 8 KV
  // heads: 512 rows over 3716 157 -> 127 us, 256 rows 93 -> 76 us; at 64
  // rows 4 waves were faster, 41 vs 47 us, now even).  Slabs of fewer than
  // 64 heads (17..63 over 2048+ rows) take 8 waves too: the waves past the
  // heads only copy tiles, and the extra copy issuers help a read-bound
  // block (5 rows over 32768: 38.0 vs 40.3 us; over 16000: 23.3 vs 24.9; 8
  // rows over 16000: 23.8 vs 25.5).
  p.waves = GV >= 512 || GV < kPrefillMinHeads ? 8 : 4;
  if (tuning().waves_per_wg) p.waves = tuning().waves_per_wg;
  // Two column blocks per wave (256 virtual heads per 8-wave block: each
  // K/V fragment read from LDS feeds twice the MFMAs) from 2048 virtual heads
  // per KV head over at least 2048 rows (on fewer rows the halved block
  // count costs more than the LDS reads save: a first 512-row layer chunk
  // 42.8 vs 55.5 us).  Measured, 32 q-heads over 8 KV heads, one / two blocks:
  // 256 rows over 3204 55.4 / 61.9 us, 512 over 3716 90.3 / 87.3, 1024 over
  // 4228 145.6 / 138.8, 2048 over 4228 283.5 / 210.0, 4096 over 8192
  // 1005.9 / 781.1 (1.06 PFLOP/s).
  const int ncb_t = tuning().prefill_ncb;
  p.ncb = p.waves == 8 && (ncb_t == 2 || (ncb_t == 0 && GV >= 2048 && kv_len >= 2048)) ? 2 : 1;
  const int cols = p.waves * 16 * p.ncb;
  p.nqb = (GV + cols - 1) / cols;
  const long units = (long)bh * p.nqb;
  const int rows = kv_len > 0 ? kv_len : 1;
  int nsplit = units >= cus ? 1 : (int)((cus + units - 1) / units);
  const int max_split = (rows + 127) / 128;  // at least 128 rows per split
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit > kMaxSplits) nsplit = kMaxSplits;
  if (nsplit < 1) nsplit = 1;
  int rps = (rows + nsplit - 1) / nsplit;
  if (tuning().rows_per_split > 0)  // forced split size, at most kMaxSplits splits
    rps = std::max(tuning().rows_per_split, (rows + kMaxSplits - 1) / kMaxSplits);
  rps = (rps + kPrefillTileRowsHost - 1) / kPrefillTileRowsHost * kPrefillTileRowsHost;
  p.rows_per_split = rps;
  p.nsplit = (rows + rps - 1) / rps;
  if (p.nsplit < 1) p.nsplit = 1;
  if (p.nsplit > 1) {
    const size_t vrows = (size_t)B * Hq * S_q;
    p.workspace_bytes = round_up(vrows * sizeof(unsigned), 256) +
                        round_up(vrows * p.nsplit * 2 * D * sizeof(float), 256) +
                        round_up(vrows * p.nsplit * 2 * sizeof(float), 256);
  }
  return p;
}

GdaPrefillPlan plan_gda_prefill(int B, int Hkv, int G_origin, int G_noise, int S, int kv_len) {
  GdaPrefillPlan p{};
  p.waves = G_origin * S >= 512 ? 8 : 4;  // as plan_prefill
  if (tuning().waves_per_wg) p.waves = tuning().waves_per_wg;
  const int ncb_t = tuning().prefill_ncb;  // as plan_prefill
  p.ncb = p.waves == 8 && (ncb_t == 2 || (ncb_t == 0 && G_origin * S >= 2048 && kv_len >= 2048))
              ? 2
              : 1;
  const int cols = p.waves * 16 * p.ncb;
  p.nqb_origin = (G_origin * S + cols - 1) / cols;
  p.nqb_noise = (G_noise * S + cols - 1) / cols;
  const long units = (long)B * Hkv * (p.nqb_origin + p.nqb_noise);
  const int cus = device_cu_count();
  const int rows = kv_len > 0 ? kv_len : 1;
  const int tiles = (rows + kPrefillTileRowsHost - 1) / kPrefillTileRowsHost;
  int nsplit = 1;
  if (tuning().rows_per_split > 0) {
    const int rps = (int)round_up((size_t)tuning().rows_per_split, kPrefillTileRowsHost);
    nsplit = (rows + rps - 1) / rps;
  } else if (units < cus / 2) {
    // Workgroups hold one CU each (the LDS ring).  Few query blocks: as many
    // splits (tiles dealt round robin) as keep the workgroups within one
    // round, at least 4 tiles each.
    nsplit = (int)std::min<long>(std::max<long>(cus / units, 1), std::max(1, tiles / 4));
  } else {
    // Enough blocks for most CUs: split only while the workgroups fit two
    // rounds and every split keeps at least 32 tiles (each workgroup's
    // prologue, partials and the merge launch cost more than a round's idle
    // CUs on short ranges).  A 512-row chunk of 32 + 8 heads over 8 KV heads
    // at offset 3204 (160 blocks): 1 / 2 / 3 / 4 splits 158 / 180 / 141 /
    // 165 us; at offset 0: 1 / 2 splits 42 / 67 us.
    for (int k = 2; units * k <= 2L * cus && tiles / k >= 32; ++k) nsplit = k;
  }
  if (nsplit > kMaxSplits) nsplit = kMaxSplits;
  int rps = (rows + nsplit - 1) / nsplit;
  rps = (int)round_up((size_t)rps, kPrefillTileRowsHost);
  p.rows_per_split = rps;
  p.nsplit = (rows + rps - 1) / rps;
  if (p.nsplit > 1) {
    const size_t vrows = (size_t)B * Hkv * (G_origin + G_noise) * S;
    p.workspace_bytes = round_up(vrows * sizeof(unsigned), 256) +
                        round_up(vrows * p.nsplit * 2 * 128 * sizeof(float), 256) +
                        round_up(vrows * p.nsplit * 2 * sizeof(float), 256);
  }
  return p;
}

QSlabPlan plan_qslab(int B, int Hq, int Hkv, int S_q, int kv_len, int D) {
  QSlabPlan p{};
  const int G = Hkv > 0 ? Hq / Hkv : 1;
  const int GV = G * S_q;
  p.ncb = GV <= 32 ? 2 : 4;
  p.nchunk = (GV + 16 * p.ncb - 1) / (16 * p.ncb);
  p.waves = tuning().waves_per_wg == 4 ? 4 : 8;
  const int step = 32 * (p.waves / p.ncb);  // rows per step of the workgroup
  const long units = (long)B * Hkv * p.nchunk;
  const int rows = kv_len > 0 ? kv_len : 1;
  const int cus = tuning().min_wgs > 0 ? tuning().min_wgs : device_cu_count();
  int nsplit = units >= cus ? 1 : (int)((cus + units - 1) / units);
  const int max_split = (rows + step - 1) / step;  // at least one step each
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit > kMaxSplits) nsplit = kMaxSplits;
  if (nsplit < 1) nsplit = 1;
  int rps = (int)round_up((size_t)((rows + nsplit - 1) / nsplit), (size_t)step);
  if (tuning().rows_per_split > 0) rps = (int)round_up((size_t)tuning().rows_per_split, (size_t)step);
  const int min_rps = (rows + kMaxSplits - 1) / kMaxSplits;
  if (rps < min_rps) rps = (int)round_up((size_t)min_rps, (size_t)step);
  p.rows_per_split = rps;
  p.nsplit = (rows + rps - 1) / rps;
  if (p.nsplit < 1) p.nsplit = 1;
  const size_t vrows = (size_t)B * Hq * S_q;
  p.workspace_bytes = round_up(vrows * sizeof(unsigned), 256);
  if (p.nsplit > 1)
    p.workspace_bytes += round_up(vrows * p.nsplit * 2 * D * sizeof(float), 256) +
                         round_up(vrows * p.nsplit * 2 * sizeof(float), 256);
  return p;
}

}  // namespace motif

using namespace motif;

extern "C" {

int motif_abi_version(void) { return MOTIF_ABI_VERSION; }

const char* motif_last_error(void) { return g_err; }

size_t motif_sdpa_counter_bytes(int B, int Hq, int Hkv, int S_q) {
  (void)Hkv;
  if (B <= 0 || Hq <= 0 || S_q <= 0) return 0;
  return round_up((size_t)B * Hq * S_q * sizeof(unsigned), 256);
}

size_t motif_sdpa_workspace_bytes(int B, int Hq, int Hkv, int S_q, int kv_len, int D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S_q <= 0 || D <= 0 || kv_len < 0) return 0;
  CallScope scope;  // one tuning snapshot for every plan below
  // Enough for every kernel family a call may take: the fp16/bf16/fp32 and
  // VALU plans and the packed-cache matrix-core plans of each group size.
  size_t ws = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, sdpa_gc_max(D), 0, 0).workspace_bytes;
  if (D == 128 || D == 64) {  // the fp16/bf16 matrix-core kernel's plans
    const size_t w16 =
        plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, kSdpaMfmaGcMax, 0, 0).workspace_bytes;
    if (w16 > ws) ws = w16;
    if (S_q == 1 && kv_len <= kShortDecodeRows) {  // short decode calls: 4-wave plan
      const size_t w4 =
          plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, kSdpaMfmaGcMax, 4, 1).workspace_bytes;
      if (w4 > ws) ws = w4;
    }
  }
  if (D == kSdpaMfmaQD) {
    for (int gs = 32; gs <= 128; gs *= 2) {
      const int nb = sdpa_q_blocks((Hkv > 0 ? Hq / Hkv : 1) * S_q, D, gs);
      const SdpaPlan p = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, sdpa_gc_max_q(D, gs),
                                   kSdpaMfmaQWaves, kSdpaMfmaQWgsPerCu,
                                   nb > 1 ? nb * sdpa_gc_max_q(D, gs) : 0);
      if (p.workspace_bytes > ws) ws = p.workspace_bytes;
    }
    if (use_shared_tiles((Hq / Hkv) * S_q, kv_len)) {
      const PrefillPlan pp = plan_prefill(B, Hq, Hkv, S_q, kv_len, D);
      if (pp.workspace_bytes > ws) ws = pp.workspace_bytes;
    }
    const int gv = (Hq / Hkv) * S_q;
    if (gv >= kQSlabMinHeads && gv <= kQSlabMaxHeads) {
      const QSlabPlan qp = plan_qslab(B, Hq, Hkv, S_q, kv_len, D);
      if (qp.workspace_bytes > ws) ws = qp.workspace_bytes;
    }
  }
  return ws;
}

int motif_set_tuning(const char* key, int value) {
  clear_error();
  if (!key) {
    set_error("motif_set_tuning: null key");
    return MOTIF_ERR_CONTRACT;
  }
  if (value < 0) {
    set_error("motif_set_tuning: negative value %d", value);
    return MOTIF_ERR_CONTRACT;
  }
  if (!strcmp(key, "rows_per_split")) {
    update_tuning([&](Tuning& t) { t.rows_per_split = value; });
  } else if (!strcmp(key, "waves_per_wg")) {
    if (value != 0 && value != 4 && value != 8) {
      set_error("motif_set_tuning: waves_per_wg must be 0, 4 or 8");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.waves_per_wg = value; });
  } else if (!strcmp(key, "min_wgs")) {
    update_tuning([&](Tuning& t) { t.min_wgs = value; });
  } else if (!strcmp(key, "mfma")) {
    if (value != 0 && value != 1) {
      set_error("motif_set_tuning: mfma must be 0 or 1");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.mfma = value; });
  } else if (!strcmp(key, "fused_merge")) {
    if (value != 0 && value != 1) {
      set_error("motif_set_tuning: fused_merge must be 0 or 1");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.fused_merge = value; });
  } else if (!strcmp(key, "qpair")) {
    if (value < 0 || value > 2) {
      set_error("motif_set_tuning: qpair must be 0, 1 or 2");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.qpair = value; });
  } else if (!strcmp(key, "qslab")) {
    if (value < 0 || value > 2) {
      set_error("motif_set_tuning: qslab must be 0, 1 or 2");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.qslab = value; });
  } else if (!strcmp(key, "qslab_ws")) {
    if (value < 0 || value > 1) {
      set_error("motif_set_tuning: qslab_ws must be 0 or 1");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.qslab_ws = value; });
  } else if (!strcmp(key, "merge_rows")) {
    if (value < 0 || value > 1) {
      set_error("motif_set_tuning: merge_rows must be 0 or 1");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.merge_rows = value; });
  } else if (!strcmp(key, "part_f16")) {
    if (value < 0 || value > 1) {
      set_error("motif_set_tuning: part_f16 must be 0 or 1");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.part_f16 = value; });
  } else if (!strcmp(key, "qslab_sets")) {
    if (value < 2 || value > 3) {
      set_error("motif_set_tuning: qslab_sets must be 2 or 3");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.qslab_sets = value; });
  } else if (!strcmp(key, "prefill_min_heads")) {
    if (value < 0) {
      set_error("motif_set_tuning: prefill_min_heads must be >= 0");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.prefill_min_heads = value; });
  } else if (!strcmp(key, "prefill_ncb")) {
    if (value < 0 || value > 2) {
      set_error("motif_set_tuning: prefill_ncb must be 0, 1 or 2");
      return MOTIF_ERR_CONTRACT;
    }
    update_tuning([&](Tuning& t) { t.prefill_ncb = value; });
  } else if (!strcmp(key, "poly_rows")) {
    update_tuning([&](Tuning& t) { t.poly_rows = value; });
  } else {
    set_error("motif_set_tuning: unknown key '%s'", key);
    return MOTIF_ERR_CONTRACT;
  }
  return MOTIF_OK;
}

}  // extern "C"
