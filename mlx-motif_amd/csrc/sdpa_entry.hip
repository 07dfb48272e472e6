// extern "C" entry points of the dual-V attention path: contract checks,
// launch plan, workspace carving, dispatch by element type.
#include <mutex>

#include "sdpa_dispatch.hpp"

namespace motif {

int sdpa_fp_align(int dtype, int D) {
  const int bytes = dtype == MOTIF_F32 ? 4 : 2;
  const int lane_bytes = (D / 16) * bytes;
  return lane_bytes % 16 == 0 ? 16 : lane_bytes % 8 == 0 ? 8 : 4;
}

int sdpa_q_align(int D, int bits) {
  const int el = 32 / bits;
  const int cpl = (D / 16 > el) ? D / 16 : el;
  const int wpl = cpl / el;
  return wpl % 4 == 0 ? 16 : wpl % 2 == 0 ? 8 : 4;
}

static bool aligned(const void* p, int a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

// Workspace of a split call: vrows u32 arrival counters (at least
// counter_reserve bytes of them), then the partial outputs (vrows, nsplit,
// 2D) fp32, then the partial (m, l) pairs (vrows, nsplit, 2) fp32, each
// region 256-byte aligned.  counter_reserve > 0 keeps the partials of every
// call clear of a fixed counter area (the no-alloc scratch, whose counters
// are cleared once and shared by calls of any size).
static size_t split_ws_bytes(size_t vrows, int nsplit, int D, size_t counter_reserve) {
  const size_t c = round256(vrows * sizeof(unsigned));
  return (c > counter_reserve ? c : counter_reserve) +
         round256(vrows * nsplit * 2 * D * sizeof(float)) +
         round256(vrows * nsplit * 2 * sizeof(float));
}

static int carve_split_ws(const char* name, SdpaArgs& a, void* ws, size_t ws_bytes, size_t vrows,
                          int nsplit, int D, size_t counter_reserve) {
  const size_t need = split_ws_bytes(vrows, nsplit, D, counter_reserve);
  if (ws == nullptr || ws_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need,
              ws == nullptr ? (size_t)0 : ws_bytes);
    return MOTIF_ERR_WORKSPACE;
  }
  MOTIF_REQUIRE(aligned(ws, 256), "%s: workspace must be 256-byte aligned", name);
  size_t c = round256(vrows * sizeof(unsigned));
  if (c < counter_reserve) c = counter_reserve;
  char* w = (char*)ws;
  a.counters = (unsigned*)w;
  a.part_o = (float*)(w + c);
  a.part_ml = (float*)(w + c + round256(vrows * nsplit * 2 * D * sizeof(float)));
  return MOTIF_OK;
}

// Last check before a launch: a kernel that publishes split partials (every
// plan of more than one split, and the fused decode kernels always) must have
// somewhere to publish them.  A plan that fails it is a library bug; the call
// returns before any launch instead of handing a kernel a null base.
static int check_partials(const char* name, const SdpaArgs& a, bool always) {
  if (!always && a.nsplit <= 1) return MOTIF_OK;
  if (a.part_o != nullptr && a.part_ml != nullptr && (!a.fused_merge || a.counters != nullptr))
    return MOTIF_OK;
  set_error("%s: internal error: a plan of %d split(s) has no partial buffers (nothing was "
            "launched)", name, a.nsplit);
  return MOTIF_ERR_INTERNAL;
}

bool mfma_q_bf16_ok(const SdpaArgs& a, int D, int gs) {
  if (D != kSdpaMfmaQD || (gs != 32 && gs != 64 && gs != 128) || !tuning().mfma) return false;
  const int ng = D / gs;
  const uintptr_t scale_bits = (uintptr_t)a.ks | (uintptr_t)a.kb | (uintptr_t)a.v1s |
                               (uintptr_t)a.v1b | (uintptr_t)a.v2s | (uintptr_t)a.v2b;
  const uintptr_t data_bits = (uintptr_t)a.kd | (uintptr_t)a.v1d | (uintptr_t)a.v2d;
  return ((data_bits | (uintptr_t)a.q) & 15u) == 0 &&
         (scale_bits & (ng == 1 ? 7u : 15u)) == 0 && a.kv_cap % 4 == 0 &&
         a.kv_len <= kMfmaMaxRows;
}

bool qpair_bf16_ok(const SdpaArgs& a, int D, int gs, int bits) {
  return tuning().qpair >= (bits == 4 ? 1 : 2) && (gs == 64 || gs == 128) &&
         mfma_q_bf16_ok(a, D, gs) && tile_softmax_scale_ok(a.qscale);
}

// Shared shape checks (the reference asserts of attention.py:237-243, 556-564)
// and plan/workspace set-up.
static int sdpa_common(const char* name, SdpaArgs& a, SdpaPlan& p, int dtype, int B, int Hq,
                       int Hkv, int S_q, int D, int kv_cap, int kv_len, int causal, float scale,
                       void* ws, size_t ws_bytes, int gc_max, int waves_pref, int wgs_per_cu,
                       int gc_fixed = 0, size_t counter_reserve = 0) {
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "%s: unknown dtype code %d", name, dtype);
  MOTIF_REQUIRE(B >= 1 && Hq >= 1 && Hkv >= 1 && S_q >= 1, "%s: B, H_q, H_kv, S_q must be >= 1",
                name);
  MOTIF_REQUIRE(D > 0 && D % 32 == 0, "%s: D=%d must be a multiple of 32", name, D);
  MOTIF_REQUIRE(Hq % Hkv == 0, "%s: H_q=%d must be a multiple of H_kv=%d", name, Hq, Hkv);
  MOTIF_REQUIRE(kv_cap >= 0 && 0 <= kv_len && kv_len <= kv_cap,
                "%s: kv_len=%d must be in [0, %d]", name, kv_len, kv_cap);
  MOTIF_REQUIRE((long)B * Hkv * (long)kv_cap * D < (1L << 40), "%s: cache too large", name);
  p = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, gc_max, waves_pref, wgs_per_cu, gc_fixed);
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.S_q = S_q;
  a.G = Hq / Hkv;
  a.GV = a.G * S_q;
  a.nchunk = p.nchunk;
  a.kv_cap = kv_cap;
  a.kv_len = kv_len;
  a.causal = causal ? 1 : 0;
  a.nsplit = p.nsplit;
  a.rows_per_split = p.rows_per_split;
  a.fused_merge = tuning().fused_merge;
  a.qscale = scale * 1.4426950408889634f;  // log2(e): the kernels use exp2
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.counters = nullptr;
  if (p.nsplit > 1)
    return carve_split_ws(name, a, ws, ws_bytes, (size_t)B * Hq * S_q, p.nsplit, D,
                          counter_reserve);
  return MOTIF_OK;
}

// Second launch of a split call: combine the partials into y.
static int sdpa_merge(const SdpaArgs& a, int dtype, int D, hipStream_t s) {
  if (a.nsplit == 1 || a.fused_merge) return MOTIF_OK;
  switch (dtype) {
    case MOTIF_F16: return launch_sdpa_merge_f16(a, D, s);
    case MOTIF_BF16: return launch_sdpa_merge_bf16(a, D, s);
    default: return launch_sdpa_merge_f32(a, D, s);
  }
}

static int sdpa_fp_run(const char* name, const void* q, const void* k, const void* v1,
                       const void* v2, void* y, int dtype, int B, int Hq, int Hkv, int S_q, int D,
                       int kv_cap, int kv_len, int causal, float scale, void* ws,
                       size_t ws_bytes, void* stream, size_t counter_reserve = 0) {
  CallScope scope;
  clear_error();
  SdpaArgs a{};
  SdpaPlan p{};
  // The matrix-core kernel takes up to 16 virtual heads per workgroup (a
  // verify slab's 5 rows x GQA 4 in two head chunks instead of three); the
  // conditions are those under which the dispatch picks that kernel.
  const bool mfma16 = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && mfma16_head_dim_ok(D, k) &&
                      tuning().mfma && aligned(q, 16) && kv_len <= kMfmaMaxRows;
  // Short single-row calls: 4-wave workgroups, one per CU (kShortDecodeRows).
  const bool short4 = mfma16 && S_q == 1 && kv_len <= kShortDecodeRows;
  int rc = sdpa_common(name, a, p, dtype, B, Hq, Hkv, S_q, D, kv_cap, kv_len, causal, scale, ws,
                       ws_bytes, mfma16 ? kSdpaMfmaGcMax : sdpa_gc_max(D), short4 ? 4 : 0,
                       short4 ? 1 : 0, 0, counter_reserve);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(q && y && (kv_cap == 0 || (k && v1 && v2)), "%s: null tensor pointer", name);
  const int al = sdpa_fp_align(dtype, D);
  MOTIF_REQUIRE(aligned(k, al) && aligned(v1, al) && aligned(v2, al),
                "%s: k/v1/v2 must be %d-byte aligned", name, al);
  a.q = q;
  a.k = k;
  a.v1 = v1;
  a.v2 = v2;
  a.y = y;
  hipStream_t s = (hipStream_t)stream;
  // Many virtual heads per KV head (a prefill chunk or a long verify slab):
  // the kernel with LDS-shared K/V tiles reads the cache once per block of
  // up to 128 heads instead of once per 8.
  if ((dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 && tuning().mfma &&
      use_shared_tiles(a.GV, kv_len) && kv_len <= kMfmaMaxRows &&
      tile_softmax_scale_ok(a.qscale) &&
      aligned(q, 16) && aligned(y, 16) && aligned(k, 16) && aligned(v1, 16) &&
      aligned(v2, 16)) {
    const PrefillPlan pp = plan_prefill(B, Hq, Hkv, S_q, kv_len, D);
    a.nchunk = pp.nqb;
    a.nsplit = pp.nsplit;
    a.rows_per_split = pp.rows_per_split;
    // Chunks (64+ virtual heads per KV head) deal their tiles to the splits
    // round robin: the causal limit then costs every split alike (512 rows
    // over 3716: 69.9 -> 67.6-68.1 us; 2048 over 4228 201.7 -> 191.8).  Long
    // slabs keep contiguous ranges (5 rows over 32768: 37.4 against 37.9
    // round robin).
    a.tiles_rr = a.GV >= kPrefillMinHeads ? 1 : 0;
    a.fused_merge = 0;
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (pp.nsplit > 1) {
      rc = carve_split_ws(name, a, ws, ws_bytes, (size_t)B * Hq * S_q, pp.nsplit, D,
                          counter_reserve);
      if (rc != MOTIF_OK) return rc;
    }
    a.part_f16 = use_part_f16((long)B * Hq * S_q, pp.nsplit, dtype == MOTIF_F16) ? 1 : 0;
    rc = check_partials(name, a, false);
    if (rc != MOTIF_OK) return rc;
    const int nblocks = sdpa_grid_blocks(B * Hkv, pp.nqb, pp.nsplit);
    rc = dtype == MOTIF_F16 ? launch_sdpa_prefill_f16(a, pp.waves, pp.ncb, nblocks, s)
                            : launch_sdpa_prefill_bf16(a, pp.waves, pp.ncb, nblocks, s);
    return rc == MOTIF_OK ? sdpa_merge(a, dtype, D, s) : rc;
  }
  rc = check_partials(name, a, false);
  if (rc != MOTIF_OK) return rc;
  switch (dtype) {
    case MOTIF_F16: rc = dispatch_sdpa_fp_f16(a, p, D, s); break;
    case MOTIF_BF16: rc = dispatch_sdpa_fp_bf16(a, p, D, s); break;
    default: rc = dispatch_sdpa_fp_f32(a, p, D, s); break;
  }
  return rc == MOTIF_OK ? sdpa_merge(a, dtype, D, s) : rc;
}

static int sdpa_q_run(const char* name, const void* q, const uint32_t* kd, const void* ks,
                      const void* kb, const uint32_t* v1d, const void* v1s, const void* v1b,
                      const uint32_t* v2d, const void* v2s, const void* v2b, void* y, int dtype,
                      int B, int Hq, int Hkv, int S_q, int D, int kv_cap, int kv_len, int causal,
                      int bits, int gs, float scale, void* ws, size_t ws_bytes, void* stream) {
  CallScope scope;
  clear_error();
  // Packed-layout contract, attention.py:556-608.
  MOTIF_REQUIRE(bits == 4 || bits == 8, "%s: bits=%d must be 4 or 8", name, bits);
  MOTIF_REQUIRE(D > 0 && D % 32 == 0, "%s: D=%d must be a multiple of 32", name, D);
  MOTIF_REQUIRE(gs > 0 && D % gs == 0, "%s: D=%d must be a multiple of group_size=%d", name, D,
                gs);
  MOTIF_REQUIRE((32 / bits) % (D / 32) == 0,
                "%s requires qk_per_thread | EL_PER_INT so each lane's D/32 channels come from "
                "ONE packed uint32 (implies D/32 <= 32/bits); got D=%d, bits=%d",
                name, D, bits);
  MOTIF_REQUIRE(gs % (D / 32) == 0,
                "%s requires qk_per_thread | group_size; got D=%d, group_size=%d", name, D, gs);
  MOTIF_REQUIRE(gs == 32 || gs == 64 || gs == 128, "%s: group_size=%d must be 32, 64 or 128",
                name, gs);
  SdpaArgs a{};
  SdpaPlan p{};
  // The matrix-core kernel puts (head, scale group) pairs on 16 columns and
  // runs 4-wave workgroups, one per CU.  When the virtual heads of a KV head
  // fill 2-3 blocks of columns (a verify slab), one workgroup carries all of
  // them (NB column blocks), provided the pointers suit that kernel; its plan
  // has one head chunk of NB blocks.
  // bf16 activations (q4 / q8): the per-tile or the paired-tile matrix-core
  // kernel and the same plan (4-wave workgroups, one per CU), in one column
  // block.
  SdpaArgs probe{};
  probe.q = q;
  probe.kd = kd; probe.ks = ks; probe.kb = kb;
  probe.v1d = v1d; probe.v1s = v1s; probe.v1b = v1b;
  probe.v2d = v2d; probe.v2s = v2s; probe.v2b = v2b;
  probe.kv_cap = kv_cap;
  probe.kv_len = kv_len;
  probe.qscale = scale * 1.4426950408889634f;
  const bool q_bf16 = dtype == MOTIF_BF16 && mfma_q_bf16_ok(probe, D, gs);
  const bool mfma_q = D == kSdpaMfmaQD && tuning().mfma && (dtype == MOTIF_F16 || q_bf16);
  int nb = 1;
  if (mfma_q && dtype == MOTIF_F16 && Hkv >= 1 && Hq % Hkv == 0) {
    const int ng = D / gs;
    const uintptr_t scale_bits = (uintptr_t)ks | (uintptr_t)kb | (uintptr_t)v1s |
                                 (uintptr_t)v1b | (uintptr_t)v2s | (uintptr_t)v2b;
    const uintptr_t data_bits = (uintptr_t)kd | (uintptr_t)v1d | (uintptr_t)v2d;
    const bool wide_ok = ((data_bits | (uintptr_t)q) & 15u) == 0 &&
                         (scale_bits & (ng == 1 ? 7u : 15u)) == 0 && kv_cap % 4 == 0 &&
                         kv_len <= kMfmaMaxRows;
    if (wide_ok) nb = sdpa_q_blocks(Hq / Hkv * S_q, D, gs);
  }
  int rc = sdpa_common(name, a, p, dtype, B, Hq, Hkv, S_q, D, kv_cap, kv_len, causal, scale, ws,
                       ws_bytes, mfma_q ? sdpa_gc_max_q(D, gs) : sdpa_gc_max(D),
                       mfma_q ? kSdpaMfmaQWaves : 0, mfma_q ? kSdpaMfmaQWgsPerCu : 0,
                       nb > 1 ? nb * sdpa_gc_max_q(D, gs) : 0);
  if (rc != MOTIF_OK) return rc;
  if (nb > 1) a.fused_merge = 0;  // multi-block launches always merge in a second launch
  MOTIF_REQUIRE(q && y && (kv_cap == 0 || (kd && ks && kb && v1d && v1s && v1b && v2d && v2s &&
                                           v2b)),
                "%s: null tensor pointer", name);
  const int al = sdpa_q_align(D, bits);
  MOTIF_REQUIRE(aligned(kd, al) && aligned(v1d, al) && aligned(v2d, al),
                "%s: packed data must be %d-byte aligned", name, al);
  a.q = q;
  a.kd = kd; a.ks = ks; a.kb = kb;
  a.v1d = v1d; a.v1s = v1s; a.v1b = v1b;
  a.v2d = v2d; a.v2s = v2s; a.v2b = v2b;
  a.y = y;
  a.group_size = gs;
  hipStream_t s = (hipStream_t)stream;
  // A verify slab of 17..64 virtual heads per KV head: packed tiles
  // dequantised once per workgroup into LDS and shared by its waves (with
  // producer and consumer waves: 5-row slab over 32768 rows, q8 33.0 against
  // 49.0 us in head chunks, q4 35.3 against 43.6 us).
  if (dtype == MOTIF_F16 && D == 128 && tuning().mfma && tuning().qslab >= (bits == 8 ? 1 : 2) &&
      a.GV >= kQSlabMinHeads && a.GV <= kQSlabMaxHeads && kv_len <= kMfmaMaxRows &&
      tile_softmax_scale_ok(a.qscale) &&
      aligned(q, 16) && aligned(y, 16) && aligned(kd, bits == 8 ? 16 : 8) &&
      aligned(v1d, bits == 8 ? 16 : 8) && aligned(v2d, bits == 8 ? 16 : 8)) {
    const QSlabPlan qp = plan_qslab(B, Hq, Hkv, S_q, kv_len, D);
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (qp.nsplit > 1) {
      rc = carve_split_ws(name, a, ws, ws_bytes, (size_t)B * Hq * S_q, qp.nsplit, D, 0);
      if (rc != MOTIF_OK) return rc;
    }
    a.nchunk = qp.nchunk;
    a.nsplit = qp.nsplit;
    a.rows_per_split = qp.rows_per_split;
    a.fused_merge = 0;
    rc = check_partials(name, a, false);
    if (rc != MOTIF_OK) return rc;
    rc = launch_sdpa_qslab(a, bits, gs, qp.ncb, qp.waves,
                           sdpa_grid_blocks(B * Hkv, qp.nchunk, qp.nsplit), s);
    return rc == MOTIF_OK ? sdpa_merge(a, dtype, D, s) : rc;
  }
  rc = check_partials(name, a, false);
  if (rc != MOTIF_OK) return rc;
  switch (dtype) {
    case MOTIF_F16: rc = dispatch_sdpa_q_f16(a, p, D, bits, s); break;
    case MOTIF_BF16: rc = dispatch_sdpa_q_bf16(a, p, D, bits, s); break;
    default: rc = dispatch_sdpa_q_f32(a, p, D, bits, s); break;
  }
  return rc == MOTIF_OK ? sdpa_merge(a, dtype, D, s) : rc;
}

// ------------------------------------------------ fused GDA decode step ---
// Partial rows of the fused path: (b, KV head, column), G1 + G2 columns (G1
// origin and G2 noise heads per KV head; G2 = 1 in the 12.7B layout).
struct GdaDecodeLayout {
  SdpaPlan plan;    // fp16-cache kernel (8-wave workgroups)
  SdpaPlan plan_q;  // packed-cache kernel (4-wave workgroups, one per CU)
  size_t counter_bytes, o_bytes, ml_bytes, fused_bytes;
  size_t sdpa_bytes, yo_bytes, yn_bytes, composed_bytes;
};

static GdaDecodeLayout gda_decode_layout(int B, int Hkv, int G1, int G2, int kv_len, int D) {
  GdaDecodeLayout L{};
  // One virtual head per KV head in the planner: the fused kernel runs one
  // workgroup per (b, KV head, split), like the unfused origin pass; 4-wave
  // workgroups, one per CU, for short contexts (kShortDecodeRows), as the
  // single-pass call takes them.
  const bool short4 = kv_len <= kShortDecodeRows;
  L.plan = plan_sdpa(B, Hkv, Hkv, 1, kv_len, D, 1, short4 ? 4 : 0, short4 ? 1 : 0);
  L.plan_q = plan_sdpa(B, Hkv, Hkv, 1, kv_len, D, 1, kSdpaMfmaQWaves, kSdpaMfmaQWgsPerCu);
  const int ns = L.plan.nsplit > L.plan_q.nsplit ? L.plan.nsplit : L.plan_q.nsplit;
  const size_t prow = (size_t)B * Hkv * (G1 + G2);
  L.counter_bytes = round256(prow * sizeof(unsigned));
  L.o_bytes = round256(prow * ns * 2 * D * sizeof(float));
  L.ml_bytes = round256(prow * ns * 2 * sizeof(float));
  L.fused_bytes = L.counter_bytes + L.o_bytes + L.ml_bytes;
  // Composed path: both attention calls' workspace (any cache format), then
  // o and n (fp32 bound).
  const size_t w1 = motif_sdpa_workspace_bytes(B, Hkv * G1, Hkv, 1, kv_len, D);
  const size_t w2 = motif_sdpa_workspace_bytes(B, Hkv * G2, Hkv, 1, kv_len, D);
  L.sdpa_bytes = round256(w1 > w2 ? w1 : w2);
  L.yo_bytes = round256((size_t)B * Hkv * G1 * 2 * D * sizeof(float));
  L.yn_bytes = round256((size_t)B * Hkv * G2 * 2 * D * sizeof(float));
  L.composed_bytes = L.sdpa_bytes + L.yo_bytes + L.yn_bytes;
  return L;
}

// Checks shared by both fused-decode entry points; the workspace check
// covers the larger of the fused and composed layouts.
static int gda_decode_common(const char* name, const GdaDecodeLayout& L, int dtype, int B,
                             int Hkv, int G1, int G2, int D, int kv_cap, int kv_len, void* ws,
                             size_t ws_bytes) {
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "%s: unknown dtype code %d", name, dtype);
  MOTIF_REQUIRE(B >= 1 && Hkv >= 1 && G1 >= 1 && G2 >= 1 && G1 % G2 == 0,
                "%s: B, H_kv, gr must be >= 1", name);
  MOTIF_REQUIRE(D > 0 && D % 32 == 0, "%s: D=%d must be a multiple of 32", name, D);
  MOTIF_REQUIRE(kv_cap >= 0 && 0 <= kv_len && kv_len <= kv_cap,
                "%s: kv_len=%d must be in [0, %d]", name, kv_len, kv_cap);
  const size_t need = L.fused_bytes > L.composed_bytes ? L.fused_bytes : L.composed_bytes;
  if (ws == nullptr || ws_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need,
              ws == nullptr ? (size_t)0 : ws_bytes);
    return MOTIF_ERR_WORKSPACE;
  }
  MOTIF_REQUIRE(aligned(ws, 256), "%s: workspace must be 256-byte aligned", name);
  return MOTIF_OK;
}

// Arguments of a fused launch: partial rows (b, KV head, column) after the
// (unused) counter block.
static SdpaArgs gda_decode_args(const GdaDecodeLayout& L, const SdpaPlan& p, const void* q1,
                                const void* q2, void* y, int B, int Hkv, int G1, int G2,
                                int kv_cap, int kv_len, float scale, const void* subln_w,
                                const float* lambda_full, float one_minus_lambda_init,
                                float eps, void* ws) {
  SdpaArgs a{};
  a.q = q1;
  a.q2 = q2;
  a.y = y;
  a.B = B;
  a.Hkv = Hkv;
  a.Hq = Hkv * G1;
  a.S_q = 1;
  a.G = G1;
  a.G2 = G2;
  a.GV = G1 + G2;
  a.nchunk = 1;
  a.kv_cap = kv_cap;
  a.kv_len = kv_len;
  a.causal = 0;
  a.nsplit = p.nsplit;
  a.rows_per_split = p.rows_per_split;
  a.fused_merge = 0;
  a.qscale = scale * 1.4426950408889634f;
  char* w = (char*)ws;
  a.counters = (unsigned*)w;
  a.part_o = (float*)(w + L.counter_bytes);
  a.part_ml = (float*)(w + L.counter_bytes + L.o_bytes);
  a.gda_w = subln_w;
  a.gda_lambda = lambda_full;
  a.gda_scale = one_minus_lambda_init;
  a.gda_eps = eps;
  return a;
}

// Scratch of motif_sdpa_dual_v_noalloc (its split partials and counters):
// one copy per device, held until the process ends.  `scratch` names the
// host-side stand-in; kernels get the device address that
// hipGetSymbolAddress returns for the current device (scratch_for_device).
static constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
// Leading bytes cleared once per device: the merge counters (the kernels
// leave them zero after every call).
static constexpr size_t kScratchClearBytes = (size_t)64 << 10;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

__global__ void __launch_bounds__(256) scratch_clear_kernel(uint4* p, unsigned n) {
  for (unsigned i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up (and its counters
// cleared, stream-ordered before the caller's kernels) on the device's
// first call.
static int scratch_for_device(void** out, hipStream_t s) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("sdpa_dual_v_noalloc: hipGetDevice failed (%s, device %d)",
              hipGetErrorString(e), dev);
    return MOTIF_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("sdpa_dual_v_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(e));
      return MOTIF_ERR_HIP;
    }
    const unsigned n = (unsigned)(kScratchClearBytes / sizeof(uint4));
    hipLaunchKernelGGL(scratch_clear_kernel, dim3(16), dim3(256), 0, s, (uint4*)p, n);
    const int rc = check_launch("sdpa_dual_v_noalloc (scratch clear)");
    if (rc != MOTIF_OK) return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOTIF_OK;
}

// Columns of a fused launch: the n = G1 + G2 heads of a KV head, rounded up
// to a compiled width.
static int gda_columns(int n) { return n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16; }

// Origin / noise heads per KV head of a step whose q1 has Hq1 and q2 Hq2
// heads over Hkv KV heads: both passes are GQA calls of sdpa_dual_v
// (attention.py:237-243: heads a multiple of Hkv), and gda_post_split pairs
// origin head h with noise head h / gr, gr = Hq1 / Hq2 (gda.py:248).
static int gda_heads(const char* name, int Hq1, int Hq2, int Hkv, int& G1, int& G2) {
  MOTIF_REQUIRE(Hkv >= 1 && Hq2 >= 1 && Hq1 >= 1, "%s: H_q1, H_q2, H_kv must be >= 1", name);
  MOTIF_REQUIRE(Hq2 % Hkv == 0, "%s: H_q2=%d must be a multiple of H_kv=%d", name, Hq2, Hkv);
  MOTIF_REQUIRE(Hq1 % Hq2 == 0, "%s: H_q1=%d must be a multiple of H_q2=%d (q_origin == "
                "q_groups * gr)", name, Hq1, Hq2);
  G1 = Hq1 / Hkv;
  G2 = Hq2 / Hkv;
  return MOTIF_OK;
}

}  // namespace motif

using namespace motif;

extern "C" {

size_t motif_gda_decode_workspace_bytes(int B, int Hkv, int gr, int kv_len, int D) {
  if (B <= 0 || Hkv <= 0 || gr <= 0 || D <= 0 || kv_len < 0) return 0;
  CallScope scope;
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, gr, 1, kv_len, D);
  return L.fused_bytes > L.composed_bytes ? L.fused_bytes : L.composed_bytes;
}

size_t motif_gda_decode_heads_workspace_bytes(int B, int Hq1, int Hq2, int Hkv, int kv_len,
                                              int D) {
  if (B <= 0 || Hkv <= 0 || Hq1 <= 0 || Hq2 <= 0 || D <= 0 || kv_len < 0 || Hq2 % Hkv != 0 ||
      Hq1 % Hq2 != 0)
    return 0;
  CallScope scope;
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, Hq1 / Hkv, Hq2 / Hkv, kv_len, D);
  return L.fused_bytes > L.composed_bytes ? L.fused_bytes : L.composed_bytes;
}

}  // extern "C"

// The fused decode step; new_kv (k1, k2, v1, v2 rows of the new token, each
// (B, Hkv, 1, D)) or null: with it, row kv_len - 1 of the cache is written
// first (inside the attention launch when fused).
static int gda_decode_fp(const char* name, const void* q1, const void* q2, const void* k1,
                         const void* k2, const void* v1, const void* v2, const void* subln_w,
                         const float* lambda_full, float one_minus_lambda_init, float eps,
                         void* y, int dtype, int B, int Hkv, int G1, int G2, int D,
                         int kv_cap, int kv_len, float scale, void* workspace,
                         size_t workspace_bytes, const void* const* new_kv, void* stream) {
  CallScope scope;
  clear_error();
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, G1, G2, kv_len, D);
  int rc = gda_decode_common(name, L, dtype, B, Hkv, G1, G2, D, kv_cap, kv_len, workspace,
                             workspace_bytes);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(q1 && q2 && y && subln_w && lambda_full &&
                    (kv_cap == 0 || (k1 && k2 && v1 && v2)),
                "%s: null pointer", name);
  if (new_kv) {
    MOTIF_REQUIRE(new_kv[0] && new_kv[1] && new_kv[2] && new_kv[3], "%s: null new row", name);
    MOTIF_REQUIRE(kv_len >= 1, "%s: kv_len=%d must count the appended row", name, kv_len);
  }
  hipStream_t s = (hipStream_t)stream;
  const bool fused = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 &&
                     tuning().mfma && G1 + G2 <= 16 &&
                     kv_len <= kMfmaMaxRows && aligned(q1, 16) && aligned(q2, 16) &&
                     aligned(k1, 16) && aligned(k2, 16) &&
                     aligned(v1, 16) && aligned(v2, 16) && aligned(y, 8) &&
                     (!new_kv || ((uintptr_t)new_kv[0] | (uintptr_t)new_kv[1] |
                                  (uintptr_t)new_kv[2] | (uintptr_t)new_kv[3]) % 16 == 0);
  if (fused) {
    SdpaArgs a = gda_decode_args(L, L.plan, q1, q2, y, B, Hkv, G1, G2, kv_cap, kv_len, scale,
                                 subln_w, lambda_full, one_minus_lambda_init, eps, workspace);
    a.k = k1;
    a.k2 = k2;
    a.v1 = v1;
    a.v2 = v2;
    if (new_kv) {
      a.new_k1 = new_kv[0]; a.new_k2 = new_kv[1]; a.new_v1 = new_kv[2]; a.new_v2 = new_kv[3];
      a.append = 1;
    }
    const int nblocks = sdpa_grid_blocks(B * Hkv, 1, a.nsplit);
    rc = check_partials(name, a, true);
    if (rc != MOTIF_OK) return rc;
    const int waves = L.plan.waves;
    const int gc = gda_columns(G1 + G2);
    return dtype == MOTIF_F16 ? launch_gda_decode_f16(a, gc, waves, nblocks, s)
                              : launch_gda_decode_bf16(a, gc, waves, nblocks, s);
  }
  if (new_kv) {  // row kv_len - 1 of each slot: B * Hkv rows of D values
    const size_t row = (size_t)D * (dtype == MOTIF_F32 ? 4 : 2);
    const void* dst[4] = {k1, k2, v1, v2};
    for (int t = 0; t < 4; ++t) {
      const hipError_t e = hipMemcpy2DAsync(
          (char*)const_cast<void*>(dst[t]) + (size_t)(kv_len - 1) * row, (size_t)kv_cap * row,
          new_kv[t], row, row, (size_t)B * Hkv, hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) {
        set_error("%s: row copy failed: %s", name, hipGetErrorString(e));
        return MOTIF_ERR_HIP;
      }
    }
  }
  // Composition of the separate calls, every step on the device.
  char* w = (char*)workspace;
  void* yo = w + L.sdpa_bytes;
  void* yn = w + L.sdpa_bytes + L.yo_bytes;
  rc = motif_sdpa_dual_v(q1, k1, v1, v2, yo, dtype, B, Hkv * G1, Hkv, D, kv_cap, kv_len, scale,
                         workspace, L.sdpa_bytes, stream);
  if (rc != MOTIF_OK) return rc;
  rc = motif_sdpa_dual_v(q2, k2, v1, v2, yn, dtype, B, Hkv * G2, Hkv, D, kv_cap, kv_len, scale,
                         workspace, L.sdpa_bytes, stream);
  if (rc != MOTIF_OK) return rc;
  return motif_gda_post_split(yo, yn, subln_w, y, dtype, B, Hkv * G1, Hkv * G2, G1 / G2, 1,
                              2 * D, lambda_full, one_minus_lambda_init, eps, stream);
}

extern "C" {

int motif_gda_decode(const void* q1, const void* q2, const void* k1, const void* k2,
                     const void* v1, const void* v2, const void* subln_w,
                     const float* lambda_full, float one_minus_lambda_init, float eps, void* y,
                     int dtype, int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                     float scale, void* workspace, size_t workspace_bytes, void* stream) {
  return gda_decode_fp("gda_decode", q1, q2, k1, k2, v1, v2, subln_w, lambda_full,
                       one_minus_lambda_init, eps, y, dtype, B, Hkv, gr, 1, D, kv_cap, kv_len,
                       scale, workspace, workspace_bytes, nullptr, stream);
}

// New rows: all four null (no write) or all four set (the token's rows,
// written at row kv_len - 1 first, as motif_gda_decode_append does).
static int gda_new_rows(const char* name, const void* k1_new, const void* k2_new,
                        const void* v1_new, const void* v2_new, bool& append) {
  const int n = (k1_new != nullptr) + (k2_new != nullptr) + (v1_new != nullptr) +
                (v2_new != nullptr);
  MOTIF_REQUIRE(n == 0 || n == 4, "%s: new rows must be all null or all set", name);
  append = n == 4;
  return MOTIF_OK;
}

int motif_gda_decode_heads(const void* q1, const void* q2, const void* k1_new,
                           const void* k2_new, const void* v1_new, const void* v2_new, void* k1,
                           void* k2, void* v1, void* v2, const void* subln_w,
                           const float* lambda_full, float one_minus_lambda_init, float eps,
                           void* y, int dtype, int B, int Hq1, int Hq2, int Hkv, int D,
                           int kv_cap, int kv_len, float scale, void* workspace,
                           size_t workspace_bytes, void* stream) {
  CallScope scope;  // one tuning snapshot for the whole call
  clear_error();
  const char* name = "gda_decode_heads";
  int G1 = 0, G2 = 0;
  bool append = false;
  int rc = gda_heads(name, Hq1, Hq2, Hkv, G1, G2);
  if (rc == MOTIF_OK) rc = gda_new_rows(name, k1_new, k2_new, v1_new, v2_new, append);
  if (rc != MOTIF_OK) return rc;
  const void* const nk[4] = {k1_new, k2_new, v1_new, v2_new};
  return gda_decode_fp(name, q1, q2, k1, k2, v1, v2, subln_w, lambda_full,
                       one_minus_lambda_init, eps, y, dtype, B, Hkv, G1, G2, D, kv_cap, kv_len,
                       scale, workspace, workspace_bytes, append ? nk : nullptr, stream);
}

int motif_gda_decode_append(const void* q1, const void* q2, const void* k1_new,
                            const void* k2_new, const void* v1_new, const void* v2_new,
                            void* k1, void* k2, void* v1, void* v2, const void* subln_w,
                            const float* lambda_full, float one_minus_lambda_init, float eps,
                            void* y, int dtype, int B, int Hkv, int gr, int D, int kv_cap,
                            int kv_len, float scale, void* workspace, size_t workspace_bytes,
                            void* stream) {
  const void* const nk[4] = {k1_new, k2_new, v1_new, v2_new};
  return gda_decode_fp("gda_decode_append", q1, q2, k1, k2, v1, v2, subln_w, lambda_full,
                       one_minus_lambda_init, eps, y, dtype, B, Hkv, gr, 1, D, kv_cap, kv_len,
                       scale, workspace, workspace_bytes, nk, stream);
}

int motif_gda_decode_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                 void* k1, void* k2, void* v1, void* v2, const void* subln_w,
                                 const float* lambda_full, float one_minus_lambda_init,
                                 float eps, void* y, int dtype, int B, int Hkv, int gr, int D,
                                 int kv_cap, int kv_len, float scale, float theta,
                                 float position_scale, int origin_first, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  CallScope scope;
  clear_error();
  const char* name = "gda_decode_proj";
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, gr, 1, kv_len, D);
  int rc = gda_decode_common(name, L, dtype, B, Hkv, gr, 1, D, kv_cap, kv_len, workspace,
                             workspace_bytes);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(q_proj && k_proj && v_proj && k1 && k2 && v1 && v2 && y && subln_w &&
                    lambda_full,
                "%s: null pointer", name);
  MOTIF_REQUIRE(kv_len >= 1, "%s: kv_len=%d must count the new token's row", name, kv_len);
  MOTIF_REQUIRE(theta > 1.f, "%s: theta must be > 1", name);
  MOTIF_REQUIRE(position_scale > 0.f && position_scale <= 3.4028234663852886e38f,
                "%s: position_scale must be positive and finite", name);
  const bool fused = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 &&
                     tuning().mfma && gr + 1 <= 16 && kv_len <= kMfmaMaxRows &&
                     aligned(q_proj, 16) && aligned(k_proj, 16) && aligned(v_proj, 16) &&
                     aligned(k1, 16) && aligned(k2, 16) && aligned(v1, 16) && aligned(v2, 16) &&
                     aligned(y, 8);
  if (!fused) {
    set_error("%s: no fused variant for this shape (dtype %d, D=%d, gr=%d); use "
              "motif_rope_split4 and motif_gda_decode", name, dtype, D, gr);
    return MOTIF_ERR_UNSUPPORTED;
  }
  SdpaArgs a = gda_decode_args(L, L.plan, q_proj, q_proj, y, B, Hkv, gr, 1, kv_cap, kv_len,
                               scale, subln_w, lambda_full, one_minus_lambda_init, eps,
                               workspace);
  a.k = k1;
  a.k2 = k2;
  a.v1 = v1;
  a.v2 = v2;
  a.new_k1 = k_proj; a.new_k2 = k_proj; a.new_v1 = v_proj; a.new_v2 = v_proj;
  a.append = 1;
  a.from_proj = 1;
  a.q_origin_first = origin_first != 0;
  a.rope_log2_theta = log2f(theta);
  a.rope_pos_scale = position_scale;
  const int nblocks = sdpa_grid_blocks(B * Hkv, 1, a.nsplit);
  rc = check_partials(name, a, true);
  if (rc != MOTIF_OK) return rc;
  return dtype == MOTIF_F16 ? launch_gda_decode_f16(a, gda_columns(gr + 1), L.plan.waves,
                                                    nblocks, (hipStream_t)stream)
                            : launch_gda_decode_bf16(a, gda_columns(gr + 1), L.plan.waves,
                                                     nblocks, (hipStream_t)stream);
}

int motif_gda_decode_proj(const void* q_proj, const void* k_proj, const void* v_proj, void* k1,
                          void* k2, void* v1, void* v2, const void* subln_w,
                          const float* lambda_full, float one_minus_lambda_init, float eps,
                          void* y, int dtype, int B, int Hkv, int gr, int D, int kv_cap,
                          int kv_len, float scale, float theta, int origin_first,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return motif_gda_decode_proj_scaled(q_proj, k_proj, v_proj, k1, k2, v1, v2, subln_w,
                                      lambda_full, one_minus_lambda_init, eps, y, dtype, B, Hkv,
                                      gr, D, kv_cap, kv_len, scale, theta, 1.f, origin_first,
                                      workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v(const void* q, const void* k, const void* v1, const void* v2, void* y,
                      int dtype, int B, int Hq, int Hkv, int D, int kv_cap, int kv_len,
                      float scale, void* workspace, size_t workspace_bytes, void* stream) {
  return sdpa_fp_run("sdpa_dual_v", q, k, v1, v2, y, dtype, B, Hq, Hkv, 1, D, kv_cap, kv_len, 0,
                     scale, workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v_noalloc(const void* q, const void* k, const void* v1, const void* v2,
                              void* y, int dtype, int B, int Hq, int Hkv, int D, int kv_cap,
                              int kv_len, float scale, void* stream) {
  CallScope scope;
  clear_error();
  // Size first (host arithmetic only): a call that needs more than the
  // static scratch is refused before any HIP call.  The counters keep the
  // first kScratchClearBytes whatever the call's size, and the partials
  // follow them, so no call's partials land on another call's counters.
  const size_t need = motif_sdpa_workspace_bytes(B, Hq, Hkv, 1, kv_len, D);
  const size_t cbytes = motif_sdpa_counter_bytes(B, Hq, Hkv, 1);
  const size_t total = need > cbytes ? kScratchClearBytes + (need - cbytes) : kScratchClearBytes;
  if (total > kNoAllocScratchBytes || cbytes > kScratchClearBytes) {
    set_error("sdpa_dual_v_noalloc: this call needs %zu bytes of scratch (%zu bytes of "
              "counters); the static scratch holds %zu (%zu of counters): use "
              "motif_sdpa_dual_v with a workspace",
              total, cbytes, kNoAllocScratchBytes, kScratchClearBytes);
    return MOTIF_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_device(&ws, (hipStream_t)stream);
    if (rc != MOTIF_OK) return rc;
  }
  return sdpa_fp_run("sdpa_dual_v_noalloc", q, k, v1, v2, y, dtype, B, Hq, Hkv, 1, D, kv_cap,
                     kv_len, 0, scale, ws, need > 0 ? kNoAllocScratchBytes : 0, stream,
                     kScratchClearBytes);
}

int motif_sdpa_dual_v_rows(const void* q, const void* k, const void* v1, const void* v2, void* y,
                           int dtype, int B, int Hq, int Hkv, int S_q, int D, int kv_cap,
                           int kv_len, int causal, float scale, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return sdpa_fp_run("sdpa_dual_v_rows", q, k, v1, v2, y, dtype, B, Hq, Hkv, S_q, D, kv_cap,
                     kv_len, causal, scale, workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v_q(const void* q, const uint32_t* k_data, const void* k_scales,
                        const void* k_biases, const uint32_t* v1_data, const void* v1_scales,
                        const void* v1_biases, const uint32_t* v2_data, const void* v2_scales,
                        const void* v2_biases, void* y, int dtype, int B, int Hq, int Hkv, int D,
                        int kv_cap, int kv_len, int bits, int group_size, float scale,
                        void* workspace, size_t workspace_bytes, void* stream) {
  return sdpa_q_run("sdpa_dual_v_q4", q, k_data, k_scales, k_biases, v1_data, v1_scales,
                    v1_biases, v2_data, v2_scales, v2_biases, y, dtype, B, Hq, Hkv, 1, D, kv_cap,
                    kv_len, 0, bits, group_size, scale, workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v_q_rows(const void* q, const uint32_t* k_data, const void* k_scales,
                             const void* k_biases, const uint32_t* v1_data,
                             const void* v1_scales, const void* v1_biases,
                             const uint32_t* v2_data, const void* v2_scales,
                             const void* v2_biases, void* y, int dtype, int B, int Hq, int Hkv,
                             int S_q, int D, int kv_cap, int kv_len, int causal, int bits,
                             int group_size, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return sdpa_q_run("sdpa_dual_v_q_rows", q, k_data, k_scales, k_biases, v1_data, v1_scales,
                    v1_biases, v2_data, v2_scales, v2_biases, y, dtype, B, Hq, Hkv, S_q, D,
                    kv_cap, kv_len, causal, bits, group_size, scale, workspace, workspace_bytes,
                    stream);
}

int motif_sdpa_dual_v_q4(const void* q, const uint32_t* k_data, const void* k_scales,
                         const void* k_biases, const uint32_t* v1_data, const void* v1_scales,
                         const void* v1_biases, const uint32_t* v2_data, const void* v2_scales,
                         const void* v2_biases, void* y, int dtype, int B, int Hq, int Hkv, int D,
                         int kv_cap, int kv_len, int bits, int group_size, float scale,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return motif_sdpa_dual_v_q(q, k_data, k_scales, k_biases, v1_data, v1_scales, v1_biases,
                             v2_data, v2_scales, v2_biases, y, dtype, B, Hq, Hkv, D, kv_cap,
                             kv_len, bits, group_size, scale, workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v_verify(const void* q, const void* k, const void* v1, const void* v2,
                             void* y, int dtype, int B, int Hq, int Hkv, int S_q, int D,
                             int kv_cap, int kv_len, int causal, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return motif_sdpa_dual_v_rows(q, k, v1, v2, y, dtype, B, Hq, Hkv, S_q, D, kv_cap, kv_len,
                                causal, scale, workspace, workspace_bytes, stream);
}

int motif_sdpa_dual_v_q4_verify(const void* q, const uint32_t* k_data, const void* k_scales,
                                const void* k_biases, const uint32_t* v1_data,
                                const void* v1_scales, const void* v1_biases,
                                const uint32_t* v2_data, const void* v2_scales,
                                const void* v2_biases, void* y, int dtype, int B, int Hq,
                                int Hkv, int S_q, int D, int kv_cap, int kv_len, int causal,
                                int bits, int group_size, float scale, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return motif_sdpa_dual_v_q_rows(q, k_data, k_scales, k_biases, v1_data, v1_scales, v1_biases,
                                  v2_data, v2_scales, v2_biases, y, dtype, B, Hq, Hkv, S_q, D,
                                  kv_cap, kv_len, causal, bits, group_size, scale, workspace,
                                  workspace_bytes, stream);
}

}  // extern "C"

// Same over the packed cache; new_kv rows are quantised into row kv_len - 1
// (inside the attention launch when fused, else by motif_quant_write4).
static int gda_decode_q(const char* name, const void* q1, const void* q2,
                        const uint32_t* k1_data, const void* k1_scales, const void* k1_biases,
                        const uint32_t* k2_data, const void* k2_scales, const void* k2_biases,
                        const uint32_t* v1_data, const void* v1_scales, const void* v1_biases,
                        const uint32_t* v2_data, const void* v2_scales, const void* v2_biases,
                        const void* subln_w, const float* lambda_full,
                        float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                        int Hkv, int G1, int G2, int D, int kv_cap, int kv_len, int bits,
                        int group_size, float scale, void* workspace, size_t workspace_bytes,
                        const void* const* new_kv, void* stream) {
  CallScope scope;
  clear_error();
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, G1, G2, kv_len, D);
  int rc = gda_decode_common(name, L, dtype, B, Hkv, G1, G2, D, kv_cap, kv_len, workspace,
                             workspace_bytes);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(bits == 4 || bits == 8, "%s: bits=%d must be 4 or 8", name, bits);
  MOTIF_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                "%s: group_size=%d must be 32, 64 or 128", name, group_size);
  MOTIF_REQUIRE(D % group_size == 0, "%s: D=%d must be a multiple of group_size=%d", name, D,
                group_size);
  MOTIF_REQUIRE(q1 && q2 && y && subln_w && lambda_full &&
                    (kv_cap == 0 || (k1_data && k1_scales && k1_biases && k2_data &&
                                     k2_scales && k2_biases && v1_data && v1_scales &&
                                     v1_biases && v2_data && v2_scales && v2_biases)),
                "%s: null pointer", name);
  if (new_kv) {
    MOTIF_REQUIRE(new_kv[0] && new_kv[1] && new_kv[2] && new_kv[3], "%s: null new row", name);
    MOTIF_REQUIRE(kv_len >= 1, "%s: kv_len=%d must count the appended row", name, kv_len);
  }
  hipStream_t s = (hipStream_t)stream;
  const int gc = gda_columns(G1 + G2);
  const int ng = D / group_size;
  const uintptr_t data_bits = (uintptr_t)k1_data | (uintptr_t)k2_data | (uintptr_t)v1_data |
                              (uintptr_t)v2_data;
  const uintptr_t scale_bits = (uintptr_t)k1_scales | (uintptr_t)k1_biases |
                               (uintptr_t)k2_scales | (uintptr_t)k2_biases |
                               (uintptr_t)v1_scales | (uintptr_t)v1_biases |
                               (uintptr_t)v2_scales | (uintptr_t)v2_biases;
  const bool fused = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 && tuning().mfma &&
                     G1 + G2 <= 16 &&
                     gc * ng <= 16 && (data_bits & 15u) == 0 &&
                     (scale_bits & (ng == 1 ? 7u : 15u)) == 0 && kv_cap % 4 == 0 &&
                     kv_len <= kMfmaMaxRows && aligned(q1, 16) && aligned(q2, 16) &&
                     aligned(y, 8) &&
                     (!new_kv || ((uintptr_t)new_kv[0] | (uintptr_t)new_kv[1] |
                                  (uintptr_t)new_kv[2] | (uintptr_t)new_kv[3]) % 16 == 0);
  if (fused) {
    SdpaArgs a = gda_decode_args(L, L.plan_q, q1, q2, y, B, Hkv, G1, G2, kv_cap, kv_len,
                                 scale, subln_w, lambda_full, one_minus_lambda_init, eps,
                                 workspace);
    a.kd = k1_data; a.ks = k1_scales; a.kb = k1_biases;
    a.k2d = k2_data; a.k2s = k2_scales; a.k2b = k2_biases;
    a.v1d = v1_data; a.v1s = v1_scales; a.v1b = v1_biases;
    a.v2d = v2_data; a.v2s = v2_scales; a.v2b = v2_biases;
    a.group_size = group_size;
    if (new_kv) {
      a.new_k1 = new_kv[0]; a.new_k2 = new_kv[1]; a.new_v1 = new_kv[2]; a.new_v2 = new_kv[3];
      a.append = 1;
    }
    rc = check_partials(name, a, true);
    if (rc != MOTIF_OK) return rc;
    const int nblocks = sdpa_grid_blocks(B * Hkv, 1, a.nsplit);
    return dtype == MOTIF_F16 ? launch_gda_decode_q_f16(a, bits, gc, nblocks, s)
                              : launch_gda_decode_q_bf16(a, bits, gc, nblocks, s);
  }
  if (new_kv) {
    uint32_t* const data[4] = {const_cast<uint32_t*>(k1_data), const_cast<uint32_t*>(k2_data),
                               const_cast<uint32_t*>(v1_data), const_cast<uint32_t*>(v2_data)};
    void* const scl[4] = {const_cast<void*>(k1_scales), const_cast<void*>(k2_scales),
                          const_cast<void*>(v1_scales), const_cast<void*>(v2_scales)};
    void* const bia[4] = {const_cast<void*>(k1_biases), const_cast<void*>(k2_biases),
                          const_cast<void*>(v1_biases), const_cast<void*>(v2_biases)};
    rc = motif_quant_write4(new_kv[0], new_kv[1], new_kv[2], new_kv[3], data, scl, bia, dtype, B,
                            Hkv, 1, D, kv_cap, kv_len - 1, bits, group_size, stream);
    if (rc != MOTIF_OK) return rc;
  }
  char* w = (char*)workspace;
  void* yo = w + L.sdpa_bytes;
  void* yn = w + L.sdpa_bytes + L.yo_bytes;
  rc = motif_sdpa_dual_v_q(q1, k1_data, k1_scales, k1_biases, v1_data, v1_scales, v1_biases,
                           v2_data, v2_scales, v2_biases, yo, dtype, B, Hkv * G1, Hkv, D, kv_cap,
                           kv_len, bits, group_size, scale, workspace, L.sdpa_bytes, stream);
  if (rc != MOTIF_OK) return rc;
  rc = motif_sdpa_dual_v_q(q2, k2_data, k2_scales, k2_biases, v1_data, v1_scales, v1_biases,
                           v2_data, v2_scales, v2_biases, yn, dtype, B, Hkv * G2, Hkv, D, kv_cap,
                           kv_len, bits, group_size, scale, workspace, L.sdpa_bytes, stream);
  if (rc != MOTIF_OK) return rc;
  return motif_gda_post_split(yo, yn, subln_w, y, dtype, B, Hkv * G1, Hkv * G2, G1 / G2, 1,
                              2 * D, lambda_full, one_minus_lambda_init, eps, stream);
}

extern "C" {

int motif_gda_decode_q(const void* q1, const void* q2, const uint32_t* k1_data,
                       const void* k1_scales, const void* k1_biases, const uint32_t* k2_data,
                       const void* k2_scales, const void* k2_biases, const uint32_t* v1_data,
                       const void* v1_scales, const void* v1_biases, const uint32_t* v2_data,
                       const void* v2_scales, const void* v2_biases, const void* subln_w,
                       const float* lambda_full, float one_minus_lambda_init, float eps, void* y,
                       int dtype, int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                       int bits, int group_size, float scale, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return gda_decode_q("gda_decode_q", q1, q2, k1_data, k1_scales, k1_biases, k2_data, k2_scales,
                      k2_biases, v1_data, v1_scales, v1_biases, v2_data, v2_scales, v2_biases,
                      subln_w, lambda_full, one_minus_lambda_init, eps, y, dtype, B, Hkv, gr, 1,
                      D, kv_cap, kv_len, bits, group_size, scale, workspace, workspace_bytes,
                      nullptr, stream);
}

int motif_gda_decode_q_heads(const void* q1, const void* q2, const void* k1_new,
                             const void* k2_new, const void* v1_new, const void* v2_new,
                             uint32_t* k1_data, void* k1_scales, void* k1_biases,
                             uint32_t* k2_data, void* k2_scales, void* k2_biases,
                             uint32_t* v1_data, void* v1_scales, void* v1_biases,
                             uint32_t* v2_data, void* v2_scales, void* v2_biases,
                             const void* subln_w, const float* lambda_full,
                             float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                             int Hq1, int Hq2, int Hkv, int D, int kv_cap, int kv_len, int bits,
                             int group_size, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
  CallScope scope;  // one tuning snapshot for the whole call
  clear_error();
  const char* name = "gda_decode_q_heads";
  int G1 = 0, G2 = 0;
  bool append = false;
  int rc = gda_heads(name, Hq1, Hq2, Hkv, G1, G2);
  if (rc == MOTIF_OK) rc = gda_new_rows(name, k1_new, k2_new, v1_new, v2_new, append);
  if (rc != MOTIF_OK) return rc;
  const void* const nk[4] = {k1_new, k2_new, v1_new, v2_new};
  return gda_decode_q(name, q1, q2, k1_data, k1_scales, k1_biases, k2_data, k2_scales,
                      k2_biases, v1_data, v1_scales, v1_biases, v2_data, v2_scales, v2_biases,
                      subln_w, lambda_full, one_minus_lambda_init, eps, y, dtype, B, Hkv, G1, G2,
                      D, kv_cap, kv_len, bits, group_size, scale, workspace, workspace_bytes,
                      append ? nk : nullptr, stream);
}

int motif_gda_decode_q_append(const void* q1, const void* q2, const void* k1_new,
                              const void* k2_new, const void* v1_new, const void* v2_new,
                              uint32_t* k1_data, void* k1_scales, void* k1_biases,
                              uint32_t* k2_data, void* k2_scales, void* k2_biases,
                              uint32_t* v1_data, void* v1_scales, void* v1_biases,
                              uint32_t* v2_data, void* v2_scales, void* v2_biases,
                              const void* subln_w, const float* lambda_full,
                              float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                              int Hkv, int gr, int D, int kv_cap, int kv_len, int bits,
                              int group_size, float scale, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const void* const nk[4] = {k1_new, k2_new, v1_new, v2_new};
  return gda_decode_q("gda_decode_q_append", q1, q2, k1_data, k1_scales, k1_biases, k2_data,
                      k2_scales, k2_biases, v1_data, v1_scales, v1_biases, v2_data, v2_scales,
                      v2_biases, subln_w, lambda_full, one_minus_lambda_init, eps, y, dtype, B,
                      Hkv, gr, 1, D, kv_cap, kv_len, bits, group_size, scale, workspace,
                      workspace_bytes, nk, stream);
}

int motif_gda_decode_q_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                   uint32_t* k1_data, void* k1_scales, void* k1_biases,
                                   uint32_t* k2_data, void* k2_scales, void* k2_biases,
                                   uint32_t* v1_data, void* v1_scales, void* v1_biases,
                                   uint32_t* v2_data, void* v2_scales, void* v2_biases,
                                   const void* subln_w, const float* lambda_full,
                                   float one_minus_lambda_init, float eps, void* y, int dtype,
                                   int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                                   int bits, int group_size, float scale, float theta,
                                   float position_scale, int origin_first, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  CallScope scope;
  clear_error();
  const char* name = "gda_decode_q_proj";
  const GdaDecodeLayout L = gda_decode_layout(B, Hkv, gr, 1, kv_len, D);
  int rc = gda_decode_common(name, L, dtype, B, Hkv, gr, 1, D, kv_cap, kv_len, workspace,
                             workspace_bytes);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(bits == 4 || bits == 8, "%s: bits=%d must be 4 or 8", name, bits);
  MOTIF_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                "%s: group_size=%d must be 32, 64 or 128", name, group_size);
  MOTIF_REQUIRE(q_proj && k_proj && v_proj && y && subln_w && lambda_full && k1_data &&
                    k1_scales && k1_biases && k2_data && k2_scales && k2_biases && v1_data &&
                    v1_scales && v1_biases && v2_data && v2_scales && v2_biases,
                "%s: null pointer", name);
  MOTIF_REQUIRE(kv_len >= 1, "%s: kv_len=%d must count the new token's row", name, kv_len);
  MOTIF_REQUIRE(theta > 1.f, "%s: theta must be > 1", name);
  MOTIF_REQUIRE(position_scale > 0.f && position_scale <= 3.4028234663852886e38f,
                "%s: position_scale must be positive and finite", name);
  const int gc = gda_columns(gr + 1);
  const int ng = D > 0 ? D / group_size : 1;
  const uintptr_t data_bits = (uintptr_t)k1_data | (uintptr_t)k2_data | (uintptr_t)v1_data |
                              (uintptr_t)v2_data;
  const uintptr_t scale_bits = (uintptr_t)k1_scales | (uintptr_t)k1_biases |
                               (uintptr_t)k2_scales | (uintptr_t)k2_biases |
                               (uintptr_t)v1_scales | (uintptr_t)v1_biases |
                               (uintptr_t)v2_scales | (uintptr_t)v2_biases;
  const bool fused = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 && tuning().mfma &&
                     gr + 1 <= 16 &&
                     gc * ng <= 16 && (data_bits & 15u) == 0 &&
                     (scale_bits & (ng == 1 ? 7u : 15u)) == 0 && kv_cap % 4 == 0 &&
                     kv_len <= kMfmaMaxRows && aligned(q_proj, 16) && aligned(k_proj, 16) &&
                     aligned(v_proj, 16) && aligned(y, 8);
  if (!fused) {
    set_error("%s: no fused variant for this shape (dtype %d, D=%d, gr=%d, group_size=%d); use "
              "motif_rope_split4 and motif_gda_decode_q_append", name, dtype, D, gr, group_size);
    return MOTIF_ERR_UNSUPPORTED;
  }
  SdpaArgs a = gda_decode_args(L, L.plan_q, q_proj, q_proj, y, B, Hkv, gr, 1, kv_cap, kv_len,
                               scale, subln_w, lambda_full, one_minus_lambda_init, eps,
                               workspace);
  a.kd = k1_data; a.ks = k1_scales; a.kb = k1_biases;
  a.k2d = k2_data; a.k2s = k2_scales; a.k2b = k2_biases;
  a.v1d = v1_data; a.v1s = v1_scales; a.v1b = v1_biases;
  a.v2d = v2_data; a.v2s = v2_scales; a.v2b = v2_biases;
  a.group_size = group_size;
  a.new_k1 = k_proj; a.new_k2 = k_proj; a.new_v1 = v_proj; a.new_v2 = v_proj;
  a.append = 1;
  a.from_proj = 1;
  a.q_origin_first = origin_first != 0;
  a.rope_log2_theta = log2f(theta);
  a.rope_pos_scale = position_scale;
  rc = check_partials(name, a, true);
  if (rc != MOTIF_OK) return rc;
  const int nblocks = sdpa_grid_blocks(B * Hkv, 1, a.nsplit);
  return dtype == MOTIF_F16 ? launch_gda_decode_q_f16(a, bits, gc, nblocks, (hipStream_t)stream)
                            : launch_gda_decode_q_bf16(a, bits, gc, nblocks, (hipStream_t)stream);
}

int motif_gda_decode_q_proj(const void* q_proj, const void* k_proj, const void* v_proj,
                            uint32_t* k1_data, void* k1_scales, void* k1_biases,
                            uint32_t* k2_data, void* k2_scales, void* k2_biases,
                            uint32_t* v1_data, void* v1_scales, void* v1_biases,
                            uint32_t* v2_data, void* v2_scales, void* v2_biases,
                            const void* subln_w, const float* lambda_full,
                            float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                            int Hkv, int gr, int D, int kv_cap, int kv_len, int bits,
                            int group_size, float scale, float theta, int origin_first,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return motif_gda_decode_q_proj_scaled(
      q_proj, k_proj, v_proj, k1_data, k1_scales, k1_biases, k2_data, k2_scales, k2_biases,
      v1_data, v1_scales, v1_biases, v2_data, v2_scales, v2_biases, subln_w, lambda_full,
      one_minus_lambda_init, eps, y, dtype, B, Hkv, gr, D, kv_cap, kv_len, bits, group_size,
      scale, theta, 1.f, origin_first, workspace, workspace_bytes, stream);
}

}  // extern "C"

// ------------------------------------------ GDA prefill chunk from projections ---
extern "C" {

size_t motif_gda_prefill_workspace_bytes(int B, int S, int q_groups, int gr, int k_groups,
                                         int D, int kv_len) {
  if (B < 1 || S < 1 || q_groups < 1 || gr < 1 || k_groups < 1 || q_groups % k_groups != 0 ||
      D != 128 || kv_len < S)
    return 0;
  CallScope scope;
  const int G_o = q_groups * gr / k_groups, G_n = q_groups / k_groups;
  return plan_gda_prefill(B, k_groups, G_o, G_n, S, kv_len).workspace_bytes;
}

int motif_gda_prefill_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                  void* k1, void* k2, void* v1, void* v2, void* y_origin,
                                  void* y_noise, int dtype, int B, int S, int q_groups, int gr,
                                  int k_groups, int D, int kv_cap, int offset, float scale,
                                  float theta, float position_scale, int origin_first,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  CallScope scope;
  clear_error();
  const char* name = "gda_prefill_proj";
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "%s: unknown dtype code %d", name, dtype);
  MOTIF_REQUIRE(B >= 1 && S >= 1, "%s: B and S must be >= 1", name);
  MOTIF_REQUIRE(q_groups >= 1 && gr >= 1 && k_groups >= 1,
                "%s: q_groups, gr and k_groups must be >= 1", name);
  MOTIF_REQUIRE(q_groups % k_groups == 0, "%s: q_groups=%d must be a multiple of k_groups=%d",
                name, q_groups, k_groups);
  MOTIF_REQUIRE(D > 0 && D % 32 == 0, "%s: D=%d must be a multiple of 32", name, D);
  MOTIF_REQUIRE(offset >= 0 && (long)offset + S <= kv_cap,
                "%s: rows [%d, %d) must fit the cache capacity %d", name, offset, offset + S,
                kv_cap);
  MOTIF_REQUIRE(theta > 1.f, "%s: theta must be > 1", name);
  MOTIF_REQUIRE(position_scale > 0.f && position_scale <= 3.4028234663852886e38f,
                "%s: position_scale must be positive and finite", name);
  MOTIF_REQUIRE((long)B * k_groups * (long)kv_cap * D < (1L << 40), "%s: cache too large", name);
  MOTIF_REQUIRE(q_proj && k_proj && v_proj && k1 && k2 && v1 && v2 && y_origin && y_noise,
                "%s: null pointer", name);
  // kv_len <= kMfmaMaxRows: the kernel's byte offsets into a KV head's rows
  // are 32-bit, as in the other matrix-core entry points.
  const bool ok = (dtype == MOTIF_F16 || dtype == MOTIF_BF16) && D == 128 && tuning().mfma &&
                  (long)offset + S <= kMfmaMaxRows &&
                  tile_softmax_scale_ok(scale * 1.4426950408889634f) &&
                  (long)S * 2 * k_groups * D * 2 < (1L << 31) && aligned(q_proj, 16) &&
                  aligned(k_proj, 16) && aligned(v_proj, 16) && aligned(k1, 16) &&
                  aligned(k2, 16) && aligned(v1, 16) && aligned(v2, 16) && aligned(y_origin, 16) &&
                  aligned(y_noise, 16);
  if (!ok) {
    set_error("%s: no fused variant for this call (dtype %d, D=%d, %d rows, scale %g); use "
              "motif_rope_split4 and motif_sdpa_dual_v_rows", name, dtype, D, offset + S,
              (double)scale);
    return MOTIF_ERR_UNSUPPORTED;
  }
  const int kv_len = offset + S;
  const int Hq_o = q_groups * gr;
  const int G_o = Hq_o / k_groups, G_n = q_groups / k_groups;
  const GdaPrefillPlan pp = plan_gda_prefill(B, k_groups, G_o, G_n, S, kv_len);
  SdpaArgs a{};
  a.q = q_proj;
  a.k = k1; a.k2 = k2; a.v1 = v1; a.v2 = v2;
  a.new_k1 = k_proj; a.new_v1 = v_proj;
  a.y = y_origin;
  a.y2 = y_noise;
  a.B = B; a.Hq = Hq_o; a.Hkv = k_groups; a.S_q = S;
  a.G = G_o; a.G2 = G_n; a.GV = G_o * S;
  a.nchunk = pp.nqb_origin + pp.nqb_noise;
  a.nqb_origin = pp.nqb_origin;
  a.kv_cap = kv_cap; a.kv_len = kv_len; a.causal = 1;
  a.nsplit = pp.nsplit; a.rows_per_split = pp.rows_per_split;
  a.fused_merge = 0;
  a.qscale = scale * 1.4426950408889634f;
  a.q_groups = q_groups; a.q_gr = gr; a.q_origin_first = origin_first != 0;
  a.rope_log2_theta = log2f(theta);
  a.rope_pos_scale = position_scale;
  a.rope_pos0 = offset;
  a.y2_row0 = (long)B * Hq_o * S;
  if (pp.nsplit > 1) {
    const int rc = carve_split_ws(name, a, workspace, workspace_bytes,
                                  (size_t)B * (Hq_o + q_groups) * S, pp.nsplit, D, 0);
    if (rc != MOTIF_OK) return rc;
  }
  a.part_f16 =
      use_part_f16((long)B * (Hq_o + q_groups) * S, pp.nsplit, dtype == MOTIF_F16) ? 1 : 0;
  int rc = check_partials(name, a, false);
  if (rc != MOTIF_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int nblocks = sdpa_grid_blocks(B * k_groups, a.nchunk, pp.nsplit);
  rc = dtype == MOTIF_F16 ? launch_gda_prefill_proj_f16(a, pp.waves, pp.ncb, nblocks, s)
                              : launch_gda_prefill_proj_bf16(a, pp.waves, pp.ncb, nblocks, s);
  if (rc != MOTIF_OK || pp.nsplit == 1) return rc;
  // One merge over both passes' partial rows (noise rows into y_noise).
  SdpaArgs m = a;
  m.Hq = Hq_o + q_groups;
  return sdpa_merge(m, dtype, D, s);
}

int motif_gda_prefill_proj(const void* q_proj, const void* k_proj, const void* v_proj, void* k1,
                           void* k2, void* v1, void* v2, void* y_origin, void* y_noise, int dtype,
                           int B, int S, int q_groups, int gr, int k_groups, int D, int kv_cap,
                           int offset, float scale, float theta, int origin_first,
                           void* workspace, size_t workspace_bytes, void* stream) {
  return motif_gda_prefill_proj_scaled(q_proj, k_proj, v_proj, k1, k2, v1, v2, y_origin, y_noise,
                                       dtype, B, S, q_groups, gr, k_groups, D, kv_cap, offset,
                                       scale, theta, 1.f, origin_first, workspace,
                                       workspace_bytes, stream);
}

// Host-only walk of every launch planner over decode, slab and prefill
// shapes (no HIP call): each plan of more than one split must have a
// workspace that holds its counters and partials, carving it must give the
// kernels non-null partial buffers inside it (check_partials passes), a
// missing workspace must be refused, and the public size query must cover
// the plans of the routes it serves.  The no-alloc layout must keep every
// call's partials past its fixed counter area.  Returns MOTIF_OK or
// MOTIF_ERR_INTERNAL with the failing plan in motif_last_error().
int motif_plan_selfcheck(void) {
  CallScope scope;
  clear_error();
  char* const fake = (char*)(uintptr_t)0x10000000u;  // never dereferenced
  auto fail = [](const char* what, int B, int Hq, int Hkv, int S_q, int kv_len, int ns) {
    set_error("plan_selfcheck: %s (B=%d Hq=%d Hkv=%d S_q=%d kv_len=%d nsplit=%d)", what, B, Hq,
              Hkv, S_q, kv_len, ns);
    return MOTIF_ERR_INTERNAL;
  };
  // One plan: nsplit in range; split plans carve cleanly and are guarded.
  auto check_plan = [&](const char* what, size_t vrows, int nsplit, size_t ws_bytes, int B,
                        int Hq, int Hkv, int S_q, int kv_len, size_t reserve) -> int {
    if (nsplit < 1 || nsplit > kMaxSplits) return fail(what, B, Hq, Hkv, S_q, kv_len, nsplit);
    SdpaArgs a{};
    a.nsplit = nsplit;
    if (nsplit == 1) return MOTIF_OK;
    const size_t need = split_ws_bytes(vrows, nsplit, 128, reserve);
    if (reserve == 0 && ws_bytes < need) return fail(what, B, Hq, Hkv, S_q, kv_len, nsplit);
    if (carve_split_ws(what, a, nullptr, 0, vrows, nsplit, 128, reserve) != MOTIF_ERR_WORKSPACE)
      return fail("missing workspace accepted", B, Hq, Hkv, S_q, kv_len, nsplit);
    if (carve_split_ws(what, a, fake, need, vrows, nsplit, 128, reserve) != MOTIF_OK ||
        check_partials(what, a, false) != MOTIF_OK)
      return fail(what, B, Hq, Hkv, S_q, kv_len, nsplit);
    const char* o = (const char*)a.part_o;
    const char* ml = (const char*)a.part_ml;
    const size_t o_end = (size_t)(o - fake) + vrows * nsplit * 2 * 128 * sizeof(float);
    const size_t ml_end = (size_t)(ml - fake) + vrows * nsplit * 2 * sizeof(float);
    if ((size_t)(o - fake) < vrows * sizeof(unsigned) || (size_t)(o - fake) < reserve ||
        o_end > (size_t)(ml - fake) || ml_end > need)
      return fail(what, B, Hq, Hkv, S_q, kv_len, nsplit);
    clear_error();
    return MOTIF_OK;
  };
  // The guard itself refuses split plans without partial buffers.
  {
    SdpaArgs a{};
    a.nsplit = 2;
    if (check_partials("selfcheck", a, false) != MOTIF_ERR_INTERNAL)
      return fail("guard let a split plan without partials through", 0, 0, 0, 0, 0, 2);
    a.nsplit = 1;
    if (check_partials("selfcheck", a, true) != MOTIF_ERR_INTERNAL)
      return fail("guard let a fused plan without partials through", 0, 0, 0, 0, 0, 1);
    clear_error();
  }
  const int heads[][2] = {{32, 8}, {40, 8}, {8, 8}, {4, 4}, {16, 4}, {64, 8}, {128, 8}};
  const int rows_q[] = {1, 2, 5, 17, 37, 128, 512};
  const int lens[] = {0, 1, 15, 16, 17, 300, 1024, 2047, 2048, 3204, 4096, 4097, 16000, 32768,
                      131072};
  constexpr int D = 128;
  for (int B = 1; B <= 2; ++B)
    for (const auto& h : heads)
      for (int S_q : rows_q)
        for (int kv_len : lens) {
          const int Hq = h[0], Hkv = h[1];
          if (kv_len < S_q && S_q > 1) continue;
          const size_t vrows = (size_t)B * Hq * S_q;
          const size_t pub = motif_sdpa_workspace_bytes(B, Hq, Hkv, S_q, kv_len, D);
          int rc;
          // fp kernels (VALU, 16-column matrix-core, short 4-wave decode)
          const SdpaPlan p0 = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, sdpa_gc_max(D), 0, 0);
          const SdpaPlan p1 = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, kSdpaMfmaGcMax, 0, 0);
          const SdpaPlan p2 = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, kSdpaMfmaGcMax, 4, 1);
          for (const SdpaPlan* p : {&p0, &p1, &p2}) {
            if (pub < p->workspace_bytes && (p != &p2 || (S_q == 1 && kv_len <= kShortDecodeRows)))
              return fail("size query below an fp plan", B, Hq, Hkv, S_q, kv_len, p->nsplit);
            if ((rc = check_plan("fp plan", vrows, p->nsplit, p->workspace_bytes, B, Hq, Hkv, S_q,
                                 kv_len, 0)) != MOTIF_OK)
              return rc;
          }
          if (S_q == 1 &&
              (rc = check_plan("no-alloc plan", vrows, p1.nsplit, 0, B, Hq, Hkv, S_q, kv_len,
                               kScratchClearBytes)) != MOTIF_OK)
            return rc;
          // packed-cache matrix-core kernels, every group size
          for (int gs = 32; gs <= 128; gs *= 2) {
            const int nb = sdpa_q_blocks(Hq / Hkv * S_q, D, gs);
            const SdpaPlan pq = plan_sdpa(B, Hq, Hkv, S_q, kv_len, D, sdpa_gc_max_q(D, gs),
                                          kSdpaMfmaQWaves, kSdpaMfmaQWgsPerCu,
                                          nb > 1 ? nb * sdpa_gc_max_q(D, gs) : 0);
            if (pub < pq.workspace_bytes)
              return fail("size query below a packed plan", B, Hq, Hkv, S_q, kv_len, pq.nsplit);
            if ((rc = check_plan("packed plan", vrows, pq.nsplit, pq.workspace_bytes, B, Hq, Hkv,
                                 S_q, kv_len, 0)) != MOTIF_OK)
              return rc;
          }
          // shared-tile kernel (prefill chunks, long slabs)
          if (use_shared_tiles(Hq / Hkv * S_q, kv_len)) {
            const PrefillPlan pp = plan_prefill(B, Hq, Hkv, S_q, kv_len, D);
            if (pub < pp.workspace_bytes)
              return fail("size query below a shared-tile plan", B, Hq, Hkv, S_q, kv_len,
                          pp.nsplit);
            if ((rc = check_plan("shared-tile plan", vrows, pp.nsplit, pp.workspace_bytes, B, Hq,
                                 Hkv, S_q, kv_len, 0)) != MOTIF_OK)
              return rc;
          }
          // packed slab kernel
          const int gv = Hq / Hkv * S_q;
          if (gv >= kQSlabMinHeads && gv <= kQSlabMaxHeads) {
            const QSlabPlan qp = plan_qslab(B, Hq, Hkv, S_q, kv_len, D);
            if (pub < qp.workspace_bytes)
              return fail("size query below a slab plan", B, Hq, Hkv, S_q, kv_len, qp.nsplit);
            if ((rc = check_plan("slab plan", vrows, qp.nsplit, qp.workspace_bytes, B, Hq, Hkv,
                                 S_q, kv_len, 0)) != MOTIF_OK)
              return rc;
          }
          // a GDA layer's prefill chunk from the projections (gr = G / 4)
          if (S_q > 1 && Hq / Hkv >= 2) {
            const int gr = Hq / Hkv >= 4 ? 4 : 2, q_groups = Hq / gr;
            if (q_groups % Hkv == 0) {
              const int G_o = q_groups * gr / Hkv, G_n = q_groups / Hkv;
              const GdaPrefillPlan gp = plan_gda_prefill(B, Hkv, G_o, G_n, S_q, kv_len);
              const size_t gv_rows = (size_t)B * (q_groups * gr + q_groups) * S_q;
              if ((rc = check_plan("gda prefill plan", gv_rows, gp.nsplit, gp.workspace_bytes, B,
                                   Hq, Hkv, S_q, kv_len, 0)) != MOTIF_OK)
                return rc;
            }
          }
          // the fused decode step: partials are always published
          if (S_q == 1 && Hq / Hkv >= 2) {
            const int gr = Hq / Hkv - 1 > 0 ? Hq / Hkv - 1 : 1;
            const GdaDecodeLayout L = gda_decode_layout(B, Hkv, gr, 1, kv_len, D);
            const size_t prow = (size_t)B * Hkv * (gr + 1);
            for (const SdpaPlan* p : {&L.plan, &L.plan_q}) {
              if (p->nsplit < 1 || p->nsplit > kMaxSplits ||
                  L.o_bytes < prow * p->nsplit * 2 * D * sizeof(float) ||
                  L.ml_bytes < prow * p->nsplit * 2 * sizeof(float) ||
                  L.fused_bytes != L.counter_bytes + L.o_bytes + L.ml_bytes)
                return fail("fused decode layout", B, Hq, Hkv, S_q, kv_len, p->nsplit);
            }
          }
        }
  clear_error();
  return MOTIF_OK;
}

}  // extern "C"
