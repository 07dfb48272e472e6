// Instantiation bodies for one element type; included by sdpa_{f16,bf16,f32}.hip
// with MOTIF_ELEM and MOTIF_SUFFIX defined.
#include <type_traits>

#include "sdpa_dispatch.hpp"
#include "sdpa_impl.hpp"
#include "sdpa_mfma.hpp"
#include "sdpa_mfma_q.hpp"
#include "sdpa_prefill.hpp"

namespace motif {

#define MOTIF_CAT2(a, b) a##b
#define MOTIF_CAT(a, b) MOTIF_CAT2(a, b)

int MOTIF_CAT(dispatch_sdpa_fp_, MOTIF_SUFFIX)(const SdpaArgs& a, const SdpaPlan& p, int D,
                                              hipStream_t s) {
  const int nblocks = sdpa_grid_blocks(a.B * a.Hkv, p.nchunk, p.nsplit);
  if constexpr (std::is_same<MOTIF_ELEM, half_t>::value ||
                std::is_same<MOTIF_ELEM, bf16_t>::value) {
    if (mfma16_head_dim_ok(D, a.k) && tuning().mfma && p.gc <= kSdpaMfmaGcMax &&
        ((uintptr_t)a.q & 15u) == 0 && a.kv_len <= kMfmaMaxRows)
      return D == 128 ? launch_sdpa_mfma_16<MOTIF_ELEM, 128>(a, p.gc, p.waves, nblocks, s)
                      : launch_sdpa_mfma_16<MOTIF_ELEM, 64>(a, p.gc, p.waves, nblocks, s);
  }
  switch (D) {
    case 32: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 32>>(a, p.gc, p.waves, nblocks, s);
    case 64: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 64>>(a, p.gc, p.waves, nblocks, s);
    case 96: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 96>>(a, p.gc, p.waves, nblocks, s);
    case 128: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 128>>(a, p.gc, p.waves, nblocks, s);
    case 160: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 160>>(a, p.gc, p.waves, nblocks, s);
    case 192: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 192>>(a, p.gc, p.waves, nblocks, s);
    case 224: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 224>>(a, p.gc, p.waves, nblocks, s);
    case 256: return launch_sdpa_gc<FpFmt<MOTIF_ELEM, 256>>(a, p.gc, p.waves, nblocks, s);
    default: break;
  }
  set_error("sdpa_dual_v: head dim D=%d has no compiled variant (supported: 32..256 step 32)", D);
  return MOTIF_ERR_UNSUPPORTED;
}

int MOTIF_CAT(launch_sdpa_merge_, MOTIF_SUFFIX)(const SdpaArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_sdpa_merge_d<MOTIF_ELEM, 32>(a, s);
    case 64: return launch_sdpa_merge_d<MOTIF_ELEM, 64>(a, s);
    case 96: return launch_sdpa_merge_d<MOTIF_ELEM, 96>(a, s);
    case 128: return launch_sdpa_merge_d<MOTIF_ELEM, 128>(a, s);
    case 160: return launch_sdpa_merge_d<MOTIF_ELEM, 160>(a, s);
    case 192: return launch_sdpa_merge_d<MOTIF_ELEM, 192>(a, s);
    case 224: return launch_sdpa_merge_d<MOTIF_ELEM, 224>(a, s);
    case 256: return launch_sdpa_merge_d<MOTIF_ELEM, 256>(a, s);
    default: break;
  }
  set_error("sdpa split merge: head dim D=%d has no compiled variant", D);
  return MOTIF_ERR_UNSUPPORTED;
}

int MOTIF_CAT(dispatch_sdpa_q_, MOTIF_SUFFIX)(const SdpaArgs& a, const SdpaPlan& p, int D,
                                             int bits, hipStream_t s) {
  const int nblocks = sdpa_grid_blocks(a.B * a.Hkv, p.nchunk, p.nsplit);
  if constexpr (std::is_same<MOTIF_ELEM, half_t>::value) {
    const int ng = D / a.group_size;
    // Multi-block plan (sdpa_q_run checked the pointers and shapes for it).
    if (D == 128 && p.gc > sdpa_gc_max_q(D, a.group_size))
      return launch_sdpa_mfma_q_wide(a, bits, a.group_size, p.gc / sdpa_gc_max_q(D, a.group_size),
                                     nblocks, s);
    const uintptr_t scale_bits = (uintptr_t)a.ks | (uintptr_t)a.kb | (uintptr_t)a.v1s |
                                 (uintptr_t)a.v1b | (uintptr_t)a.v2s | (uintptr_t)a.v2b;
    const uintptr_t data_bits = (uintptr_t)a.kd | (uintptr_t)a.v1d | (uintptr_t)a.v2d;
    const bool aligned = ((data_bits | (uintptr_t)a.q) & 15u) == 0 &&
                         (scale_bits & (ng == 1 ? 7u : 15u)) == 0 && a.kv_cap % 4 == 0 &&
                         a.kv_len <= kMfmaMaxRows;
    if (D == 128 && tuning().mfma && aligned && p.gc * ng <= 16) {
      // Paired-tile kernel with qpair 2 only: for fp16 activations the
      // per-tile kernel is faster at both code widths.
      if (tuning().qpair >= 2 && ng <= 2 && tile_softmax_scale_ok(a.qscale))
        return launch_sdpa_qpair(a, bits, a.group_size, p.gc, p.waves, nblocks, s);
      return launch_sdpa_mfma_q(a, bits, a.group_size, p.gc, p.waves, nblocks, s);
    }
  }
  if constexpr (std::is_same<MOTIF_ELEM, bf16_t>::value) {
    // bf16 activations on the matrix cores (sdpa_q_run planned it: 4-wave
    // workgroups, one per CU): 4-bit caches at group size 64/128 on the
    // paired-tile kernel (faster there), the others on the per-tile kernel.
    if (mfma_q_bf16_ok(a, D, a.group_size) && p.gc * (D / a.group_size) <= 16) {
      if (qpair_bf16_ok(a, D, a.group_size, bits))
        return launch_sdpa_qpair(a, bits, a.group_size, p.gc, p.waves, nblocks, s, true);
      return launch_sdpa_mfma_q<bf16_t>(a, bits, a.group_size, p.gc, p.waves, nblocks, s);
    }
  }
  if (bits == 4) {
    switch (D) {
      case 32: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 32, 4>>(a, p.gc, p.waves, nblocks, s);
      case 64: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 64, 4>>(a, p.gc, p.waves, nblocks, s);
      case 128: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 128, 4>>(a, p.gc, p.waves, nblocks, s);
      case 256: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 256, 4>>(a, p.gc, p.waves, nblocks, s);
      default: break;
    }
  } else if (bits == 8) {
    switch (D) {
      case 32: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 32, 8>>(a, p.gc, p.waves, nblocks, s);
      case 64: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 64, 8>>(a, p.gc, p.waves, nblocks, s);
      case 128: return launch_sdpa_gc<QFmt<MOTIF_ELEM, 128, 8>>(a, p.gc, p.waves, nblocks, s);
      default: break;
    }
  }
  set_error("sdpa_dual_v_q: no compiled variant for D=%d bits=%d", D, bits);
  return MOTIF_ERR_UNSUPPORTED;
}

// Fused GDA decode step: one attention launch for the origin and noise
// passes, then the merge + gda_post_split launch.  Compiled for the fp16 and
// bf16 caches at head_dim 128 only; the entry point composes the separate
// calls otherwise.
int MOTIF_CAT(launch_gda_decode_, MOTIF_SUFFIX)(const SdpaArgs& a, int gc, int waves,
                                               int nblocks, hipStream_t s) {
  if constexpr (std::is_same<MOTIF_ELEM, half_t>::value ||
                std::is_same<MOTIF_ELEM, bf16_t>::value) {
    const int rc = launch_gda_decode_mfma_16<MOTIF_ELEM>(a, gc, waves, nblocks, s);
    if (rc != MOTIF_OK) return rc;
    return launch_gda_decode_merge_d<MOTIF_ELEM, 128>(a, s);
  }
  set_error("gda_decode: no fused variant for this element type");
  return MOTIF_ERR_UNSUPPORTED;
}

// Multi-row attention with LDS-shared K/V tiles (fp16 or bf16 cache,
// head_dim 128).
int MOTIF_CAT(launch_sdpa_prefill_, MOTIF_SUFFIX)(const SdpaArgs& a, int waves, int ncb, int nblocks,
                                                 hipStream_t s) {
  if constexpr (std::is_same<MOTIF_ELEM, half_t>::value ||
                std::is_same<MOTIF_ELEM, bf16_t>::value) {
    return launch_prefill_kernel_16<MOTIF_ELEM>(a, waves, ncb, nblocks, s);
  }
  set_error("sdpa_dual_v_rows: no shared-tile variant for this element type");
  return MOTIF_ERR_UNSUPPORTED;
}

// Prefill chunk of a GDA layer from the projections (fp16 or bf16, head_dim
// 128).
int MOTIF_CAT(launch_gda_prefill_proj_, MOTIF_SUFFIX)(const SdpaArgs& a, int waves, int ncb,
                                                     int nblocks, hipStream_t s) {
  if constexpr (std::is_same<MOTIF_ELEM, half_t>::value ||
                std::is_same<MOTIF_ELEM, bf16_t>::value) {
    return launch_gda_prefill_proj_16<MOTIF_ELEM>(a, waves, ncb, nblocks, s);
  }
  set_error("gda_prefill_proj: no variant for this element type");
  return MOTIF_ERR_UNSUPPORTED;
}

// Same over the packed q4/q8 cache (fp16 scales, head_dim 128).
int MOTIF_CAT(launch_gda_decode_q_, MOTIF_SUFFIX)(const SdpaArgs& a, int bits, int gc, int nblocks,
                                                 hipStream_t s) {
  if constexpr (!std::is_same<MOTIF_ELEM, float>::value) {  // fp16 and bf16
    const int rc = launch_gda_decode_mfma_q<MOTIF_ELEM>(a, bits, a.group_size, gc, nblocks, s);
    if (rc != MOTIF_OK) return rc;
    return launch_gda_decode_merge_d<MOTIF_ELEM, 128>(a, s);
  }
  set_error("gda_decode_q: no fused variant for this element type");
  return MOTIF_ERR_UNSUPPORTED;
}

}  // namespace motif
