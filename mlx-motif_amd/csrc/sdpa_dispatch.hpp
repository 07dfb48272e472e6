// Per-format dispatch of the split-KV attention kernel.  Each dispatch
// function is defined in its own translation unit (one per element type) so
// the variants compile in parallel.
#pragma once

#include "motif_common.hpp"
#include "sdpa_plan.hpp"

namespace motif {

// fp16 / bf16 / fp32 cache.  Returns MOTIF_ERR_UNSUPPORTED for a head dim
// with no compiled variant.
int dispatch_sdpa_fp_f16(const SdpaArgs& a, const SdpaPlan& p, int D, hipStream_t s);
int dispatch_sdpa_fp_bf16(const SdpaArgs& a, const SdpaPlan& p, int D, hipStream_t s);
int dispatch_sdpa_fp_f32(const SdpaArgs& a, const SdpaPlan& p, int D, hipStream_t s);

// Packed q4 / q8 cache with scales/biases of the given element type.
int dispatch_sdpa_q_f16(const SdpaArgs& a, const SdpaPlan& p, int D, int bits, hipStream_t s);
int dispatch_sdpa_q_bf16(const SdpaArgs& a, const SdpaPlan& p, int D, int bits, hipStream_t s);
int dispatch_sdpa_q_f32(const SdpaArgs& a, const SdpaPlan& p, int D, int bits, hipStream_t s);

// Packed cache, head_dim 128, group size 64 or 128, fp16 (or, with bf16,
// bf16) activations, scales and biases: the paired-tile matrix-core kernel
// (sdpa_qpair.hip).  gc heads per workgroup with gc * 128 / gs <= 16, waves 4
// or 8.
int launch_sdpa_qpair(const SdpaArgs& a, int bits, int gs, int gc, int waves, int nblocks,
                      hipStream_t s, bool bf16 = false);

// A bf16 call the matrix-core kernels take: head_dim 128, the pointer
// alignment and row bounds of those kernels.
bool mfma_q_bf16_ok(const SdpaArgs& a, int D, int gs);
// ... on the paired-tile kernel: group size 64 or 128, a scale its tile
// softmax handles, and qpair 1 (4-bit caches; the default) or 2 (both).
bool qpair_bf16_ok(const SdpaArgs& a, int D, int gs, int bits);

// Packed cache (fp16 scales, head dim 128), a verify slab of 17..64 virtual
// heads per KV head: tiles dequantised once per workgroup into LDS
// (sdpa_qslab.hip); ncb column blocks of 16 heads (2 or 4), 4 or 8 waves.
int launch_sdpa_qslab(const SdpaArgs& a, int bits, int gs, int ncb, int waves, int nblocks,
                      hipStream_t s);

// Split merge (second launch when a.fused_merge == 0 and nsplit > 1) for
// outputs of the given element type.
int launch_sdpa_merge_f16(const SdpaArgs& a, int D, hipStream_t s);
int launch_sdpa_merge_bf16(const SdpaArgs& a, int D, hipStream_t s);
int launch_sdpa_merge_f32(const SdpaArgs& a, int D, hipStream_t s);

// Fused GDA decode step (attention + merge/epilogue launches); the f16 and
// bf16 instances have kernels (head_dim 128), the others return
// MOTIF_ERR_UNSUPPORTED.
int launch_gda_decode_f16(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t s);
int launch_gda_decode_bf16(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t s);
int launch_gda_decode_f32(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t s);
int launch_gda_decode_q_f16(const SdpaArgs& a, int bits, int gc, int nblocks, hipStream_t s);
int launch_gda_decode_q_bf16(const SdpaArgs& a, int bits, int gc, int nblocks, hipStream_t s);
int launch_gda_decode_q_f32(const SdpaArgs& a, int bits, int gc, int nblocks, hipStream_t s);

// Multi-row attention with LDS-shared K/V tiles; the f16 and bf16 instances
// have a kernel (head_dim 128).
int launch_sdpa_prefill_f16(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);
int launch_sdpa_prefill_bf16(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);
int launch_sdpa_prefill_f32(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);

// A GDA layer's prefill chunk from the projection outputs (RoPE, the
// chunk's cache rows and both dual-V passes in one launch); f16 and bf16
// instances have a kernel (head_dim 128).
int launch_gda_prefill_proj_f16(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);
int launch_gda_prefill_proj_bf16(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);
int launch_gda_prefill_proj_f32(const SdpaArgs& a, int waves, int ncb, int nblocks, hipStream_t s);

// Pointer alignment (bytes) the kernels need for head dim D.
int sdpa_fp_align(int dtype, int D);
int sdpa_q_align(int D, int bits);

}  // namespace motif
