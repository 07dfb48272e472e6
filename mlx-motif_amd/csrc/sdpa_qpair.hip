// Paired-tile packed-cache decode kernels (sdpa_qpair.hpp).  Built on its
// own with VGPR-form MFMAs (see the Makefile): the accumulators then stay in
// arch VGPRs, and the rarely taken rescale branch costs no register copies
// on the other iterations.
#include "sdpa_dispatch.hpp"
#include "sdpa_qpair.hpp"

namespace motif {

int launch_sdpa_qpair(const SdpaArgs& a, int bits, int gs, int gc, int waves, int nblocks,
                      hipStream_t st, bool bf16) {
  if (bf16) {
    if (bits == 4) {
      if (gs == 64) return launch_sdpa_qpair_gs<4, 64, bf16_t>(a, gc, waves, nblocks, st);
      if (gs == 128) return launch_sdpa_qpair_gs<4, 128, bf16_t>(a, gc, waves, nblocks, st);
    } else {
      if (gs == 64) return launch_sdpa_qpair_gs<8, 64, bf16_t>(a, gc, waves, nblocks, st);
      if (gs == 128) return launch_sdpa_qpair_gs<8, 128, bf16_t>(a, gc, waves, nblocks, st);
    }
  } else if (bits == 4) {
    if (gs == 64) return launch_sdpa_qpair_gs<4, 64, half_t>(a, gc, waves, nblocks, st);
    if (gs == 128) return launch_sdpa_qpair_gs<4, 128, half_t>(a, gc, waves, nblocks, st);
  } else {
    if (gs == 64) return launch_sdpa_qpair_gs<8, 64, half_t>(a, gc, waves, nblocks, st);
    if (gs == 128) return launch_sdpa_qpair_gs<8, 128, half_t>(a, gc, waves, nblocks, st);
  }
  set_error("sdpa_dual_v_q: no paired MFMA variant for group size %d", gs);
  return MOTIF_ERR_UNSUPPORTED;
}

}  // namespace motif
