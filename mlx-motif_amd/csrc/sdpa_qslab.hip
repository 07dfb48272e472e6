// Packed-cache verify-slab kernels (sdpa_qslab.hpp): tiles dequantised once
// per workgroup into LDS and shared by its waves.
#include "sdpa_dispatch.hpp"
#include "sdpa_qslab.hpp"

namespace motif {

template <int BITS, int GS, int NCB>
static void launch_qslab_ws(const SdpaArgs& a, int sets, int nblocks, hipStream_t st) {
  if (sets == 3)
    hipLaunchKernelGGL((sdpa_qslab_ws_kernel<BITS, GS, NCB, 3>), dim3(nblocks), dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((sdpa_qslab_ws_kernel<BITS, GS, NCB, 2>), dim3(nblocks), dim3(512), 0, st, a);
}

template <int BITS, int GS>
static int launch_qslab_gs(const SdpaArgs& a, int ncb, int waves, int nblocks, hipStream_t st) {
  // 8 waves: producer / consumer roles (dequantisation beside the attention)
  if (waves == 8 && tuning().qslab_ws) {
    const int sets = tuning().qslab_sets;
    if (ncb == 2)
      launch_qslab_ws<BITS, GS, 2>(a, sets, nblocks, st);
    else
      launch_qslab_ws<BITS, GS, 4>(a, sets, nblocks, st);
    return check_launch("sdpa_dual_v_q (slab, producer/consumer)");
  }
  if (ncb == 2 && waves == 8)
    hipLaunchKernelGGL((sdpa_qslab_kernel<BITS, GS, 2, 8>), dim3(nblocks), dim3(512), 0, st, a);
  else if (ncb == 4 && waves == 8)
    hipLaunchKernelGGL((sdpa_qslab_kernel<BITS, GS, 4, 8>), dim3(nblocks), dim3(512), 0, st, a);
  else if (ncb == 2 && waves == 4)
    hipLaunchKernelGGL((sdpa_qslab_kernel<BITS, GS, 2, 4>), dim3(nblocks), dim3(256), 0, st, a);
  else if (ncb == 4 && waves == 4)
    hipLaunchKernelGGL((sdpa_qslab_kernel<BITS, GS, 4, 4>), dim3(nblocks), dim3(256), 0, st, a);
  else {
    set_error("sdpa_dual_v_q: no slab variant with %d column blocks and %d waves", ncb, waves);
    return MOTIF_ERR_UNSUPPORTED;
  }
  return check_launch("sdpa_dual_v_q (slab)");
}

int launch_sdpa_qslab(const SdpaArgs& a, int bits, int gs, int ncb, int waves, int nblocks,
                      hipStream_t st) {
  if (bits == 4) {
    if (gs == 32) return launch_qslab_gs<4, 32>(a, ncb, waves, nblocks, st);
    if (gs == 64) return launch_qslab_gs<4, 64>(a, ncb, waves, nblocks, st);
    if (gs == 128) return launch_qslab_gs<4, 128>(a, ncb, waves, nblocks, st);
  } else {
    if (gs == 32) return launch_qslab_gs<8, 32>(a, ncb, waves, nblocks, st);
    if (gs == 64) return launch_qslab_gs<8, 64>(a, ncb, waves, nblocks, st);
    if (gs == 128) return launch_qslab_gs<8, 128>(a, ncb, waves, nblocks, st);
  }
  set_error("sdpa_dual_v_q: no slab variant for group size %d", gs);
  return MOTIF_ERR_UNSUPPORTED;
}

}  // namespace motif
