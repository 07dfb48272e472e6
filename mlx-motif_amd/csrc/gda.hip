// Fused GDA epilogue on gfx950 (gda_post_split / gda_post):
//   d = o - lambda * n,  y = T(d * rsqrt(mean(d^2) + eps) * w * (1 - lambda_init))
// per output row of C channels, fp32 math (src/mlx_motif/kernels/gda.py:131-192).
//
// Fast path (C % 8 == 0, 2-byte types, C <= 1024): 16 lanes per row, each
// lane holds NCH chunks of 8 channels in registers between the sum-of-squares
// pass and the store, so o and n are read from HBM once.  Other shapes use a
// strided scalar path (one wave per row) that reads its inputs twice.
#include "motif_common.hpp"

namespace motif {

struct GdaArgs {
  const void* o;  // (B, n_o_heads, S, C): rows of origin heads
  const void* n;  // (B, n_n_heads, S, C): rows of noise heads
  const void* w;  // (C)
  void* y;        // (B, q_origin, S, C)
  const float* lambda;
  long rows;      // B * q_origin * S
  int q_origin, gr, S, C;
  int o_heads;    // heads in the tensor holding origin rows
  int n_heads;    // heads in the tensor holding noise rows
  int n_head0;    // head index of noise head 0 in that tensor
  float scale, eps;
};

// Row r = (b, h_o, s) -> element offsets of its origin and noise rows.
__device__ inline void gda_rows(const GdaArgs& a, long r, long& o_off, long& n_off, long& y_off) {
  const long hs = (long)a.q_origin * a.S;
  const long b = r / hs;
  const long rem = r - b * hs;
  const int h_o = (int)(rem / a.S);
  const int s = (int)(rem - (long)h_o * a.S);
  const int h_n = a.n_head0 + h_o / a.gr;
  o_off = (((b * a.o_heads + h_o) * a.S) + s) * (long)a.C;
  n_off = (((b * a.n_heads + h_n) * a.S) + s) * (long)a.C;
  y_off = r * (long)a.C;
}

template <typename T, int NCH>
__global__ void __launch_bounds__(256) gda_vec_kernel(GdaArgs a) {
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const long r = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;  // 16 lanes per row
  const bool active = r < a.rows;
  long o_off = 0, n_off = 0, y_off = 0;
  if (active) gda_rows(a, r, o_off, n_off, y_off);
  const float lam = *a.lambda;
  const int nchunks = a.C / 8;

  float d[NCH][8];
  float ssq = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = sub + 16 * j;
    if (active && c < nchunks) {
      // o is read once (streaming); a noise row serves gr origin rows, so it
      // stays cacheable.
      uint4 ov = ld_stream4((const uint16_t*)a.o + o_off + c * 8);
      uint4 nv = *reinterpret_cast<const uint4*>((const uint16_t*)a.n + n_off + c * 8);
      uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w};
      uint32_t nw[4] = {nv.x, nv.y, nv.z, nv.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d[j][e] = Elem<T>::get(ow, e) - lam * Elem<T>::get(nw, e);
        ssq = fmaf(d[j][e], d[j][e], ssq);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) d[j][e] = 0.f;
    }
  }
  ssq = group_sum<16>(ssq);
  const float rms_inv = rsqrtf(ssq / (float)a.C + a.eps);
  if (!active) return;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = sub + 16 * j;
    if (c < nchunks) {
      uint4 wv = *reinterpret_cast<const uint4*>((const uint16_t*)a.w + c * 8);
      uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t out[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float y0 = d[j][e] * rms_inv * Elem<T>::get(ww, e) * a.scale;
        float y1 = d[j][e + 1] * rms_inv * Elem<T>::get(ww, e + 1) * a.scale;
        out[e / 2] = (uint32_t)Elem<T>::from_f32(y0) | ((uint32_t)Elem<T>::from_f32(y1) << 16);
      }
      st_stream4((uint16_t*)a.y + y_off + c * 8, out[0], out[1], out[2], out[3]);
    }
  }
}

// Any C, any element type: one wave per row, channels strided over lanes.
template <typename T>
__global__ void __launch_bounds__(256) gda_scalar_kernel(GdaArgs a) {
  const int lane = threadIdx.x & 63;
  const long r = ((long)blockIdx.x * 256 + threadIdx.x) >> 6;
  const bool active = r < a.rows;
  long o_off = 0, n_off = 0, y_off = 0;
  if (active) gda_rows(a, r, o_off, n_off, y_off);
  const float lam = *a.lambda;
  float ssq = 0.f;
  if (active) {
    for (int c = lane; c < a.C; c += 64) {
      float dv = Elem<T>::load(a.o, o_off + c) - lam * Elem<T>::load(a.n, n_off + c);
      ssq = fmaf(dv, dv, ssq);
    }
  }
  ssq = group_sum<64>(ssq);
  const float rms_inv = rsqrtf(ssq / (float)a.C + a.eps);
  if (!active) return;
  for (int c = lane; c < a.C; c += 64) {
    float dv = Elem<T>::load(a.o, o_off + c) - lam * Elem<T>::load(a.n, n_off + c);
    Elem<T>::store(a.y, y_off + c, dv * rms_inv * Elem<T>::load(a.w, c) * a.scale);
  }
}

template <typename T>
static int launch_gda(const GdaArgs& a, bool vec_ok, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    const int nch = (a.C / 8 + 15) / 16;
    if (vec_ok && a.C % 8 == 0 && nch <= 8) {
      const unsigned blocks = (unsigned)((a.rows * 16 + 255) / 256);
      switch (nch) {
        case 1: hipLaunchKernelGGL((gda_vec_kernel<T, 1>), blocks, 256, 0, st, a); break;
        case 2: hipLaunchKernelGGL((gda_vec_kernel<T, 2>), blocks, 256, 0, st, a); break;
        case 3: hipLaunchKernelGGL((gda_vec_kernel<T, 3>), blocks, 256, 0, st, a); break;
        case 4: hipLaunchKernelGGL((gda_vec_kernel<T, 4>), blocks, 256, 0, st, a); break;
        case 5: hipLaunchKernelGGL((gda_vec_kernel<T, 5>), blocks, 256, 0, st, a); break;
        case 6: hipLaunchKernelGGL((gda_vec_kernel<T, 6>), blocks, 256, 0, st, a); break;
        case 7: hipLaunchKernelGGL((gda_vec_kernel<T, 7>), blocks, 256, 0, st, a); break;
        default: hipLaunchKernelGGL((gda_vec_kernel<T, 8>), blocks, 256, 0, st, a); break;
      }
      return check_launch("gda_post_split");
    }
  }
  const unsigned blocks = (unsigned)((a.rows * 64 + 255) / 256);
  hipLaunchKernelGGL((gda_scalar_kernel<T>), blocks, 256, 0, st, a);
  return check_launch("gda_post_split");
}

static int run_gda(const char* name, GdaArgs& a, int dtype, hipStream_t st) {
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "%s: unknown dtype code %d", name, dtype);
  if (a.rows == 0 || a.C == 0) return MOTIF_OK;
  MOTIF_REQUIRE(a.o && a.n && a.w && a.y && a.lambda, "%s: null pointer", name);
  const bool vec_ok = (((uintptr_t)a.o | (uintptr_t)a.n | (uintptr_t)a.w | (uintptr_t)a.y) &
                       15u) == 0;
  switch (dtype) {
    case MOTIF_F16: return launch_gda<half_t>(a, vec_ok, st);
    case MOTIF_BF16: return launch_gda<bf16_t>(a, vec_ok, st);
    default: return launch_gda<float>(a, vec_ok, st);
  }
}

}  // namespace motif

using namespace motif;

extern "C" {

int motif_gda_post_split(const void* attn_o, const void* attn_n, const void* subln_w, void* y,
                         int dtype, int B, int q_origin, int q_groups, int gr, int S, int C,
                         const float* lambda_full, float one_minus_lambda_init, float eps,
                         void* stream) {
  CallScope scope;
  clear_error();
  MOTIF_REQUIRE(B >= 0 && q_origin >= 0 && q_groups >= 0 && gr >= 1 && S >= 0 && C >= 0,
                "gda_post_split: negative extent");
  MOTIF_REQUIRE(q_origin == q_groups * gr, "q_origin=%d != q_groups(%d) * gr(%d)", q_origin,
                q_groups, gr);
  GdaArgs a{};
  a.o = attn_o;
  a.n = attn_n;
  a.w = subln_w;
  a.y = y;
  a.lambda = lambda_full;
  a.rows = (long)B * q_origin * S;
  a.q_origin = q_origin;
  a.gr = gr;
  a.S = S;
  a.C = C;
  a.o_heads = q_origin;
  a.n_heads = q_groups;
  a.n_head0 = 0;
  a.scale = one_minus_lambda_init;
  a.eps = eps;
  return run_gda("gda_post_split", a, dtype, (hipStream_t)stream);
}

int motif_gda_post(const void* merged, const void* subln_w, void* y, int dtype, int B,
                   int q_groups, int gr, int S, int C, const float* lambda_full,
                   float one_minus_lambda_init, float eps, void* stream) {
  CallScope scope;
  clear_error();
  MOTIF_REQUIRE(B >= 0 && q_groups >= 0 && gr >= 1 && S >= 0 && C >= 0,
                "gda_post: negative extent");
  const int q_origin = q_groups * gr;
  GdaArgs a{};
  a.o = merged;
  a.n = merged;
  a.w = subln_w;
  a.y = y;
  a.lambda = lambda_full;
  a.rows = (long)B * q_origin * S;
  a.q_origin = q_origin;
  a.gr = gr;
  a.S = S;
  a.C = C;
  a.o_heads = q_origin + q_groups;
  a.n_heads = q_origin + q_groups;
  a.n_head0 = q_origin;
  a.scale = one_minus_lambda_init;
  a.eps = eps;
  return run_gda("gda_post", a, dtype, (hipStream_t)stream);
}

}  // extern "C"
