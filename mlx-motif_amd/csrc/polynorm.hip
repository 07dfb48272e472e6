// Fused PolyNorm on gfx950 (src/mlx_motif/kernels/mlp.py:21-93):
//   rs_k = rsqrt(mean(x^(2k)) + eps), k = 1..3
//   y    = T(w0*(x^3*rs3) + w1*(x^2*rs2) + w2*(x*rs1) + b), fp32 math.
// The reference kernel reads each row twice (sums, then outputs).  Here a
// row is held in registers between the reduction and the store, so x is read
// from HBM once: LPR lanes per row, NCH chunks of 8 values per lane, with
// nontemporal loads and stores (each byte is touched once).
//   LPR = 16   : rows of <= 128 values, 16 rows per 256-thread workgroup
//   LPR = 64   : rows of <= 2048 values, one wave per row
//   LPR = 512  : rows of <= 16384 values, one 512-thread workgroup per row
//                (fp32); 16-bit rows run persistent workgroups that load
//                the next row while the current one is reduced and stored
//   LPR = 1024 : rows of <= 32768 values, one 1024-thread workgroup per row
// (the wide rows merge their wave sums in LDS; 4 loads in flight per lane
// measured faster than 7 at 256 lanes for 13824-value rows)
// Rows whose length is not a multiple of 8, or longer, take a strided
// scalar path that reads x twice.
#include <algorithm>

#include "motif_common.hpp"

namespace motif {

struct PolyArgs {
  const void* x;
  const void* w;  // (3)
  const void* b;  // (1)
  void* y;
  long rows;
  int D;
  float eps;
};

template <typename T>
__device__ inline void load8v(const void* base, long idx, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 q = ld_stream4((const uint16_t*)base + idx);
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<T>::get(w, i);
  } else {
    const uint4 a = ld_stream4((const float*)base + idx);
    const uint4 c = ld_stream4((const float*)base + idx + 4);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(float, w[i]);
  }
}

template <typename T>
__device__ inline void store8v(void* base, long idx, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)Elem<T>::from_f32(v[2 * i]) |
             ((uint32_t)Elem<T>::from_f32(v[2 * i + 1]) << 16);
    st_stream4((uint16_t*)base + idx, w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __builtin_bit_cast(uint32_t, v[i]);
    st_stream4((float*)base + idx, w[0], w[1], w[2], w[3]);
    st_stream4((float*)base + idx + 4, w[4], w[5], w[6], w[7]);
  }
}

__device__ inline float poly_out(float v, float rs2, float rs4, float rs6, float w0, float w1,
                                 float w2, float b) {
  const float v2 = v * v;
  const float v3 = v2 * v;
  return w0 * (v3 * rs6) + w1 * (v2 * rs4) + w2 * (v * rs2) + b;
}

template <typename T, int LPR, int NCH, int TPB>
__global__ void __launch_bounds__(TPB) polynorm_vec_kernel(PolyArgs a) {
  constexpr int RPB = TPB / LPR;  // rows per block
  const int tid = threadIdx.x;
  const int sub = tid % LPR;
  const long row = (long)blockIdx.x * RPB + tid / LPR;
  const bool active = row < a.rows;
  const int nchunks = a.D / 8;
  const long base = (active ? row : 0) * (long)a.D;

  float v[NCH][8];
  float s2 = 0.f, s4 = 0.f, s6 = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = sub + LPR * j;
    if (active && c < nchunks) {
      load8v<T>(a.x, base + (long)c * 8, v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x2 = v[j][e] * v[j][e];
      const float x4 = x2 * x2;
      s2 += x2;
      s4 += x4;
      s6 += x4 * x2;
    }
  }
  if constexpr (LPR <= 64) {
    s2 = group_sum<LPR>(s2);
    s4 = group_sum<LPR>(s4);
    s6 = group_sum<LPR>(s6);
  } else {  // one row per workgroup: LPR / 64 wave sums meet in LDS
    constexpr int NWV = LPR / 64;
    static_assert(RPB == 1, "wide rows take the whole workgroup");
    __shared__ float red[3][NWV];
    s2 = group_sum<64>(s2);
    s4 = group_sum<64>(s4);
    s6 = group_sum<64>(s6);
    const int wave = tid >> 6;
    if ((tid & 63) == 0) {
      red[0][wave] = s2;
      red[1][wave] = s4;
      red[2][wave] = s6;
    }
    __syncthreads();
    s2 = s4 = s6 = 0.f;
#pragma unroll
    for (int i = 0; i < NWV; ++i) {
      s2 += red[0][i];
      s4 += red[1][i];
      s6 += red[2][i];
    }
  }
  if (!active) return;
  const float inv_d = 1.0f / (float)a.D;
  const float rs2 = rsqrtf(s2 * inv_d + a.eps);
  const float rs4 = rsqrtf(s4 * inv_d + a.eps);
  const float rs6 = rsqrtf(s6 * inv_d + a.eps);
  const float w0 = Elem<T>::load(a.w, 0), w1 = Elem<T>::load(a.w, 1), w2 = Elem<T>::load(a.w, 2);
  const float bb = Elem<T>::load(a.b, 0);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = sub + LPR * j;
    if (c < nchunks) {
      float out[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = poly_out(v[j][e], rs2, rs4, rs6, w0, w1, w2, bb);
      store8v<T>(a.y, base + (long)c * 8, out);
    }
  }
}

// Wide 16-bit rows, persistent: workgroup b takes rows b, b + grid, ...
// and loads row r + grid into a second register set while row r is reduced
// and stored, so every workgroup keeps a row of loads in flight.  The
// cross-wave sums alternate between two LDS slots, one barrier per row.
template <typename T, int NCH, int TPB>
__global__ void __launch_bounds__(TPB) polynorm_rows_kernel(PolyArgs a) {
  static_assert(sizeof(T) == 2, "16-bit rows");
  constexpr int NWV = TPB / 64;
  const int tid = threadIdx.x;
  const int nchunks = a.D / 8;
  __shared__ float red[2][3][NWV];
  uint4 raw0[NCH], raw1[NCH];
  auto load_row = [&](uint4 (&dst)[NCH], long row) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = tid + TPB * j;
      dst[j] = row < a.rows && c < nchunks
                   ? ld_stream4((const uint16_t*)a.x + row * (long)a.D + (long)c * 8)
                   : make_uint4(0, 0, 0, 0);
    }
  };
  const float inv_d = 1.0f / (float)a.D;
  const float w0 = Elem<T>::load(a.w, 0), w1 = Elem<T>::load(a.w, 1), w2 = Elem<T>::load(a.w, 2);
  const float bb = Elem<T>::load(a.b, 0);
  // Row `row` from cur (loaded), with row + grid loading into nxt.
  auto process = [&](const uint4 (&cur)[NCH], uint4 (&nxt)[NCH], long row, int par) {
    load_row(nxt, row + gridDim.x);  // zeros past the last row
    float s2 = 0.f, s4 = 0.f, s6 = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint32_t w[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = Elem<T>::get(w, e);
        const float x2 = v * v;
        const float x4 = x2 * x2;
        s2 += x2;
        s4 += x4;
        s6 += x4 * x2;
      }
    }
    s2 = group_sum<64>(s2);
    s4 = group_sum<64>(s4);
    s6 = group_sum<64>(s6);
    if ((tid & 63) == 0) {
      red[par][0][tid >> 6] = s2;
      red[par][1][tid >> 6] = s4;
      red[par][2][tid >> 6] = s6;
    }
    __syncthreads();
    s2 = s4 = s6 = 0.f;
#pragma unroll
    for (int i = 0; i < NWV; ++i) {
      s2 += red[par][0][i];
      s4 += red[par][1][i];
      s6 += red[par][2][i];
    }
    const float rs2 = rsqrtf(s2 * inv_d + a.eps);
    const float rs4 = rsqrtf(s4 * inv_d + a.eps);
    const float rs6 = rsqrtf(s6 * inv_d + a.eps);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = tid + TPB * j;
      if (c < nchunks) {
        const uint32_t w[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
        float out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          out[e] = poly_out(Elem<T>::get(w, e), rs2, rs4, rs6, w0, w1, w2, bb);
        store8v<T>(a.y, row * (long)a.D + (long)c * 8, out);
      }
    }
  };
  // The trip count depends only on blockIdx, so every barrier is reached by
  // the whole workgroup.
  long row = blockIdx.x;
  load_row(raw0, row);
  while (row < a.rows) {
    process(raw0, raw1, row, 0);
    row += gridDim.x;
    if (row >= a.rows) break;
    process(raw1, raw0, row, 1);
    row += gridDim.x;
  }
}

// Any D: one workgroup per row, two passes over x.
template <typename T>
__global__ void __launch_bounds__(256) polynorm_scalar_kernel(PolyArgs a) {
  const long row = blockIdx.x;
  const int tid = threadIdx.x;
  const long base = row * (long)a.D;
  float s2 = 0.f, s4 = 0.f, s6 = 0.f;
  for (int i = tid; i < a.D; i += 256) {
    const float v = Elem<T>::load(a.x, base + i);
    const float x2 = v * v, x4 = x2 * x2;
    s2 += x2;
    s4 += x4;
    s6 += x4 * x2;
  }
  __shared__ float red[3][4];
  s2 = group_sum<64>(s2);
  s4 = group_sum<64>(s4);
  s6 = group_sum<64>(s6);
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    red[0][wave] = s2;
    red[1][wave] = s4;
    red[2][wave] = s6;
  }
  __syncthreads();
  s2 = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
  s4 = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  s6 = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
  const float inv_d = 1.0f / (float)a.D;
  const float rs2 = rsqrtf(s2 * inv_d + a.eps);
  const float rs4 = rsqrtf(s4 * inv_d + a.eps);
  const float rs6 = rsqrtf(s6 * inv_d + a.eps);
  const float w0 = Elem<T>::load(a.w, 0), w1 = Elem<T>::load(a.w, 1), w2 = Elem<T>::load(a.w, 2);
  const float bb = Elem<T>::load(a.b, 0);
  for (int i = tid; i < a.D; i += 256)
    Elem<T>::store(a.y, base + i,
                   poly_out(Elem<T>::load(a.x, base + i), rs2, rs4, rs6, w0, w1, w2, bb));
}

template <typename T, int LPR, int TPB>
static void launch_poly_lpr(const PolyArgs& a, int nch, hipStream_t st) {
  const unsigned blocks = (unsigned)((a.rows + TPB / LPR - 1) / (TPB / LPR));
  switch (nch) {
    case 1: hipLaunchKernelGGL((polynorm_vec_kernel<T, LPR, 1, TPB>), blocks, TPB, 0, st, a); break;
    case 2: hipLaunchKernelGGL((polynorm_vec_kernel<T, LPR, 2, TPB>), blocks, TPB, 0, st, a); break;
    case 3: hipLaunchKernelGGL((polynorm_vec_kernel<T, LPR, 3, TPB>), blocks, TPB, 0, st, a); break;
    case 4: hipLaunchKernelGGL((polynorm_vec_kernel<T, LPR, 4, TPB>), blocks, TPB, 0, st, a); break;
    default: break;
  }
}

template <typename T>
static int launch_poly(const PolyArgs& a, bool vec_ok, hipStream_t st) {
  const int nchunks = a.D / 8;
  if (vec_ok && a.D % 8 == 0) {
    if (nchunks <= 16) {
      launch_poly_lpr<T, 16, 256>(a, 1, st);
      return check_launch("polynorm");
    }
    if (nchunks <= 64 * 4) {
      launch_poly_lpr<T, 64, 256>(a, (nchunks + 63) / 64, st);
      return check_launch("polynorm");
    }
    if (nchunks <= 512 * 4) {
      if constexpr (sizeof(T) == 2) {
        // Persistent rows: as many workgroups per CU as the register use of
        // NCH chunks per lane lets reside (measured at [3204, 13824]:
        // 44.0 us one row per workgroup, 33.9 us persistent at 2 per CU).
        const int nch = (nchunks + 511) / 512;
        const int per_cu = tuning().poly_rows > 0 ? tuning().poly_rows
                                                  : (nch == 1 ? 4 : nch == 2 ? 3 : 2);
        {
          const long grid = std::min<long>(a.rows, (long)device_cu_count() * per_cu);
          switch (nch) {
            case 1: hipLaunchKernelGGL((polynorm_rows_kernel<T, 1, 512>), (unsigned)grid, 512, 0, st, a); break;
            case 2: hipLaunchKernelGGL((polynorm_rows_kernel<T, 2, 512>), (unsigned)grid, 512, 0, st, a); break;
            case 3: hipLaunchKernelGGL((polynorm_rows_kernel<T, 3, 512>), (unsigned)grid, 512, 0, st, a); break;
            default: hipLaunchKernelGGL((polynorm_rows_kernel<T, 4, 512>), (unsigned)grid, 512, 0, st, a); break;
          }
          return check_launch("polynorm");
        }
      }
      launch_poly_lpr<T, 512, 512>(a, (nchunks + 511) / 512, st);
      return check_launch("polynorm");
    }
    if (nchunks <= 1024 * 4) {
      launch_poly_lpr<T, 1024, 1024>(a, (nchunks + 1023) / 1024, st);
      return check_launch("polynorm");
    }
  }
  hipLaunchKernelGGL((polynorm_scalar_kernel<T>), (unsigned)a.rows, 256, 0, st, a);
  return check_launch("polynorm");
}

}  // namespace motif

using namespace motif;

extern "C" int motif_polynorm(const void* x, const void* weight, const void* bias, void* y,
                              int dtype, int64_t rows, int D, float eps, void* stream) {
  CallScope scope;
  clear_error();
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "polynorm: unknown dtype code %d", dtype);
  MOTIF_REQUIRE(rows >= 0 && D >= 0, "polynorm: negative extent");
  if (rows == 0 || D == 0) return MOTIF_OK;
  MOTIF_REQUIRE(x && weight && bias && y, "polynorm: null pointer");
  PolyArgs a{x, weight, bias, y, (long)rows, D, eps};
  const bool vec_ok = (((uintptr_t)x | (uintptr_t)y) & 15u) == 0;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case MOTIF_F16: return launch_poly<half_t>(a, vec_ok, st);
    case MOTIF_BF16: return launch_poly<bf16_t>(a, vec_ok, st);
    default: return launch_poly<float>(a, vec_ok, st);
  }
}
