// Shared device helpers for the gfx950 kernels: element types, 16-byte
// vector loads, wave64 DPP reductions and the thread-local error channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "motif_hip.h"

namespace motif {

// ---------------------------------------------------------------- errors --
// Thread-local last-error message behind motif_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define MOTIF_REQUIRE(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::motif::set_error(__VA_ARGS__);           \
      return MOTIF_ERR_CONTRACT;                 \
    }                                            \
  } while (0)

// Check the launch that was just enqueued.
int check_launch(const char* what);

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Process-wide tuning values (motif_set_tuning).
struct Tuning {
  int rows_per_split = 0;  // 0 = automatic
  int waves_per_wg = 0;    // 0 = automatic
  int min_wgs = 0;         // 0 = automatic
  int mfma = 1;            // 1 = matrix-core kernels where compiled, 0 = VALU kernels
  int fused_merge = 0;     // 1 = last-arriving workgroup merges splits, 0 = merge kernel
  int poly_rows = 0;       // persistent PolyNorm workgroups per CU (0 = by register use)
  int qpair = 1;           // paired-tile packed-cache kernel (group size 64/128): 0 off, 1 bf16 q4, 2 every call
  int qslab = 2;           // slabs of 17..64 virtual heads, tiles dequantised into LDS: 0 off, 1 q8, 2 q4+q8
  int qslab_ws = 1;        // slab kernel with producer / consumer waves (8 waves): 1 on, 0 off
  int merge_rows = 1;      // row-per-wave merge launch from 2048 partial rows: 1 on, 0 off
  int qslab_sets = 2;      // producer register sets of the producer / consumer slab kernel (2 or 3)
  int prefill_ncb = 0;     // column blocks per wave of the 8-wave prefill kernel (0 = automatic)
  int prefill_min_heads = 0;  // virtual heads per KV head from which multi-row fp16/bf16 calls take the shared-tile kernel (0: automatic)
  int part_f16 = 1;       // shared-tile kernels' split partials over fp16 caches as fp16 o / l when the row-per-wave merge reads them: 1 on, 0 fp32
};
// The calling thread's snapshot of the process-wide knobs.  Inside a
// CallScope it is the copy taken when the outermost scope opened, so every
// read of one call (plan, workspace carving, dispatch) sees the same values
// and a concurrent motif_set_tuning affects the next call only.  Outside a
// scope each read takes a fresh copy.
const Tuning& tuning();
// Opened first thing by every extern "C" entry point that reads tuning()
// (nested entry points share the outer snapshot).
struct CallScope {
  CallScope();
  ~CallScope();
  CallScope(const CallScope&) = delete;
  CallScope& operator=(const CallScope&) = delete;
};

// ------------------------------------------------------------ elements ----
// bf16 is carried as its 16 storage bits; conversion is exact (to f32) and
// round-to-nearest-even (from f32), NaN kept quiet.
struct bf16_t {
  uint16_t bits;
};

typedef _Float16 half_t;

template <typename T>
struct Elem;

template <>
struct Elem<half_t> {
  static constexpr int kBytes = 2;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(half_t, b);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (half_t)f);
  }
  // Element i of a packed 32-bit word array.
  __device__ static inline float get(const uint32_t* w, int i) {
    uint32_t x = w[i >> 1];
    return to_f32((uint16_t)((i & 1) ? (x >> 16) : (x & 0xFFFFu)));
  }
  __device__ static inline float load(const void* p, long i) {
    return to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static inline void store(void* p, long i, float f) {
    ((uint16_t*)p)[i] = from_f32(f);
  }
};

template <>
struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ static inline float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, ((uint32_t)b) << 16);
  }
  __device__ static inline uint16_t from_f32(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
  __device__ static inline float get(const uint32_t* w, int i) {
    uint32_t x = w[i >> 1];
    return (i & 1) ? __builtin_bit_cast(float, x & 0xFFFF0000u)
                   : __builtin_bit_cast(float, x << 16);
  }
  __device__ static inline float load(const void* p, long i) {
    return to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static inline void store(void* p, long i, float f) {
    ((uint16_t*)p)[i] = from_f32(f);
  }
};

template <>
struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static inline float get(const uint32_t* w, int i) {
    return __builtin_bit_cast(float, w[i]);
  }
  __device__ static inline float load(const void* p, long i) { return ((const float*)p)[i]; }
  __device__ static inline void store(void* p, long i, float f) { ((float*)p)[i] = f; }
};

// ---------------------------------------------------------------- loads ---
// Load NW 32-bit words from a pointer aligned to the widest power-of-two
// divisor of 4*NW bytes (<= 16): dwordx4 / dwordx2 / dword.
template <int NW>
__device__ inline void load_words(uint32_t (&dst)[NW], const uint32_t* src) {
  if constexpr (NW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      uint4 v = *reinterpret_cast<const uint4*>(src + i);
      dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
    }
  } else if constexpr (NW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < NW; i += 2) {
      uint2 v = *reinterpret_cast<const uint2*>(src + i);
      dst[i] = v.x; dst[i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) dst[i] = src[i];
  }
}

// Streaming loads for data read once per call (the KV cache): the
// nontemporal hint keeps these lines from displacing reusable ones.  On the
// 16k decode it saves about 1.5 us per call against plain loads.
typedef unsigned u32x4_nt_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_nt_t __attribute__((ext_vector_type(2)));
__device__ inline uint4 ld_stream4(const void* p) {
  const u32x4_nt_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline uint2 ld_stream2(const void* p) {
  const u32x2_nt_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_nt_t*>(p));
  return make_uint2(v.x, v.y);
}
__device__ inline uint32_t ld_stream1(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
// Streaming 16-byte store (output written once).
__device__ inline void st_stream4(void* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  __builtin_nontemporal_store(u32x4_nt_t{a, b, c, d}, reinterpret_cast<u32x4_nt_t*>(p));
}

// load_words with streaming loads.
template <int NW>
__device__ inline void load_words_stream(uint32_t (&dst)[NW], const uint32_t* src) {
  if constexpr (NW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      const uint4 v = ld_stream4(src + i);
      dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
    }
  } else if constexpr (NW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < NW; i += 2) {
      const uint2 v = ld_stream2(src + i);
      dst[i] = v.x; dst[i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) dst[i] = ld_stream1(src + i);
  }
}

// ------------------------------------------------------------ reductions --
// DPP row (16-lane) controls of gfx9: quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of W lanes (W a power of two <= 64).  Every lane of
// a group ends with the same bits: each step adds two operands that are the
// same pair for both partner lanes.
template <int W>
__device__ inline float group_sum(float x) {
  if constexpr (W >= 2) x += dpp<kDppQuadXor1>(x);
  if constexpr (W >= 4) x += dpp<kDppQuadXor2>(x);
  if constexpr (W >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (W >= 16) x += dpp<kDppMirror>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16);
  if constexpr (W >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Maximum of two floats as v_maximum(3)_f32 (the IEEE 754-2019 maximum):
// fmaxf (maxnum) first canonicalises each operand the compiler cannot prove
// canonical -- MFMA results, cross-lane moves -- with a v_max_f32 x, x of
// its own, tripling a max tree over scores.  For non-NaN operands the value
// is fmaxf's (a NaN operand gives NaN instead of the other operand).
__device__ inline float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

template <int W>
__device__ inline float group_max(float x) {
  if constexpr (W >= 2) x = fmaxf(x, dpp<kDppQuadXor1>(x));
  if constexpr (W >= 4) x = fmaxf(x, dpp<kDppQuadXor2>(x));
  if constexpr (W >= 8) x = fmaxf(x, dpp<kDppHalfMirror>(x));
  if constexpr (W >= 16) x = fmaxf(x, dpp<kDppMirror>(x));
  if constexpr (W >= 32) x = fmaxf(x, __shfl_xor(x, 16));
  if constexpr (W >= 64) x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

// exp2 on the hardware unit (v_exp_f32); inputs here are <= 0 or the
// -1e30 sentinel, whose result 0 is exact.
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace motif
