// MLX-affine quantisation on gfx950: mx.quantize (affine mode) restated,
// the single-dispatch 4-slot cache write, and dequantisation.
//
// Layout per group of `gs` consecutive values along the last axis:
//   scale, bias of type T; value i of a row packed at bits
//   [(i % (32/bits))*bits, +bits) of uint32 word i / (32/bits).
//
// The per-group arithmetic (lane mapping, bit-exact fp32 steps) is in
// quant_impl.hpp.
#include "quant_impl.hpp"

namespace motif {

// Plain quantisation of `rows` rows of D values.
template <typename T, int BITS, int LPG>
__global__ void __launch_bounds__(256) quantize_kernel(const void* x, uint32_t* data,
                                                       void* scales, void* biases, long nchunks,
                                                       int D, int gs) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const bool active = i < nchunks;
  const long ic = active ? i : 0;  // inactive lanes form whole groups; keep them in lockstep
  const int cpr = D / 8;           // chunks per row
  const long row = ic / cpr;
  const int c = (int)(ic % cpr);
  float v[8];
  load8<T>(x, row * D + (long)c * 8, v);
  uint32_t w[2];
  float scale, bias;
  quantize8<BITS, LPG>(v, w, scale, bias);
  if (!active) return;
  const int wpc = 8 * BITS / 32;  // words per chunk
  store_words<BITS>(data, row * (D * BITS / 32) + (long)c * wpc, w);
  if ((c % LPG) == 0) {
    const long si = row * (D / gs) + c / LPG;
    Elem<T>::store(scales, si, scale);
    Elem<T>::store(biases, si, bias);
  }
}

struct Write4Args {
  const void* src[4];  // k1, k2, v1, v2: (B, H, S, D)
  uint32_t* data[4];   // (B, H, kv_cap, D*bits/32)
  void* scales[4];     // (B, H, kv_cap, D/gs)
  void* biases[4];
  long slot_chunks;    // B*H*S*D/8
  int D, S, kv_cap, offset, gs;
};

// One dispatch for the four slots: chunk index runs over slot-major
// (slot, b, h, s, chunk); rows land at [offset, offset + S) of each slot.
template <typename T, int BITS, int LPG>
__global__ void __launch_bounds__(256) quant_write4_kernel(Write4Args a) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const bool active = i < 4 * a.slot_chunks;
  const long ic = active ? i : 0;
  const int slot = (int)(ic / a.slot_chunks);
  const long j = ic % a.slot_chunks;
  const int cpr = a.D / 8;
  const long srow = j / cpr;  // (b*H + h)*S + s
  const int c = (int)(j % cpr);
  float v[8];
  load8<T>(a.src[slot], srow * a.D + (long)c * 8, v);
  uint32_t w[2];
  float scale, bias;
  quantize8<BITS, LPG>(v, w, scale, bias);
  if (!active) return;
  const long bh = srow / a.S;
  const int s = (int)(srow % a.S);
  const long crow = bh * a.kv_cap + a.offset + s;
  const int wpc = 8 * BITS / 32;
  store_words<BITS>(a.data[slot], crow * (a.D * BITS / 32) + (long)c * wpc, w);
  if ((c % LPG) == 0) {
    const long si = crow * (a.D / a.gs) + c / LPG;
    Elem<T>::store(a.scales[slot], si, scale);
    Elem<T>::store(a.biases[slot], si, bias);
  }
}

// y = T(float(scale) * float(u) + float(bias)), one thread per value.
template <typename T, int BITS>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint32_t* data, const void* scales,
                                                         const void* biases, void* y, long n,
                                                         int D, int gs) {
#pragma clang fp contract(off)
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  constexpr int EL = 32 / BITS;
  const long row = i / D;
  const int c = (int)(i % D);
  const uint32_t word = data[row * (D / EL) + c / EL];
  const uint32_t u = (word >> ((c % EL) * BITS)) & ((1u << BITS) - 1u);
  const long si = row * (D / gs) + c / gs;
  const float s = Elem<T>::load(scales, si);
  const float b = Elem<T>::load(biases, si);
  Elem<T>::store(y, i, s * (float)u + b);
}

// ----------------------------------------------------------------- host ---
static int quant_checks(const char* name, int dtype, int D, int bits, int gs) {
  MOTIF_REQUIRE(dtype == MOTIF_F16 || dtype == MOTIF_BF16 || dtype == MOTIF_F32,
                "%s: unknown dtype code %d", name, dtype);
  MOTIF_REQUIRE(bits == 4 || bits == 8, "%s: bits=%d must be 4 or 8", name, bits);
  MOTIF_REQUIRE(gs == 32 || gs == 64 || gs == 128, "%s: group_size=%d must be 32, 64 or 128",
                name, gs);
  MOTIF_REQUIRE(D > 0 && D % gs == 0, "%s: last axis %d must be a multiple of group_size=%d",
                name, D, gs);
  return MOTIF_OK;
}

template <typename T, int BITS>
static void launch_quantize(const void* x, uint32_t* d, void* s, void* b, long nchunks, int D,
                            int gs, hipStream_t st) {
  const unsigned blocks = (unsigned)((nchunks + 255) / 256);
  switch (gs / 8) {
    case 4:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 4>), blocks, 256, 0, st, x, d, s, b, nchunks,
                         D, gs);
      break;
    case 8:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 8>), blocks, 256, 0, st, x, d, s, b, nchunks,
                         D, gs);
      break;
    default:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 16>), blocks, 256, 0, st, x, d, s, b,
                         nchunks, D, gs);
      break;
  }
}

template <typename T, int BITS>
static void launch_write4(const Write4Args& a, hipStream_t st) {
  const unsigned blocks = (unsigned)((4 * a.slot_chunks + 255) / 256);
  switch (a.gs / 8) {
    case 4: hipLaunchKernelGGL((quant_write4_kernel<T, BITS, 4>), blocks, 256, 0, st, a); break;
    case 8: hipLaunchKernelGGL((quant_write4_kernel<T, BITS, 8>), blocks, 256, 0, st, a); break;
    default: hipLaunchKernelGGL((quant_write4_kernel<T, BITS, 16>), blocks, 256, 0, st, a); break;
  }
}

template <template <typename, int> class F, typename... Args>
static void by_type_bits(int dtype, int bits, Args&&... args) {
  if (dtype == MOTIF_F16) {
    bits == 4 ? F<half_t, 4>::run(args...) : F<half_t, 8>::run(args...);
  } else if (dtype == MOTIF_BF16) {
    bits == 4 ? F<bf16_t, 4>::run(args...) : F<bf16_t, 8>::run(args...);
  } else {
    bits == 4 ? F<float, 4>::run(args...) : F<float, 8>::run(args...);
  }
}

template <typename T, int BITS>
struct QuantizeOp {
  static void run(const void* x, uint32_t* d, void* s, void* b, long nchunks, int D, int gs,
                  hipStream_t st) {
    launch_quantize<T, BITS>(x, d, s, b, nchunks, D, gs, st);
  }
};

template <typename T, int BITS>
struct Write4Op {
  static void run(const Write4Args& a, hipStream_t st) { launch_write4<T, BITS>(a, st); }
};

template <typename T, int BITS>
struct DequantOp {
  static void run(const uint32_t* d, const void* s, const void* b, void* y, long n, int D,
                  int gs, hipStream_t st) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL((dequantize_kernel<T, BITS>), blocks, 256, 0, st, d, s, b, y, n, D, gs);
  }
};

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace motif

using namespace motif;

extern "C" {

int motif_quantize(const void* x, uint32_t* data, void* scales, void* biases, int dtype,
                   int64_t rows, int D, int bits, int group_size, void* stream) {
  CallScope scope;
  clear_error();
  int rc = quant_checks("quantize", dtype, D, bits, group_size);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(rows >= 0, "quantize: rows=%lld must be >= 0", (long long)rows);
  if (rows == 0) return MOTIF_OK;
  MOTIF_REQUIRE(x && data && scales && biases, "quantize: null tensor pointer");
  MOTIF_REQUIRE(aligned16(x), "quantize: input must be 16-byte aligned");
  MOTIF_REQUIRE(((uintptr_t)data & (bits == 8 ? 7u : 3u)) == 0,
                "quantize: packed output misaligned");
  const long nchunks = (long)rows * (D / 8);
  by_type_bits<QuantizeOp>(dtype, bits, x, data, scales, biases, nchunks, D, group_size,
                           (hipStream_t)stream);
  return check_launch("quantize");
}

int motif_dequantize(const uint32_t* data, const void* scales, const void* biases, void* y,
                     int dtype, int64_t rows, int D, int bits, int group_size, void* stream) {
  CallScope scope;
  clear_error();
  int rc = quant_checks("dequantize", dtype, D, bits, group_size);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(rows >= 0, "dequantize: rows=%lld must be >= 0", (long long)rows);
  if (rows == 0) return MOTIF_OK;
  MOTIF_REQUIRE(data && scales && biases && y, "dequantize: null tensor pointer");
  by_type_bits<DequantOp>(dtype, bits, data, scales, biases, y, (long)rows * D, D, group_size,
                          (hipStream_t)stream);
  return check_launch("dequantize");
}

int motif_quant_write4(const void* k1, const void* k2, const void* v1, const void* v2,
                       uint32_t* const data[4], void* const scales[4], void* const biases[4],
                       int dtype, int B, int H, int S, int D, int kv_cap, int offset, int bits,
                       int group_size, void* stream) {
  CallScope scope;
  clear_error();
  int rc = quant_checks("quant_write4", dtype, D, bits, group_size);
  if (rc != MOTIF_OK) return rc;
  MOTIF_REQUIRE(B >= 1 && H >= 1 && S >= 0, "quant_write4: B, H must be >= 1 and S >= 0");
  MOTIF_REQUIRE(offset >= 0 && (long)offset + S <= kv_cap,
                "quant_write4: rows [%d, %d) exceed capacity %d", offset, offset + S, kv_cap);
  if (S == 0) return MOTIF_OK;
  MOTIF_REQUIRE(data && scales && biases, "quant_write4: null slot array");
  Write4Args a{};
  const void* src[4] = {k1, k2, v1, v2};
  for (int i = 0; i < 4; ++i) {
    MOTIF_REQUIRE(src[i] && data[i] && scales[i] && biases[i], "quant_write4: null pointer");
    MOTIF_REQUIRE(aligned16(src[i]), "quant_write4: inputs must be 16-byte aligned");
    MOTIF_REQUIRE(((uintptr_t)data[i] & (bits == 8 ? 7u : 3u)) == 0,
                  "quant_write4: packed cache misaligned");
    a.src[i] = src[i];
    a.data[i] = data[i];
    a.scales[i] = scales[i];
    a.biases[i] = biases[i];
  }
  a.slot_chunks = (long)B * H * S * (D / 8);
  a.D = D;
  a.S = S;
  a.kv_cap = kv_cap;
  a.offset = offset;
  a.gs = group_size;
  by_type_bits<Write4Op>(dtype, bits, a, (hipStream_t)stream);
  return check_launch("quant_write4");
}

}  // extern "C"
