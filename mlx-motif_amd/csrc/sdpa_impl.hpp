// Split-KV shared-QK dual-V attention for gfx950, one template for every
// cache format.
//
// Work decomposition (one launch):
//   workgroup = (batch b, KV head, chunk of <= GC "virtual heads", KV split)
//   A virtual head is one (query head, query row) pair that reads this KV
//   head: GQA factor G times S_q rows.  All of them are served by the same
//   K/V/V rows, so each KV row is read from HBM once per chunk.
//   Within the workgroup, LPR lanes share one KV row (16-byte loads for the
//   fp16 cache), a wave covers 64/LPR rows per load, and each wave walks its
//   rows keeping an online softmax (running max m, sum l, two accumulators)
//   per virtual head in log2 units.
// Merges: row groups of a wave (lane shuffles), waves of a workgroup (LDS),
// then splits: every workgroup writes (m, l, o1, o2) to the workspace, and
// either sdpa_merge_kernel (a second launch, the default) or the last
// workgroup to arrive for its (b, KV head, chunk) combines all splits and
// writes y; the in-kernel merge re-arms its arrival counter.
//
// Reference semantics (src/mlx_motif/kernels/attention.py:53-166, 293-445):
// q scaled once in fp32, fp32 accumulation, running-max sentinel -1e30,
// output o/l with o left unnormalised (zero) when l == 0.
#pragma once

#include "motif_common.hpp"
#include "sdpa_plan.hpp"

namespace motif {

constexpr float kNegSentinel = -1e30f;

// Four floats as fp16 (round to nearest even), packed in two words, and back.
__device__ inline uint2 half4_bits(float4 v) {
  return make_uint2(
      (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.x) |
          ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.y) << 16),
      (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.z) |
          ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.w) << 16));
}
__device__ inline float4 half4_floats(uint2 w) {
  return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(w.x & 0xFFFFu)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x >> 16)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y & 0xFFFFu)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y >> 16)));
}

// Cross-workgroup hand-off of split partials without whole-cache maintenance.
// Partials are stored and re-loaded through raw buffer operations with the
// sc0|sc1 cache policy: stores are written through the XCD's L2 to memory,
// loads miss in L1/L2 and read memory, both 16 bytes per lane and without
// the per-access waits a volatile access would add.  A writer waits for all
// its stores to complete (s_waitcnt 0) before it takes an arrival ticket, so
// the workgroup that takes the last ticket reads complete partials.  (An
// agent-scope __threadfence() here costs a buffer_wbl2 + buffer_inv of the
// whole L2 per workgroup, which serialises per XCD.)
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
constexpr int kCachePolicyThrough = 1 | 16;  // sc0 | sc1

// Buffer resource over [base, base + bytes); lanes outside it read 0 and
// drop their stores.
__device__ inline __amdgpu_buffer_rsrc_t part_rsrc(const float* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// Per-split buffer resources: base at the split's first row, range = its
// rows, so loads past the split's end return 0 with no memory traffic and
// need no branch.  Cache policy nt: the KV cache is read once per call.
constexpr int kCachePolicyStream = 2;  // nt

__device__ inline __amdgpu_buffer_rsrc_t stream_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// POL: kCachePolicyStream for data read once per call, 0 (cached) where
// several workgroups read the same rows (head chunks of a verify slab).
template <int POL = kCachePolicyStream>
__device__ inline uint4 bload4(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL));
}
template <int POL = kCachePolicyStream>
__device__ inline uint2 bload2(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL));
}
template <int POL = kCachePolicyStream>
__device__ inline uint32_t bload1(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
}

__device__ inline void store_through4(__amdgpu_buffer_rsrc_t r, unsigned byte_off, float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, byte_off, 0,
                                         kCachePolicyThrough);
}
__device__ inline float4 load_through4(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
  return __builtin_bit_cast(
      float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicyThrough));
}
__device__ inline void store_through2(__amdgpu_buffer_rsrc_t r, unsigned byte_off, float2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, byte_off, 0,
                                        kCachePolicyThrough);
}
__device__ inline float2 load_through2(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
  return __builtin_bit_cast(
      float2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kCachePolicyThrough));
}
__device__ inline void wait_stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // keep the compiler from moving memory ops
  __builtin_amdgcn_s_waitcnt(0);             // vmcnt = expcnt = lgkmcnt = 0
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Workgroup -> (unit = (b, KV head, chunk), split).  With one chunk per KV
// head, consecutive workgroups take the KV heads of one split.  With several
// chunks (more virtual heads than one workgroup holds, e.g. a verify slab),
// the chunks of one (b, KV head, split) go to workgroups 8 apart: the
// dispatcher deals workgroups round-robin to the 8 XCDs, so those chunks run
// on one XCD and all but the first find the shared K/V rows in its L2.
// Placement only affects speed.  Padding workgroups (see sdpa_grid_blocks)
// return false and exit.
__device__ inline bool sdpa_block_coords(const SdpaArgs& a, int bid, int& unit, int& split) {
  const int bh = a.B * a.Hkv;
  if (a.nchunk == 1) {
    unit = bid % bh;
    split = bid / bh;
    return true;
  }
  const int slot = bid >> 3;
  const int chunk = slot % a.nchunk;
  const int g = (slot / a.nchunk) * 8 + (bid & 7);  // g = split * bh + (b, KV head)
  if (g >= bh * a.nsplit) return false;
  split = g / bh;
  unit = (g % bh) * a.nchunk + chunk;
  return true;
}

// --------------------------------------------------------------- formats --
// fp16 / bf16 / fp32 cache rows of D elements.  16 lanes per row.
template <typename T_, int D_>
struct FpFmt {
  using T = T_;
  static constexpr int D = D_;
  static constexpr int LPR = 16;
  static constexpr int CPL = D / 16;  // channels per lane
  static constexpr int WPL = CPL * Elem<T>::kBytes / 4;
  static constexpr int WPR = D * Elem<T>::kBytes / 4;
  // Byte alignment every tensor base pointer must have.
  static constexpr int kAlign = (WPL % 4 == 0) ? 16 : (WPL % 2 == 0) ? 8 : 4;

  struct Frag {
    uint32_t w[WPL];
  };

  const uint32_t* k;
  const uint32_t* v1;
  const uint32_t* v2;

  __device__ FpFmt(const SdpaArgs& a, long bk, int sub) {
    long off = bk * (long)a.kv_cap * WPR + (long)sub * WPL;
    k = (const uint32_t*)a.k + off;
    v1 = (const uint32_t*)a.v1 + off;
    v2 = (const uint32_t*)a.v2 + off;
  }
  __device__ inline void load(int row, Frag& kf, Frag& v1f, Frag& v2f) const {
    long o = (long)row * WPR;
    load_words_stream<WPL>(kf.w, k + o);
    load_words_stream<WPL>(v1f.w, v1 + o);
    load_words_stream<WPL>(v2f.w, v2 + o);
  }
  __device__ static inline void zero(Frag& f) {
#pragma unroll
    for (int i = 0; i < WPL; ++i) f.w[i] = 0;
  }
  __device__ static inline void values(const Frag& f, float (&x)[CPL]) {
#pragma unroll
    for (int e = 0; e < CPL; ++e) x[e] = Elem<T>::get(f.w, e);
  }
};

// Packed MLX-affine cache: u32 words of 32/BITS unsigned values, one
// (scale, bias) pair of type T per group_size values; value = s*u + b.
template <typename T_, int D_, int BITS>
struct QFmt {
  using T = T_;
  static constexpr int D = D_;
  static constexpr int EL = 32 / BITS;                      // values per word
  static constexpr int CPL = (D / 16 > EL) ? D / 16 : EL;  // channels per lane
  static constexpr int WPL = CPL / EL;                      // words per lane
  static constexpr int LPR = D / CPL;
  static constexpr int WPR = D / EL;
  static constexpr uint32_t MASK = (1u << BITS) - 1u;
  static constexpr int kAlign = (WPL % 4 == 0) ? 16 : (WPL % 2 == 0) ? 8 : 4;

  struct Frag {
    uint32_t w[WPL];
    float s, b;
  };

  const uint32_t* kd;
  const uint32_t* v1d;
  const uint32_t* v2d;
  const void* ks;
  const void* kb;
  const void* v1s;
  const void* v1b;
  const void* v2s;
  const void* v2b;
  long sbase;  // scale index of row 0 of this (b, KV head) plus the lane's group
  int ngroups;

  __device__ QFmt(const SdpaArgs& a, long bk, int sub) {
    long off = bk * (long)a.kv_cap * WPR + (long)sub * WPL;
    kd = a.kd + off;
    v1d = a.v1d + off;
    v2d = a.v2d + off;
    ks = a.ks; kb = a.kb; v1s = a.v1s; v1b = a.v1b; v2s = a.v2s; v2b = a.v2b;
    ngroups = D / a.group_size;
    sbase = bk * (long)a.kv_cap * ngroups + (sub * CPL) / a.group_size;
  }
  __device__ inline void load(int row, Frag& kf, Frag& v1f, Frag& v2f) const {
    long o = (long)row * WPR;
    load_words_stream<WPL>(kf.w, kd + o);
    load_words_stream<WPL>(v1f.w, v1d + o);
    load_words_stream<WPL>(v2f.w, v2d + o);
    long si = sbase + (long)row * ngroups;
    kf.s = Elem<T>::load(ks, si);   kf.b = Elem<T>::load(kb, si);
    v1f.s = Elem<T>::load(v1s, si); v1f.b = Elem<T>::load(v1b, si);
    v2f.s = Elem<T>::load(v2s, si); v2f.b = Elem<T>::load(v2b, si);
  }
  __device__ static inline void zero(Frag& f) {
#pragma unroll
    for (int i = 0; i < WPL; ++i) f.w[i] = 0;
    f.s = 0.f;
    f.b = 0.f;
  }
  // Dequantise in fp32 exactly as the reference kernel: s * float(u) + b.
  __device__ static inline void values(const Frag& f, float (&x)[CPL]) {
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      uint32_t u = (f.w[e / EL] >> ((e % EL) * BITS)) & MASK;
      x[e] = f.s * (float)u + f.b;
    }
  }
};

// Floats of padding per LDS head row: keeps the head rows of the
// cross-wave staging buffer on different LDS banks.
constexpr int kLdsPad = 4;

// y[off .. off+3] = v / L (v itself where L == 0: no visible key), one
// 8-byte store for 2-byte types (off is a multiple of 4).
template <typename T, int D>
__device__ inline void store_y4_to(void* y, long off, float4 v, float L) {
  const bool z = L == 0.f;
  const float o[4] = {z ? v.x : v.x / L, z ? v.y : v.y / L, z ? v.z : v.z / L,
                      z ? v.w : v.w / L};
  if constexpr (Elem<T>::kBytes == 2) {
    const uint2 w = make_uint2(
        (uint32_t)Elem<T>::from_f32(o[0]) | ((uint32_t)Elem<T>::from_f32(o[1]) << 16),
        (uint32_t)Elem<T>::from_f32(o[2]) | ((uint32_t)Elem<T>::from_f32(o[3]) << 16));
    *reinterpret_cast<uint2*>((uint16_t*)y + off) = w;
  } else {
    *reinterpret_cast<float4*>((float*)y + off) = make_float4(o[0], o[1], o[2], o[3]);
  }
}
template <typename T, int D>
__device__ inline void store_y4(const SdpaArgs& a, long off, float4 v, float L) {
  store_y4_to<T, D>(a.y, off, v, L);
}

// ------------------------------------------------------- split merge ---
// Combine the nsplit partials (m, l, o1, o2) of virtual heads qrow0 ..
// qrow0+nvh-1 and write y.  One round trip: every thread issues its first
// (m, l) load and the 16-byte loads of its first UNR partials before
// anything is consumed; one wave per head then turns the maxima into factors
// exp2(m_s - M) and the total L, and P threads per output float4 sum their
// splits, meeting in LDS.
template <typename T, int D, int GC, int NW>
__device__ void merge_splits(const SdpaArgs& a, long qrow0, int nvh) {
  constexpr int NT = NW * 64;
  constexpr int C4 = 2 * D / 4;
  constexpr int UNR = 16;
  __shared__ float lds_f[GC][kMaxSplits];  // m_s, then exp2(m_s - M)
  __shared__ float lds_l[GC][kMaxSplits];
  __shared__ float lds_L[GC];
  __shared__ __attribute__((aligned(16))) float4 lds_acc[NT];
  const int tid = threadIdx.x;
  const int ns = a.nsplit;
  const auto ro = part_rsrc(a.part_o + qrow0 * ns * 2 * D, (unsigned)(nvh * ns * 2 * D * 4));
  const auto rml = part_rsrc(a.part_ml + qrow0 * ns * 2, (unsigned)(nvh * ns * 2 * 4));

  const int nml = nvh * ns;
  const float2 ml0 = tid < nml ? load_through2(rml, (unsigned)tid * 8u) : make_float2(0.f, 0.f);
  const int items = nvh * C4;
  const int P = items >= NT ? 1 : NT / items;  // threads per output float4
  const int passes = P > 1 ? 1 : (items + NT - 1) / NT;
  // this thread's output float4 of pass 0 and its share of the splits
  const int item0 = P > 1 ? tid % items : tid;
  const int part = P > 1 ? tid / items : 0;
  const bool on0 = item0 < items && part < P;
  float4 pre[UNR];
#pragma unroll
  for (int j = 0; j < UNR; ++j) {
    const int s = part + j * P;
    const unsigned off = (unsigned)((((item0 / C4) * ns + s) * 2 * D + (item0 % C4) * 4) * 4);
    pre[j] = (on0 && s < ns) ? load_through4(ro, off) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid < nml) {
    lds_f[tid / ns][tid % ns] = ml0.x;
    lds_l[tid / ns][tid % ns] = ml0.y;
  }
  for (int i = tid + NT; i < nml; i += NT) {  // more than NT (head, split) pairs
    const float2 v = load_through2(rml, (unsigned)i * 8u);
    lds_f[i / ns][i % ns] = v.x;
    lds_l[i / ns][i % ns] = v.y;
  }
  __syncthreads();

  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int g = wave; g < nvh; g += NW) {
    float M = kNegSentinel;
    for (int s = lane; s < ns; s += 64) M = fmaxf(M, lds_f[g][s]);
    M = group_max<64>(M);
    float L = 0.f;
    for (int s = lane; s < ns; s += 64) {
      const float f = fast_exp2(lds_f[g][s] - M);
      lds_f[g][s] = f;
      L = fmaf(lds_l[g][s], f, L);
    }
    L = group_sum<64>(L);
    if (lane == 0) lds_L[g] = L;
  }
  __syncthreads();

  for (int ps = 0; ps < passes; ++ps) {
    const int item = P > 1 ? item0 : ps * NT + tid;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (item < items && part < P) {
      const int g = item / C4;
      const int c = (item % C4) * 4;
      for (int s0 = part; s0 < ns; s0 += P * UNR) {
        float4 v[UNR];
#pragma unroll
        for (int j = 0; j < UNR; ++j) {
          const int s = s0 + j * P;
          if (ps == 0 && s0 == part) {
            v[j] = pre[j];
          } else {
            const unsigned off = (unsigned)(((g * ns + s) * 2 * D + c) * 4);
            v[j] = s < ns ? load_through4(ro, off) : make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
#pragma unroll
        for (int j = 0; j < UNR; ++j) {
          const int s = s0 + j * P;
          const float f = s < ns ? lds_f[g][s] : 0.f;
          acc.x = fmaf(v[j].x, f, acc.x);
          acc.y = fmaf(v[j].y, f, acc.y);
          acc.z = fmaf(v[j].z, f, acc.z);
          acc.w = fmaf(v[j].w, f, acc.w);
        }
      }
    }
    if (P > 1) {
      lds_acc[tid] = acc;
      __syncthreads();
      if (tid < items) {
        float4 t = lds_acc[tid];
        for (int p = 1; p < P; ++p) {
          const float4 u = lds_acc[p * items + tid];
          t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        const int g = tid / C4;
        store_y4<T, D>(a, (qrow0 + g) * 2 * D + (tid % C4) * 4, t, lds_L[g]);
      }
    } else if (item < items) {
      const int g = item / C4;
      store_y4<T, D>(a, (qrow0 + g) * 2 * D + (item % C4) * 4, acc, lds_L[g]);
    }
  }
}

// ------------------------------------------------- workgroup epilogue ---
// Combine the NW waves' (m, l, o1, o2) staged in LDS (log2-domain running
// max, sum and unnormalised accumulators per virtual head), then either
// write y (single split) or publish this split's partial with 16-byte
// write-through stores and, in the workgroup that arrives last for its
// (b, KV head, chunk), merge all splits.  Called by every thread of the
// workgroup after a barrier.  PARTIALS: always publish partials (also for a
// single split) and leave the merge to a second launch.
template <typename T, int D, int GC, int NW, bool PARTIALS = false, bool FUSED_MERGE = true>
__device__ void wg_epilogue(const SdpaArgs& a, const float (&lds_o)[NW][GC][2 * D + kLdsPad],
                            const float (&lds_m)[NW][GC], const float (&lds_l)[NW][GC],
                            long qrow0, int nvh, int split, int unit) {
  constexpr int C4 = 2 * D / 4;
  const bool single = !PARTIALS && a.nsplit == 1;
  const int ns = a.nsplit;
  // (single split: no workspace, empty resources that are never used)
  const auto ro = part_rsrc(single ? nullptr : a.part_o + qrow0 * ns * 2 * D,
                            single ? 0u : (unsigned)(nvh * ns * 2 * D * 4));
  const auto rml = part_rsrc(single ? nullptr : a.part_ml + qrow0 * ns * 2,
                             single ? 0u : (unsigned)(nvh * ns * 2 * 4));
  for (int it = threadIdx.x; it < nvh * C4; it += NW * 64) {
    const int g = it / C4;
    const int c = (it % C4) * 4;
    float M = kNegSentinel;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, lds_m[w][g]);
    float L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = fast_exp2(lds_m[w][g] - M);
      L = fmaf(lds_l[w][g], f, L);
      const float4 v = *reinterpret_cast<const float4*>(&lds_o[w][g][c]);
      O.x = fmaf(v.x, f, O.x);
      O.y = fmaf(v.y, f, O.y);
      O.z = fmaf(v.z, f, O.z);
      O.w = fmaf(v.w, f, O.w);
    }
    if (single) {
      store_y4<T, D>(a, (qrow0 + g) * 2 * D + c, O, L);
    } else if (!PARTIALS && a.fused_merge) {
      store_through4(ro, (unsigned)(((g * ns + split) * 2 * D + c) * 4), O);
      if (c == 0) store_through2(rml, (unsigned)((g * ns + split) * 8), make_float2(M, L));
    } else {  // read by the merge launch: the kernel boundary publishes them
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, O), ro,
                                             (unsigned)(((g * ns + split) * 2 * D + c) * 4), 0, 0);
      if (c == 0)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, make_float2(M, L)), rml,
                                              (unsigned)((g * ns + split) * 8), 0, 0);
    }
  }
  if constexpr (PARTIALS || !FUSED_MERGE) {
    return;  // a merge launch combines the splits
  } else {
    if (single || !a.fused_merge) return;

    // ---- last workgroup of this (b, KV head, chunk) combines all splits.
    __shared__ int is_last;
    wait_stores_done();
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned t = __hip_atomic_fetch_add(&a.counters[unit], 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_SYSTEM);
      is_last = (t == (unsigned)(a.nsplit - 1));
      if (is_last)  // re-arm for the next call
        __hip_atomic_store(&a.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    if (!is_last) return;
    merge_splits<T, D, GC, NW>(a, qrow0, nvh);
  }
}

// ------------------------------------------------------- merge kernel ---
// Second launch of a split call: combines the nsplit partials of every
// virtual-head row.  One wave per (row, slice of CW float4 output columns),
// no LDS and no barrier: lane (column, group) sums the splits group,
// group + NGR, ...; the row max M and total L come from lane-strided loads
// of the (m, l) pairs and wave reductions, and each lane reads the m of its
// own splits to form its factors exp2(m_s - M).  Every load of a batch is
// issued before any is consumed.  The kernel boundary makes the attention
// launch's partials visible, so plain loads suffice.
template <int D>
struct MergeShape {
  static constexpr int C4 = 2 * D / 4;          // float4 columns of one output row
  static constexpr int CW = C4 < 16 ? C4 : 16;  // columns per wave
  static constexpr int NSL = C4 / CW;           // waves per row
  static constexpr int NGR = 64 / CW;           // split groups
  static constexpr int UNR = 8;                 // partial loads in flight per lane
};

// Unnormalised merged accumulator of float4 column col of partial row vrow
// (every lane of the column gets it) and the row's total L.
// Loads of one partial row for merge_row_column, issued before any is
// consumed (merge_row_column_issue), so that a caller merging several rows
// issues all of their loads in one round trip.  They go through buffer
// resources over the row's ns splits: loads past them return 0 with no
// branch (a branch per load made the compiler wait on loads in flight), and
// merge_row_column_finish masks those splits.
template <int D>
struct MergeColumnLoads {
  float4 v[MergeShape<D>::UNR];
  float mj[MergeShape<D>::UNR];
  float2 ml[kMaxSplits / 64];
};

template <int D>
__device__ inline void merge_load_batch(const SdpaArgs& a, long vrow, int col, int lane, int s0,
                                        MergeColumnLoads<D>& ld) {
  using S = MergeShape<D>;
  const int grp = lane / S::CW;
  const int ns = a.nsplit;
  const auto ro = part_rsrc(a.part_o + vrow * ns * 2 * D, (unsigned)(ns * 2 * D * 4));
  const auto rml = part_rsrc(a.part_ml + vrow * ns * 2, (unsigned)(ns * 2 * 4));
#pragma unroll
  for (int j = 0; j < S::UNR; ++j) {
    const unsigned s = (unsigned)(s0 + grp + j * S::NGR);
    ld.v[j] = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(ro, (s * 2 * D + col * 4) * 4u, 0, 0));
    ld.mj[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rml, s * 8u, 0, 0));
  }
}

// (m, l) of splits lane, lane + 64, ... and the first batch together.
template <int D>
__device__ inline void merge_row_column_issue(const SdpaArgs& a, long vrow, int col, int lane,
                                              MergeColumnLoads<D>& ld) {
  const int ns = a.nsplit;
  const auto rml = part_rsrc(a.part_ml + vrow * ns * 2, (unsigned)(ns * 2 * 4));
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i)
    ld.ml[i] = __builtin_bit_cast(
        float2, __builtin_amdgcn_raw_buffer_load_b64(rml, (unsigned)(lane + 64 * i) * 8u, 0, 0));
  merge_load_batch<D>(a, vrow, col, lane, 0, ld);
  // Keep the loads here: the scheduler would otherwise sink the batch below
  // the wait for the (m, l) pairs, a second round trip.
  __builtin_amdgcn_sched_barrier(0);
}

// Unnormalised merged accumulator of float4 column col of partial row vrow
// (every lane of the column gets it) and the row's total L, from the loads
// merge_row_column_issue started.
template <int D>
__device__ inline float4 merge_row_column_finish(const SdpaArgs& a, long vrow, int col, int lane,
                                                 MergeColumnLoads<D>& ld, float& L_out) {
  using S = MergeShape<D>;
  const int ns = a.nsplit;
  const int grp = lane / S::CW;
  float mi[kMaxSplits / 64];  // m of split lane + 64 i, the sentinel past ns
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) mi[i] = lane + 64 * i < ns ? ld.ml[i].x : kNegSentinel;
  float M = kNegSentinel;
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) M = fmaxf(M, mi[i]);
  M = group_max<64>(M);
  float L = 0.f;  // (l past ns reads 0)
#pragma unroll
  for (int i = 0; i < kMaxSplits / 64; ++i) L = fmaf(ld.ml[i].y, fast_exp2(mi[i] - M), L);
  L_out = group_sum<64>(L);

  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += S::NGR * S::UNR) {
    if (s0 > 0) merge_load_batch<D>(a, vrow, col, lane, s0, ld);
#pragma unroll
    for (int j = 0; j < S::UNR; ++j) {
      // 0 for splits past ns (their m is replaced by the sentinel; o reads 0)
      const float mjv = s0 + grp + j * S::NGR < ns ? ld.mj[j] : kNegSentinel;
      const float f = fast_exp2(mjv - M);
      acc.x = fmaf(ld.v[j].x, f, acc.x);
      acc.y = fmaf(ld.v[j].y, f, acc.y);
      acc.z = fmaf(ld.v[j].z, f, acc.z);
      acc.w = fmaf(ld.v[j].w, f, acc.w);
    }
  }
  // Sum the NGR split groups of each column (lanes col, col + CW, ...).
#pragma unroll
  for (int off = S::CW; off < 64; off *= 2) {
    acc.x += __shfl_xor(acc.x, off);
    acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off);
    acc.w += __shfl_xor(acc.w, off);
  }
  return acc;
}

// Unnormalised merged accumulator of float4 column col of partial row vrow
// (every lane of the column gets it) and the row's total L.
template <int D>
__device__ inline float4 merge_row_column(const SdpaArgs& a, long vrow, int col, int lane,
                                          float& L_out) {
  MergeColumnLoads<D> ld;
  merge_row_column_issue<D>(a, vrow, col, lane, ld);
  return merge_row_column_finish<D>(a, vrow, col, lane, ld, L_out);
}

// Merge block -> (virtual row, slice of NSL).  With one head chunk per KV
// head (decode), the attention workgroups of unit u = (b, KV head) were
// dispatched to XCD u % 8 (round-robin over the 8 XCDs), where their
// partials were written; the merge blocks of u's rows take the same residue,
// block = 8 k + u % 8.  Placement affects speed only.
__device__ inline bool merge_block_coords(const SdpaArgs& a, int bid, int nsl, int rows_per_unit,
                                          long& vrow, int& slice) {
  if (a.nchunk != 1) {
    vrow = bid / nsl;
    slice = bid % nsl;
    return true;
  }
  const int per_unit = rows_per_unit * nsl;
  const int k = bid >> 3;
  const int u = (k / per_unit) * 8 + (bid & 7);
  if (u >= a.B * a.Hkv) return false;  // padding of the last group of 8
  const int rem = k % per_unit;
  vrow = (long)u * rows_per_unit + rem / nsl;
  slice = rem % nsl;
  return true;
}

inline unsigned merge_grid_blocks(const SdpaArgs& a, int nsl, long rows, int rows_per_unit) {
  if (a.nchunk != 1) return (unsigned)(rows * nsl);
  const int bh = a.B * a.Hkv;
  return (unsigned)((bh + 7) / 8 * 8 * rows_per_unit * nsl);
}

template <typename T, int D>
__global__ void __launch_bounds__(64) sdpa_merge_kernel(SdpaArgs a) {
  using S = MergeShape<D>;
  const int lane = threadIdx.x;
  long vrow;
  int slice;
  if (!merge_block_coords(a, blockIdx.x, S::NSL, a.G * a.S_q, vrow, slice)) return;
  const int col = slice * S::CW + lane % S::CW;
  float L;
  const float4 acc = merge_row_column<D>(a, vrow, col, lane, L);
  if (lane < S::CW) {
    if (a.y2 != nullptr && vrow >= a.y2_row0)  // second output (fused prefill's noise pass)
      store_y4_to<T, D>(a.y2, (vrow - a.y2_row0) * 2 * D + col * 4, acc, L);
    else
      store_y4<T, D>(a, vrow * 2 * D + col * 4, acc, L);
  }
}

// Merge launch for many partial rows (prefill chunks, long slabs split over
// few workgroups each): one wave per row, lane c holding float4 columns c,
// c + 64, .. of the row's 2D channels, four rows per workgroup.  The
// one-wave workgroups of sdpa_merge_kernel are capped by how many
// workgroups a CU holds at once (16384 rows x 4 slices of a 512-row chunk
// took ~24 us for 34 MB); here the splits are taken in batches of 8 with
// every load of a batch issued before any is consumed, and the running
// maximum rescales earlier batches.  With at most 8 splits the result is
// sum_s o_s * exp2(m_s - M) in split order, M the largest m_s.
// F16: the partials are fp16 o / l (SdpaArgs::part_f16); split s then weighs
// l_s * exp2(m_s - M) instead of exp2(m_s - M).
template <typename T, int D, bool F16>
__device__ inline void merge_rows(const SdpaArgs& a, long vrow, int lane) {
  constexpr int C4 = 2 * D / 4;
  constexpr int CPL = (C4 + 63) / 64;  // float4 columns per lane
  constexpr int NB = 8;                // splits per batch
  const int ns = a.nsplit;
  const float4* po = reinterpret_cast<const float4*>(a.part_o + vrow * ns * 2 * D);
  const uint2* ph = reinterpret_cast<const uint2*>((const uint16_t*)a.part_o + vrow * ns * 2 * D);
  const float2* pml = reinterpret_cast<const float2*>(a.part_ml + vrow * ns * 2);
  float4 acc[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  float M = kNegSentinel, L = 0.f;
  for (int s0 = 0; s0 < ns; s0 += NB) {
    // Every load of the batch is issued before any is consumed: the split
    // and column indices are clamped to valid ones (no branch per load, at
    // which the compiler would wait on loads in flight) and the splits past
    // ns and columns past C4 are masked afterwards.
    float2 mlr[NB];
    float4 vr[NB][CPL];
    uint2 hr[NB][CPL];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int sc = min(s0 + j, ns - 1);
      mlr[j] = pml[sc];
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const int cc = min(lane + 64 * k, C4 - 1);
        if constexpr (F16)
          hr[j][k] = ph[(long)sc * C4 + cc];
        else
          vr[j][k] = po[(long)sc * C4 + cc];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float2 ml[NB];
    float4 v[NB][CPL];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int s = s0 + j;
      ml[j] = s < ns ? mlr[j] : make_float2(kNegSentinel, 0.f);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const bool in = s < ns && lane + 64 * k < C4;
        if constexpr (F16)
          v[j][k] = in ? half4_floats(hr[j][k]) : make_float4(0.f, 0.f, 0.f, 0.f);
        else
          v[j][k] = in ? vr[j][k] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float Mb = M;
#pragma unroll
    for (int j = 0; j < NB; ++j) Mb = fmaxf(Mb, ml[j].x);
    if (s0 > 0) {
      const float r = fast_exp2(M - Mb);
      L *= r;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        acc[k].x *= r;
        acc[k].y *= r;
        acc[k].z *= r;
        acc[k].w *= r;
      }
    }
    M = Mb;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float e = fast_exp2(ml[j].x - M);  // 0 for splits past ns (sentinel m)
      L = fmaf(ml[j].y, e, L);
      const float f = F16 ? ml[j].y * e : e;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        acc[k].x = fmaf(v[j][k].x, f, acc[k].x);
        acc[k].y = fmaf(v[j][k].y, f, acc[k].y);
        acc[k].z = fmaf(v[j][k].z, f, acc[k].z);
        acc[k].w = fmaf(v[j][k].w, f, acc[k].w);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + 64 * k;
    if (c >= C4) continue;
    if (a.y2 != nullptr && vrow >= a.y2_row0)  // second output (fused prefill's noise pass)
      store_y4_to<T, D>(a.y2, (vrow - a.y2_row0) * 2 * D + c * 4, acc[k], L);
    else
      store_y4<T, D>(a, vrow * 2 * D + c * 4, acc[k], L);
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(256) sdpa_merge_rows_kernel(SdpaArgs a, long rows) {
  const int lane = threadIdx.x & 63;
  const long vrow = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (vrow >= rows) return;
  if (a.part_f16)
    merge_rows<T, D, true>(a, vrow, lane);
  else
    merge_rows<T, D, false>(a, vrow, lane);
}

// fp16 partials with 16-byte loads (D with 2D/8 dividing 64; other D take
// merge_rows<T, D, true>): lane (r, c) of a wave merges 8
// channels c*8 .. c*8 + 7 of row vrow0 + r, 64 / (2D/8) rows per wave, with
// the same per-element operations as merge_rows<T, D, true> (bit-identical
// results).
template <typename T, int D>
__global__ void __launch_bounds__(256) sdpa_merge_rows16_kernel(SdpaArgs a, long rows) {
  constexpr int C8 = 2 * D / 8;  // 16-byte chunks of a partial row
  static_assert(64 % C8 == 0, "whole rows per wave");
  constexpr int RPW = 64 / C8;
  constexpr int NB = 8;  // splits per batch
  const int lane = threadIdx.x & 63;
  const long vrow = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / C8;
  const int c = lane % C8;
  if (vrow >= rows) return;  // no cross-lane operations below
  const int ns = a.nsplit;
  const uint4* ph = reinterpret_cast<const uint4*>((const uint16_t*)a.part_o + vrow * ns * 2 * D);
  const float2* pml = reinterpret_cast<const float2*>(a.part_ml + vrow * ns * 2);
  float4 acc[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  float M = kNegSentinel, L = 0.f;
  for (int s0 = 0; s0 < ns; s0 += NB) {
    // All loads first, at clamped split indices, then the masks (as in
    // merge_rows).
    float2 mlr[NB];
    uint4 wr[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int sc = min(s0 + j, ns - 1);
      mlr[j] = pml[sc];
      wr[j] = ph[(long)sc * C8 + c];
    }
    __builtin_amdgcn_sched_barrier(0);
    float2 ml[NB];
    float4 v[NB][2];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const bool in = s0 + j < ns;
      ml[j] = in ? mlr[j] : make_float2(kNegSentinel, 0.f);
      const uint4 w = in ? wr[j] : make_uint4(0, 0, 0, 0);
      v[j][0] = half4_floats(make_uint2(w.x, w.y));
      v[j][1] = half4_floats(make_uint2(w.z, w.w));
    }
    float Mb = M;
#pragma unroll
    for (int j = 0; j < NB; ++j) Mb = fmaxf(Mb, ml[j].x);
    if (s0 > 0) {
      const float r = fast_exp2(M - Mb);
      L *= r;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        acc[k].x *= r;
        acc[k].y *= r;
        acc[k].z *= r;
        acc[k].w *= r;
      }
    }
    M = Mb;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float e = fast_exp2(ml[j].x - M);  // 0 for splits past ns (sentinel m)
      L = fmaf(ml[j].y, e, L);
      const float f = ml[j].y * e;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        acc[k].x = fmaf(v[j][k].x, f, acc[k].x);
        acc[k].y = fmaf(v[j][k].y, f, acc[k].y);
        acc[k].z = fmaf(v[j][k].z, f, acc[k].z);
        acc[k].w = fmaf(v[j][k].w, f, acc[k].w);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (a.y2 != nullptr && vrow >= a.y2_row0)  // second output (fused prefill's noise pass)
      store_y4_to<T, D>(a.y2, (vrow - a.y2_row0) * 2 * D + c * 8 + 4 * k, acc[k], L);
    else
      store_y4<T, D>(a, vrow * 2 * D + c * 8 + 4 * k, acc[k], L);
  }
}

// The merge launch takes the row-per-wave kernel for this call (many partial
// rows, or fp16 partials, which only that kernel reads).
inline bool merge_uses_rows_kernel(const SdpaArgs& a) {
  return a.part_f16 || ((long)a.B * a.Hq * a.S_q >= kMergeRowsMin && tuning().merge_rows);
}

template <typename T, int D>
int launch_sdpa_merge_d(const SdpaArgs& a, hipStream_t s) {
  constexpr int C4 = 2 * D / 4;
  constexpr int NSL = C4 / (C4 < 16 ? C4 : 16);
  const long rows = (long)a.B * a.Hq * a.S_q;
  if constexpr (64 % (2 * D / 8) == 0) {
    // fp16 partials: 16-byte loads, whole rows per wave (prefill chunk of
    // 512 rows over 3716: 69.6 against 71.5-75.8 us per call with the
    // 8-byte row-per-wave kernel; 256 over 3204: 43.7-44.0 against 45.5-48.0)
    if (a.part_f16) {
      constexpr long rpb = 4 * (64 / (2 * D / 8));  // rows per 4-wave block
      hipLaunchKernelGGL((sdpa_merge_rows16_kernel<T, D>), dim3((unsigned)((rows + rpb - 1) / rpb)),
                         dim3(256), 0, s, a, rows);
      return check_launch("sdpa split merge (rows, 16-byte)");
    }
  }
  if (merge_uses_rows_kernel(a)) {
    hipLaunchKernelGGL((sdpa_merge_rows_kernel<T, D>), dim3((unsigned)((rows + 3) / 4)), dim3(256),
                       0, s, a, rows);
    return check_launch("sdpa split merge (rows)");
  }
  hipLaunchKernelGGL((sdpa_merge_kernel<T, D>), dim3(merge_grid_blocks(a, NSL, rows, a.G * a.S_q)),
                     dim3(64), 0, s, a);
  return check_launch("sdpa split merge");
}

// --------------------------------------------- fused GDA decode merge ---
// Second launch of a fused GDA decode step (origin and noise passes share
// one attention launch): one workgroup per origin row (b, h) merges the
// splits of that row and of its noise head h / gr, rounds both to T (the
// reference's attention outputs are T tensors), and applies gda_post_split
// (src/mlx_motif/kernels/gda.py:131-192):
//   d = o - lambda * n,  y = T(d * rsqrt(mean(d^2) + eps) * w * (1 - lambda_init)).
// Wave w of the NSL waves holds float4 columns [w*CW, (w+1)*CW) of the 2D
// channels; the sum of squares meets in LDS.
template <typename T, int D>
__global__ void __launch_bounds__(MergeShape<D>::NSL * 64) gda_decode_merge_kernel(SdpaArgs a) {
  using S = MergeShape<D>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  long orow;  // (b, h) over B * Hq
  int unused_slice;
  if (!merge_block_coords(a, blockIdx.x, 1, a.G, orow, unused_slice)) return;
  const long b = orow / a.Hq;
  const int h = (int)(orow - b * a.Hq);
  const int j = h / a.G;  // KV head
  const int i = h - j * a.G;  // origin column within it
  // Partial rows of KV head j: G origin columns, then G2 noise columns;
  // origin head h pairs with noise head h / gr (gr = G / G2), column
  // G + i / gr of the same KV head.
  const long prow0 = (b * a.Hkv + j) * (a.G + a.G2);
  const long orow_p = prow0 + i;
  const long nrow_p = prow0 + a.G + i / (a.G / a.G2);
  const int col = wave * S::CW + lane % S::CW;
  const bool head_lane = lane < S::CW;  // one lane per column stores

  // Both rows' loads (and lambda's) are in flight before either is consumed.
  MergeColumnLoads<D> lo, ln;
  merge_row_column_issue<D>(a, orow_p, col, lane, lo);
  merge_row_column_issue<D>(a, nrow_p, col, lane, ln);
  const float lam = *a.gda_lambda;
  float wv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) wv[e] = Elem<T>::load(a.gda_w, col * 4 + e);
  float Lo, Ln;
  const float4 ao = merge_row_column_finish<D>(a, orow_p, col, lane, lo, Lo);
  const float4 an = merge_row_column_finish<D>(a, nrow_p, col, lane, ln, Ln);
  auto out_t = [](float v, float L) {  // o / l rounded to T (o when l == 0)
    const float x = L == 0.f ? v : v / L;
    if constexpr (Elem<T>::kBytes == 2) return Elem<T>::to_f32(Elem<T>::from_f32(x));
    return x;
  };
  const float o4[4] = {out_t(ao.x, Lo), out_t(ao.y, Lo), out_t(ao.z, Lo), out_t(ao.w, Lo)};
  const float n4[4] = {out_t(an.x, Ln), out_t(an.y, Ln), out_t(an.z, Ln), out_t(an.w, Ln)};
  float d[4];
  float ssq = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    d[e] = o4[e] - lam * n4[e];
    ssq = fmaf(d[e], d[e], ssq);
  }
  ssq = group_sum<64>(head_lane ? ssq : 0.f);
  __shared__ float lds_ss[S::NSL];
  if (lane == 0) lds_ss[wave] = ssq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < S::NSL; ++w) tot += lds_ss[w];
  const float rms_inv = rsqrtf(tot / (float)(2 * D) + a.gda_eps);
  if (!head_lane) return;
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    y[e] = d[e] * rms_inv * wv[e] * a.gda_scale;
  const long off = orow * 2 * D + col * 4;
  if constexpr (Elem<T>::kBytes == 2) {
    *reinterpret_cast<uint2*>((uint16_t*)a.y + off) = make_uint2(
        (uint32_t)Elem<T>::from_f32(y[0]) | ((uint32_t)Elem<T>::from_f32(y[1]) << 16),
        (uint32_t)Elem<T>::from_f32(y[2]) | ((uint32_t)Elem<T>::from_f32(y[3]) << 16));
  } else {
    *reinterpret_cast<float4*>((float*)a.y + off) = make_float4(y[0], y[1], y[2], y[3]);
  }
}

template <typename T, int D>
int launch_gda_decode_merge_d(const SdpaArgs& a, hipStream_t s) {
  const long rows = (long)a.B * a.Hq;
  hipLaunchKernelGGL((gda_decode_merge_kernel<T, D>), dim3(merge_grid_blocks(a, 1, rows, a.G)),
                     dim3(MergeShape<D>::NSL * 64), 0, s, a);
  return check_launch("gda decode merge");
}

// ---------------------------------------------------------------- kernel --
template <class Fmt, int GC, int NW, int U>
__global__ void __launch_bounds__(NW * 64) sdpa_dual_v_kernel(SdpaArgs a) {
  using T = typename Fmt::T;
  constexpr int D = Fmt::D;
  constexpr int LPR = Fmt::LPR;
  constexpr int CPL = Fmt::CPL;
  constexpr int RG = 64 / LPR;  // rows per wave per load
  using Frag = typename Fmt::Frag;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPR;
  const int rg = lane / LPR;

  // Consecutive workgroup ids walk (b, KV head, chunk) first, so all splits
  // of one KV head share an id residue (and the XCD round-robin puts them on
  // one XCD, whose L2 then serves the final merge).
  int unit, split;
  if (!sdpa_block_coords(a, blockIdx.x, unit, split)) return;  // grid padding
  const int chunk = unit % a.nchunk;
  const int bk = unit / a.nchunk;  // b * Hkv + kv head
  const int b = bk / a.Hkv;
  const int kvh = bk % a.Hkv;

  const int vh0 = chunk * GC;
  const int nvh = min(GC, a.GV - vh0);
  // Query/output rows of virtual heads vh0.. are contiguous: (b, head, s).
  const long qrow0 = ((long)b * a.Hq + (long)kvh * a.G) * a.S_q + vh0;

  float qf[GC][CPL];
  int lim[GC];
  int max_lim = 0;
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    if (g < nvh) {
#pragma unroll
      for (int e = 0; e < CPL; ++e)
        qf[g][e] = a.qscale * Elem<T>::load(a.q, (qrow0 + g) * D + sub * CPL + e);
      int s = (vh0 + g) % a.S_q;
      int L = a.causal ? a.kv_len - a.S_q + s + 1 : a.kv_len;
      L = L < 0 ? 0 : (L > a.kv_len ? a.kv_len : L);
      lim[g] = L;
      max_lim = max(max_lim, L);
    } else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) qf[g][e] = 0.f;
      lim[g] = 0;
    }
  }

  const int r_begin = split * a.rows_per_split;
  const int r_end = min(r_begin + a.rows_per_split, max_lim);

  Fmt fmt(a, bk, sub);

  float m[GC], l[GC], o1[GC][CPL], o2[GC][CPL];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = kNegSentinel;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) { o1[g][e] = 0.f; o2[g][e] = 0.f; }
  }

  for (int base = r_begin + wave * RG; base < r_end; base += NW * RG * U) {
    Frag kf[U], v1f[U], v2f[U];
    int row[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      row[u] = base + u * NW * RG + rg;
      if (row[u] < r_end) {
        fmt.load(row[u], kf[u], v1f[u], v2f[u]);
      } else {
        Fmt::zero(kf[u]); Fmt::zero(v1f[u]); Fmt::zero(v2f[u]);
      }
    }

    float s[U][GC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kx[CPL];
      Fmt::values(kf[u], kx);
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < CPL; ++e) acc = fmaf(qf[g][e], kx[e], acc);
        acc = group_sum<LPR>(acc);
        bool ok = row[u] < r_end && row[u] < lim[g];
        s[u][g] = ok ? acc : kNegSentinel;
      }
    }

    float p[U][GC];
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][g]);
      // Rescale only when some row group's max moved (wave-uniform branch).
      if (__ballot(mx > m[g]) != 0) {
        float fac = fast_exp2(m[g] - mx);
        l[g] *= fac;
#pragma unroll
        for (int e = 0; e < CPL; ++e) { o1[g][e] *= fac; o2[g][e] *= fac; }
        m[g] = mx;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u][g] = (s[u][g] > kNegSentinel) ? fast_exp2(s[u][g] - mx) : 0.f;
        l[g] += p[u][g];
      }
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x1[CPL], x2[CPL];
      Fmt::values(v1f[u], x1);
      Fmt::values(v2f[u], x2);
#pragma unroll
      for (int g = 0; g < GC; ++g) {
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          o1[g][e] = fmaf(p[u][g], x1[e], o1[g][e]);
          o2[g][e] = fmaf(p[u][g], x2[e], o2[g][e]);
        }
      }
    }
  }

  // ---- merge the RG row groups of this wave (lanes sharing `sub`).
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    float M = m[g];
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) M = fmaxf(M, __shfl_xor(M, off));
    float f = fast_exp2(m[g] - M);
    float L = l[g] * f;
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) L += __shfl_xor(L, off);
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      float x = o1[g][e] * f, z = o2[g][e] * f;
#pragma unroll
      for (int off = LPR; off < 64; off *= 2) {
        x += __shfl_xor(x, off);
        z += __shfl_xor(z, off);
      }
      o1[g][e] = x;
      o2[g][e] = z;
    }
    m[g] = M;
    l[g] = L;
  }

  // ---- hand the wave results to the shared epilogue through LDS.
  __shared__ __attribute__((aligned(16))) float lds_o[NW][GC][2 * D + kLdsPad];
  __shared__ float lds_m[NW][GC];
  __shared__ float lds_l[NW][GC];
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        lds_o[wave][g][sub * CPL + e] = o1[g][e];
        lds_o[wave][g][D + sub * CPL + e] = o2[g][e];
      }
      if (sub == 0) {
        lds_m[wave][g] = m[g];
        lds_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();
  wg_epilogue<T, D, GC, NW>(a, lds_o, lds_m, lds_l, qrow0, nvh, split, unit);
}

// Host launcher for one format.
template <class Fmt, int GC>
int launch_sdpa(const SdpaArgs& a, int waves, int nblocks, hipStream_t stream) {
  constexpr int U = Fmt::CPL <= 8 ? 4 : 2;
  if constexpr (Fmt::D * GC <= 512) {
    if (waves == 8) {
      hipLaunchKernelGGL((sdpa_dual_v_kernel<Fmt, GC, 8, U>), dim3(nblocks), dim3(8 * 64), 0,
                         stream, a);
      return check_launch("sdpa_dual_v");
    }
  }
  hipLaunchKernelGGL((sdpa_dual_v_kernel<Fmt, GC, 4, U>), dim3(nblocks), dim3(4 * 64), 0,
                     stream, a);
  return check_launch("sdpa_dual_v");
}

template <class Fmt>
int launch_sdpa_gc(const SdpaArgs& a, int gc, int waves, int nblocks, hipStream_t stream) {
  switch (gc) {
    case 1: return launch_sdpa<Fmt, 1>(a, waves, nblocks, stream);
    case 2: return launch_sdpa<Fmt, 2>(a, waves, nblocks, stream);
    case 4: return launch_sdpa<Fmt, 4>(a, waves, nblocks, stream);
    case 8:
      if constexpr (Fmt::CPL <= 8) return launch_sdpa<Fmt, 8>(a, waves, nblocks, stream);
      break;
    default: break;
  }
  set_error("sdpa_dual_v: no variant for %d heads per workgroup", gc);
  return MOTIF_ERR_UNSUPPORTED;
}

}  // namespace motif
