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
// then splits: every workgroup writes (m, l, o1, o2) to the workspace and the
// last one to arrive for its (b, KV head, chunk) combines all splits and
// writes y, then re-arms the arrival counter.
//
// Reference semantics (src/mlx_motif/kernels/attention.py:53-166, 293-445):
// q scaled once in fp32, fp32 accumulation, running-max sentinel -1e30,
// output o/l with o left unnormalised (zero) when l == 0.
#pragma once

#include "motif_common.hpp"
#include "sdpa_plan.hpp"

namespace motif {

constexpr float kNegSentinel = -1e30f;

// Cross-workgroup hand-off of split partials without whole-cache maintenance.
// Partials are stored and re-loaded with system-scope relaxed atomics, which
// gfx950 issues with sc0 sc1: stores are written through the XCD's L2 to
// memory, loads miss in L1/L2 and read memory.  A writer waits for all its
// stores to complete (s_waitcnt 0) before it takes an arrival ticket, so
// the workgroup that takes the last ticket reads complete partials.  (An
// agent-scope __threadfence() here costs a buffer_wbl2 + buffer_inv of the
// whole L2 per workgroup, which serialises per XCD.)
__device__ inline void store_through(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ inline float load_through(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ inline void wait_stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // keep the compiler from moving memory ops
  __builtin_amdgcn_s_waitcnt(0);             // vmcnt = expcnt = lgkmcnt = 0
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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
    load_words<WPL>(kf.w, k + o);
    load_words<WPL>(v1f.w, v1 + o);
    load_words<WPL>(v2f.w, v2 + o);
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
    load_words<WPL>(kf.w, kd + o);
    load_words<WPL>(v1f.w, v1d + o);
    load_words<WPL>(v2f.w, v2d + o);
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

// ------------------------------------------------------- split merge ---
// Combine the nsplit partials (m, l, o1, o2) of virtual heads qrow0 ..
// qrow0+nvh-1 and write y.  Every load of a phase is independent of the
// others so they are in flight together: (m, l) pairs go to LDS, one wave
// per head turns them into factors exp2(m_s - M) and the total L, then each
// output float4 is summed over its splits by P threads with 16 loads in
// flight each, and the P partial sums meet in LDS.
template <typename T, int D, int GC, int NW>
__device__ void merge_splits(const SdpaArgs& a, long qrow0, int nvh) {
  constexpr int NT = NW * 64;
  constexpr int C4 = 2 * D / 4;
  constexpr int UNR = 16;
  __shared__ float lds_f[GC][kMaxSplits];  // m_s, then exp2(m_s - M)
  __shared__ float lds_l[GC][kMaxSplits];
  __shared__ float lds_L[GC];
  __shared__ float4 lds_acc[NT];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ns = a.nsplit;

  for (int i = tid; i < nvh * ns; i += NT) {
    const int g = i / ns, s = i % ns;
    const float* ml = a.part_ml + ((qrow0 + g) * ns + s) * 2;
    lds_f[g][s] = load_through(ml);
    lds_l[g][s] = load_through(ml + 1);
  }
  __syncthreads();
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

  const int items = nvh * C4;
  const int P = items >= NT ? 1 : NT / items;  // threads per output float4
  for (int base = 0; base < items; base += NT) {
    const int idx = base + tid;
    const int item = P == 1 ? idx : tid % items;
    const int part = P == 1 ? 0 : tid / items;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const bool active = item < items && part < P;
    if (active) {
      const int g = item / C4;
      const int c = (item % C4) * 4;
      const float* po = a.part_o + (qrow0 + g) * ns * 2 * D + c;
      for (int s0 = part; s0 < ns; s0 += P * UNR) {
        float4 v[UNR];
        float f[UNR];
#pragma unroll
        for (int j = 0; j < UNR; ++j) {
          const int s = s0 + j * P;
          if (s < ns) {
            const float* src = po + (long)s * 2 * D;
            v[j] = make_float4(load_through(src), load_through(src + 1), load_through(src + 2),
                               load_through(src + 3));
            f[j] = lds_f[g][s];
          } else {
            v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            f[j] = 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < UNR; ++j) {
          acc.x = fmaf(v[j].x, f[j], acc.x);
          acc.y = fmaf(v[j].y, f[j], acc.y);
          acc.z = fmaf(v[j].z, f[j], acc.z);
          acc.w = fmaf(v[j].w, f[j], acc.w);
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
        acc = t;
      }
    }
    const int out_item = P == 1 ? idx : tid;
    if (out_item < items && (P == 1 || tid < items)) {
      const int g = out_item / C4;
      const int c = (out_item % C4) * 4;
      const float L = lds_L[g];
      const bool zero_l = L == 0.f;
      const long yo = (qrow0 + g) * 2 * D + c;
      Elem<T>::store(a.y, yo + 0, zero_l ? acc.x : acc.x / L);
      Elem<T>::store(a.y, yo + 1, zero_l ? acc.y : acc.y / L);
      Elem<T>::store(a.y, yo + 2, zero_l ? acc.z : acc.z / L);
      Elem<T>::store(a.y, yo + 3, zero_l ? acc.w : acc.w / L);
    }
    if (P > 1) break;  // items < NT: a single pass covers every item
  }
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
  const int units = a.B * a.Hkv * a.nchunk;
  const int unit = blockIdx.x % units;
  const int split = blockIdx.x / units;
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

  // ---- merge the NW waves through LDS.
  __shared__ float lds_o[NW][GC][2 * D];
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

  const bool single = a.nsplit == 1;
  for (int idx = threadIdx.x; idx < nvh * 2 * D; idx += NW * 64) {
    const int g = idx / (2 * D);
    const int c = idx % (2 * D);
    float M = kNegSentinel;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, lds_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      float f = fast_exp2(lds_m[w][g] - M);
      L = fmaf(lds_l[w][g], f, L);
      O = fmaf(lds_o[w][g][c], f, O);
    }
    const long r = qrow0 + g;
    if (single) {
      Elem<T>::store(a.y, r * 2 * D + c, L == 0.f ? O : O / L);
    } else {
      store_through(a.part_o + (r * a.nsplit + split) * 2 * D + c, O);
      if (c == 0) {
        store_through(a.part_ml + (r * a.nsplit + split) * 2, M);
        store_through(a.part_ml + (r * a.nsplit + split) * 2 + 1, L);
      }
    }
  }
  if (single) return;

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
