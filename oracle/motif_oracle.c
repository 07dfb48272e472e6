/*
 * C restatement of the Motif decode-attention hot path for the CPU.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a second, independent
 * restatement checked against oracle/oracle.py, and by bench.py's
 * cpu_baseline leg as the timed CPU port (OpenMP over query rows).  The
 * product never links or calls it.
 *
 * Reference semantics followed (paths in the junhoyeo/mlx-motif tree):
 *   sdpa_dual_v      src/mlx_motif/kernels/attention.py:181-229 — slice to
 *                    kv_len, query head h reads KV head h / (Hq/Hkv),
 *                    y = [softmax(scale q K^T) V1 || softmax(scale q K^T) V2];
 *                    fp32 accumulation like the reference kernel
 *                    (attention.py:53-166); rows with no visible key -> 0.
 *   sdpa_dual_v_q    attention.py:473-507 — same on dequantised K/V1/V2,
 *                    value = scale * code + bias (mlp.py:176-198).
 *   quantize         mx.quantize affine mode as called at cache.py:498, fp32
 *                    arithmetic in the order of oracle/oracle.py:quantize.
 * fp16 is stored as uint16_t and converted with F16C (round to nearest even).
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

int motif_oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Row limits of query row s for a bottom-right causal mask. */
static inline int row_limit(int kv_len, int S_q, int s, int causal) {
  int lim = causal ? kv_len - S_q + s + 1 : kv_len;
  if (lim < 0) lim = 0;
  if (lim > kv_len) lim = kv_len;
  return lim;
}

/* One query row against rows [0, lim) of one KV head.  kvrow(j, buf) fills
 * buf with the dequantised/converted row j of the given tensor. */
typedef void (*row_fn)(const void* ctx, int tensor, long row, float* out);

static void attend_row(const float* qs, int D, int lim, const void* ctx, long row0, row_fn fetch,
                       float* scores, float* krow, float* o1, float* o2, float* y) {
  float m = -INFINITY;
  for (int j = 0; j < lim; ++j) {
    fetch(ctx, 0, row0 + j, krow);
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += qs[d] * krow[d];
    scores[j] = acc;
    if (acc > m) m = acc;
  }
  memset(o1, 0, sizeof(float) * D);
  memset(o2, 0, sizeof(float) * D);
  float l = 0.f;
  for (int j = 0; j < lim; ++j) {
    float p = expf(scores[j] - m);
    l += p;
    fetch(ctx, 1, row0 + j, krow);
    for (int d = 0; d < D; ++d) o1[d] += p * krow[d];
    fetch(ctx, 2, row0 + j, krow);
    for (int d = 0; d < D; ++d) o2[d] += p * krow[d];
  }
  for (int d = 0; d < D; ++d) {
    y[d] = l == 0.f ? o1[d] : o1[d] / l;
    y[D + d] = l == 0.f ? o2[d] : o2[d] / l;
  }
}

typedef struct {
  const uint16_t* t[3];
  int D;
} fp16_ctx;

static void fetch_f16(const void* vctx, int tensor, long row, float* out) {
  const fp16_ctx* c = (const fp16_ctx*)vctx;
  const uint16_t* p = c->t[tensor] + row * c->D;
  for (int d = 0; d < c->D; ++d) out[d] = h2f(p[d]);
}

typedef struct {
  const uint32_t* data[3];
  const uint16_t* scales[3];
  const uint16_t* biases[3];
  int D, bits, gs;
} q_ctx;

static void fetch_q(const void* vctx, int tensor, long row, float* out) {
  const q_ctx* c = (const q_ctx*)vctx;
  const int el = 32 / c->bits;
  const uint32_t mask = (1u << c->bits) - 1u;
  const uint32_t* w = c->data[tensor] + row * (c->D / el);
  const uint16_t* s = c->scales[tensor] + row * (c->D / c->gs);
  const uint16_t* b = c->biases[tensor] + row * (c->D / c->gs);
  for (int d = 0; d < c->D; ++d) {
    uint32_t u = (w[d / el] >> ((d % el) * c->bits)) & mask;
    out[d] = h2f(s[d / c->gs]) * (float)u + h2f(b[d / c->gs]);
  }
}

static void run_rows(int B, int Hq, int Hkv, int S_q, int D, int cap, int kv_len, int causal,
                     float scale, const uint16_t* q, float* y, const void* ctx, row_fn fetch,
                     int nthreads) {
  const int G = Hq / Hkv;
  const long nrows = (long)B * Hq * S_q;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float* scores = (float*)malloc(sizeof(float) * (kv_len > 0 ? kv_len : 1));
    float* buf = (float*)malloc(sizeof(float) * 4 * D);
    float* qs = buf;
    float* krow = buf + D;
    float* o1 = buf + 2 * D;
    float* o2 = buf + 3 * D;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (long r = 0; r < nrows; ++r) {
      const int s = (int)(r % S_q);
      const long bh = r / S_q;
      const int h = (int)(bh % Hq);
      const int b = (int)(bh / Hq);
      const int kvh = h / G;
      for (int d = 0; d < D; ++d) qs[d] = scale * h2f(q[r * D + d]);
      const long row0 = ((long)b * Hkv + kvh) * cap;
      attend_row(qs, D, row_limit(kv_len, S_q, s, causal), ctx, row0, fetch, scores, krow, o1,
                 o2, y + r * 2 * D);
    }
    free(scores);
    free(buf);
  }
}

/* q (B,Hq,S_q,D) fp16, k/v1/v2 (B,Hkv,cap,D) fp16, y (B,Hq,S_q,2D) fp32. */
void motif_oracle_sdpa_dual_v_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v1,
                                  const uint16_t* v2, float* y, int B, int Hq, int Hkv, int S_q,
                                  int D, int cap, int kv_len, int causal, float scale,
                                  int nthreads) {
  fp16_ctx c = {{k, v1, v2}, D};
  run_rows(B, Hq, Hkv, S_q, D, cap, kv_len, causal, scale, q, y, &c, fetch_f16, nthreads);
}

/* Packed cache: data (B,Hkv,cap,D*bits/32) u32, scales/biases (B,Hkv,cap,D/gs) fp16. */
void motif_oracle_sdpa_dual_v_q_f16(const uint16_t* q, const uint32_t* kd, const uint16_t* ks,
                                    const uint16_t* kb, const uint32_t* v1d,
                                    const uint16_t* v1s, const uint16_t* v1b,
                                    const uint32_t* v2d, const uint16_t* v2s,
                                    const uint16_t* v2b, float* y, int B, int Hq, int Hkv,
                                    int S_q, int D, int cap, int kv_len, int causal, int bits,
                                    int gs, float scale, int nthreads) {
  q_ctx c = {{kd, v1d, v2d}, {ks, v1s, v2s}, {kb, v1b, v2b}, D, bits, gs};
  run_rows(B, Hq, Hkv, S_q, D, cap, kv_len, causal, scale, q, y, &c, fetch_q, nthreads);
}

/* MLX affine quantisation of rows x D fp16 values (fp32 arithmetic). */
void motif_oracle_quantize_f16(const uint16_t* x, uint32_t* data, uint16_t* scales,
                               uint16_t* biases, long rows, int D, int bits, int gs) {
  const int el = 32 / bits;
  const float n_bins = (float)((1 << bits) - 1);
  const long ngroups = rows * (D / gs);
  for (long g = 0; g < ngroups; ++g) {
    const uint16_t* w = x + g * gs;
    float mn = h2f(w[0]), mx = mn;
    for (int i = 1; i < gs; ++i) {
      float v = h2f(w[i]);
      mn = v < mn ? v : mn;
      mx = v > mx ? v : mx;
    }
    volatile float span = mx - mn;  /* keep each fp32 step separately rounded */
    float scale = span / n_bins;
    if (scale < 1e-7f) scale = 1e-7f;
    const int side = fabsf(mn) > fabsf(mx);
    scale = side ? scale : -scale;
    const float edge = side ? mn : mx;
    const float q0 = rintf(edge / scale);
    float bias = 0.f;
    if (q0 != 0.f) {
      scale = edge / q0;
      bias = edge;
    }
    uint32_t* out = data + g * (gs / el);
    for (int j = 0; j < gs / el; ++j) {
      uint32_t word = 0;
      for (int k = 0; k < el; ++k) {
        volatile float diff = h2f(w[j * el + k]) - bias;
        float qv = rintf(diff / scale);
        qv = qv < 0.f ? 0.f : (qv > n_bins ? n_bins : qv);
        word |= ((uint32_t)qv) << (k * bits);
      }
      out[j] = word;
    }
    scales[g] = f2h(scale);
    biases[g] = f2h(bias);
  }
}
