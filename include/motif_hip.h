/*
 * motif_hip.h — C ABI of the MI355X (gfx950) decode-attention hot path of
 * junhoyeo/mlx-motif.
 *
 * One ABI serves every host binding: Python (ctypes, mlx-motif_amd/mlx_motif)
 * and a Swift C-module (module map in mlx-motif_amd/swift/).  The signatures
 * hold only plain pointers, integers and floats: no HIP, torch or MLX types.
 *
 * Conventions
 *  - Every device pointer is caller-owned device memory on the current HIP
 *    device; tensors are dense row-major ("row-contiguous") in the shapes
 *    given per function.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Calls only enqueue work; they never synchronise the stream.  A split-KV
 *    attention call enqueues two kernels (attention, then the split merge).
 *  - Return value: MOTIF_OK, or a negative status.  motif_last_error() then
 *    returns a message (thread-local, valid until the next call on the same
 *    thread).  Contract checks run before any HIP call, so a rejected call
 *    touches no device state.
 *  - dtype codes name the element type of q / k / v / y and of quantisation
 *    scales and biases: MOTIF_F16 (IEEE half), MOTIF_BF16, MOTIF_F32.
 *  - Split-KV attention needs a workspace: size it with
 *    motif_sdpa_workspace_bytes().  Its first motif_sdpa_counter_bytes()
 *    bytes are arrival counters that must be zero before the first call;
 *    every call leaves them zero again.  Calls that share one workspace must
 *    be ordered (same stream); concurrent calls need separate workspaces.
 */
#ifndef MOTIF_HIP_H
#define MOTIF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOTIF_ABI_VERSION 1

#define MOTIF_OK 0
#define MOTIF_ERR_CONTRACT (-1)    /* violates the reference kernel contract   */
#define MOTIF_ERR_UNSUPPORTED (-2) /* legal shape with no compiled variant     */
#define MOTIF_ERR_WORKSPACE (-3)   /* workspace missing or too small           */
#define MOTIF_ERR_HIP (-4)         /* HIP runtime error (launch, device query) */
#define MOTIF_ERR_INTERNAL (-5)    /* library plan inconsistency; nothing launched */

#define MOTIF_F16 0
#define MOTIF_BF16 1
#define MOTIF_F32 2

/* Version of this ABI (MOTIF_ABI_VERSION of the build). */
int motif_abi_version(void);

/* Message for the last non-OK status on this thread ("" if none). */
const char* motif_last_error(void);

/* ------------------------------------------------------------------------ *
 * Workspace sizing for the split-KV attention entry points.
 * S_q = query rows per head (1 for decode), kv_len = live KV rows,
 * D = head dim.  Counters come first, then partial results.
 * ------------------------------------------------------------------------ */
size_t motif_sdpa_counter_bytes(int B, int Hq, int Hkv, int S_q);
size_t motif_sdpa_workspace_bytes(int B, int Hq, int Hkv, int S_q, int kv_len, int D);

/* ------------------------------------------------------------------------ *
 * Shared-QK dual-V SDPA over an fp16/bf16/fp32 4-slot cache.
 * Replaces sdpa_dual_v (src/mlx_motif/kernels/attention.py:190-260) and its
 * Metal kernel motif_sdpa_dual_v (attention.py:53-166).
 *
 *   q      (B, Hq, 1, D)          dtype
 *   k,v1,v2 (B, Hkv, kv_cap, D)   dtype, rows >= kv_len never read
 *   y      (B, Hq, 1, 2D)         dtype = [softmax(scale q K^T) V1 || ... V2]
 * Query head h reads KV head h / (Hq/Hkv) (repeat-interleave GQA).
 * kv_len == 0 writes zeros.
 * Contract (reference asserts attention.py:237-243): D % 32 == 0,
 * Hq % Hkv == 0, 0 <= kv_len <= kv_cap.
 * ------------------------------------------------------------------------ */
int motif_sdpa_dual_v(const void* q, const void* k, const void* v1, const void* v2, void* y,
                      int dtype, int B, int Hq, int Hkv, int D, int kv_cap, int kv_len,
                      float scale, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ *
 * motif_sdpa_dual_v without a workspace argument: it allocates nothing.
 * No counterpart in the reference (whose kernels need no workspace); it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split partials and
 * counters live in a static device array of 8 MiB per device (held until
 * the process ends), whose first 64 KiB of counters are cleared by one fill
 * kernel on the device's first call; the partials of every call follow
 * that counter area.  A call needing more (64 KiB + the partial bytes of
 * motif_sdpa_workspace_bytes > 8 MiB, or more than 16384 B*Hq rows)
 * returns MOTIF_ERR_WORKSPACE before touching the GPU.  All calls on one
 * device share the array: calls that may overlap on a device (several
 * streams, or several threads) race, so order them; results equal
 * motif_sdpa_dual_v's bit for bit.
 * ------------------------------------------------------------------------ */
int motif_sdpa_dual_v_noalloc(const void* q, const void* k, const void* v1, const void* v2,
                              void* y, int dtype, int B, int Hq, int Hkv, int D, int kv_cap,
                              int kv_len, float scale, void* stream);

/* ------------------------------------------------------------------------ *
 * Same, reading the packed MLX-affine q4/q8 cache directly.
 * Replaces sdpa_dual_v_q4 (attention.py:510-645) and its Metal kernel
 * motif_sdpa_dual_v_q4 (attention.py:293-445).
 *
 *   *_data   (B, Hkv, kv_cap, D*bits/32) uint32, value i of a row at bits
 *            [(i % (32/bits))*bits, +bits) of word i / (32/bits)
 *   *_scales (B, Hkv, kv_cap, D/group_size) dtype
 *   *_biases (B, Hkv, kv_cap, D/group_size) dtype
 *   dequantised value = scale * u + bias (u unsigned, no zero point).
 * Contract (attention.py:556-608): bits in {4,8}, D % 32 == 0,
 * D % group_size == 0, (32/bits) % (D/32) == 0, group_size % (D/32) == 0,
 * Hq % Hkv == 0, 0 <= kv_len <= kv_cap.
 * MOTIF_BF16 at D = 128 runs on fp16 matrix cores, whose softmax weights
 * carry the V scales in fp16: V scales must stay below 16376 (bits 4) or
 * 1023 (bits 8), i.e. V groups spanning less than ~2.4e5, or the output is
 * not finite (an fp16 cache always holds them; bf16 caches beyond them take
 * motif_set_tuning("mfma", 0)).
 * ------------------------------------------------------------------------ */
int motif_sdpa_dual_v_q(const void* q,
                        const uint32_t* k_data, const void* k_scales, const void* k_biases,
                        const uint32_t* v1_data, const void* v1_scales, const void* v1_biases,
                        const uint32_t* v2_data, const void* v2_scales, const void* v2_biases,
                        void* y, int dtype, int B, int Hq, int Hkv, int D, int kv_cap,
                        int kv_len, int bits, int group_size, float scale, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ *
 * Multi-row (speculative-verify / chunked-prefill) dual-V SDPA, S_q query
 * rows per head, bottom-right-aligned causal mask when causal != 0: row i of
 * S_q attends keys [0, kv_len - S_q + i].  q (B,Hq,S_q,D), y (B,Hq,S_q,2D).
 * Replaces the FALLBACK composition model.py:769-807 (4 masked
 * mx.fast.scaled_dot_product_attention calls + concat) for the 4-slot cache;
 * the reference has no kernel for it.
 * The _q variant reads the packed cache like motif_sdpa_dual_v_q (the
 * reference dequantises through cache.py:448-465 first).
 * With an fp16 or bf16 cache at D = 128 and >= 64 virtual heads (query heads x rows)
 * per KV head -- a prefill chunk or a long slab -- the call runs the kernel
 * whose workgroups share each K/V tile through LDS among up to 128 virtual
 * heads; motif_sdpa_workspace_bytes() covers its row splits.
 * ------------------------------------------------------------------------ */
int motif_sdpa_dual_v_rows(const void* q, const void* k, const void* v1, const void* v2, void* y,
                           int dtype, int B, int Hq, int Hkv, int S_q, int D, int kv_cap,
                           int kv_len, int causal, float scale, void* workspace,
                           size_t workspace_bytes, void* stream);

int motif_sdpa_dual_v_q_rows(const void* q,
                             const uint32_t* k_data, const void* k_scales, const void* k_biases,
                             const uint32_t* v1_data, const void* v1_scales,
                             const void* v1_biases, const uint32_t* v2_data,
                             const void* v2_scales, const void* v2_biases, void* y, int dtype,
                             int B, int Hq, int Hkv, int S_q, int D, int kv_cap, int kv_len,
                             int causal, int bits, int group_size, float scale,
                             void* workspace, size_t workspace_bytes, void* stream);

/* The same three calls under the names a port of the reference binds: the
 * Metal kernel's name motif_sdpa_dual_v_q4 (attention.py:293) for
 * motif_sdpa_dual_v_q, and motif_sdpa_dual_v_verify / _q4_verify for the
 * multi-row calls of the speculative-verify caller
 * (MotifSpeculativeDecoding.swift:204-206).  Arguments and results are
 * those of motif_sdpa_dual_v_q, motif_sdpa_dual_v_rows and
 * motif_sdpa_dual_v_q_rows. */
int motif_sdpa_dual_v_q4(const void* q,
                         const uint32_t* k_data, const void* k_scales, const void* k_biases,
                         const uint32_t* v1_data, const void* v1_scales, const void* v1_biases,
                         const uint32_t* v2_data, const void* v2_scales, const void* v2_biases,
                         void* y, int dtype, int B, int Hq, int Hkv, int D, int kv_cap,
                         int kv_len, int bits, int group_size, float scale, void* workspace,
                         size_t workspace_bytes, void* stream);

int motif_sdpa_dual_v_verify(const void* q, const void* k, const void* v1, const void* v2,
                             void* y, int dtype, int B, int Hq, int Hkv, int S_q, int D,
                             int kv_cap, int kv_len, int causal, float scale, void* workspace,
                             size_t workspace_bytes, void* stream);

int motif_sdpa_dual_v_q4_verify(const void* q,
                                const uint32_t* k_data, const void* k_scales,
                                const void* k_biases, const uint32_t* v1_data,
                                const void* v1_scales, const void* v1_biases,
                                const uint32_t* v2_data, const void* v2_scales,
                                const void* v2_biases, void* y, int dtype, int B, int Hq,
                                int Hkv, int S_q, int D, int kv_cap, int kv_len, int causal,
                                int bits, int group_size, float scale, void* workspace,
                                size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ *
 * RoPE, head split and 4-slot write of one attention step in one launch.
 * Replaces, for a layer's step, the two self.rope calls on q and k
 * (src/mlx_motif/model.py:590-594; initialize_rope with traditional=False
 * and no scaling, i.e. channel pairs (i, i + D/2) rotated by
 * (pos0 + s) * theta^(-2i/D)), the k1/k2 and v1/v2 split with
 * update_and_fetch_4 (model.py:620-629, cache.py:337) and the q1/q2 split
 * (model.py:669-679).
 *   q (B, S, q_groups*(gr+1)*D), k (B, S, k_groups*(kr+1)*D),
 *   v (B, S, 2*k_groups*D)                            projection outputs
 *   q1 (B, q_groups*gr, S, D), q2 (B, q_groups, S, D)  roped, rows 0..S-1
 *   k1 (B, k_groups*kr, cap, D), k2 (B, k_groups, cap, D) roped, and
 *   v1, v2 (B, k_groups, cap, D): rows row0 .. row0 + S - 1.
 * q head h of group g is h = g*(gr+1) + j (j < gr: q1, j == gr: q2), or with
 * origin_first the q1 heads first; k likewise with kr; v head 2n -> v1[n],
 * 2n+1 -> v2[n].  With cap/row0 the cache capacity/offset the rows go
 * straight into the 4-slot fp cache; with cap = S, row0 = 0 they are plain
 * (B, H, S, D) tensors (e.g. for motif_quant_write4 or the *_append entries).
 * fp32 math, outputs rounded once to dtype.  D % 32 == 0, D <= 256.
 * ------------------------------------------------------------------------ */
int motif_rope_split4(const void* q, const void* k, const void* v, void* q1, void* q2, void* k1,
                      void* k2, void* v1, void* v2, int dtype, int B, int S, int q_groups, int gr,
                      int k_groups, int kr, int D, int cap, int row0, int pos0, float theta,
                      int origin_first, void* stream);

/* RoPE scaling.  The reference builds its rope with
 * initialize_rope(..., scaling_config=args.rope_scaling) (model.py:414-419;
 * mlx-lm 0.29.1), and a "linear" config of factor f ropes position p at
 * p / f (nn.RoPE's scale = 1 / f; the reference's grouped fixture
 * swift/Tests/MotifKitTests/Fixtures/motif_config_grouped.json:17 uses
 * f = 2).  Each *_scaled entry point is its unscaled namesake with
 * position_scale (> 0, finite) after theta: angle = (pos * position_scale)
 * * theta^(-2i/D), the position scaled first as mx.fast.rope scales it.
 * The unscaled entry points pass 1, which leaves every angle's bits
 * unchanged. */
int motif_rope_split4_scaled(const void* q, const void* k, const void* v, void* q1, void* q2,
                             void* k1, void* k2, void* v1, void* v2, int dtype, int B, int S,
                             int q_groups, int gr, int k_groups, int kr, int D, int cap,
                             int row0, int pos0, float theta, float position_scale,
                             int origin_first, void* stream);

/* ------------------------------------------------------------------------ *
 * A GDA layer's prefill chunk from the projection outputs, in one attention
 * launch (plus the split merge when its rows are split).  Replaces, for a
 * chunk of S tokens at cache offset `offset`, the rope calls on q and k
 * (src/mlx_motif/model.py:590-594), the 4-slot split with
 * update_and_fetch_4 (model.py:620-629, cache.py:337) and the four
 * mx.fast.scaled_dot_product_attention calls of the k_ratio-1 fallback with
 * the causal mask (model.py:769-797), whose outputs feed gda_post_split.
 *   q_proj (B, S, q_groups*(gr+1)*D): heads g*(gr+1)+j (origin j < gr,
 *          noise j = gr), or with origin_first the q_groups*gr origin heads
 *          first
 *   k_proj (B, S, 2*k_groups*D): k1[g] = head 2g, k2[g] = head 2g+1
 *   v_proj (B, S, 2*k_groups*D): v1[g] = head 2g, v2[g] = head 2g+1
 *   k1, k2, v1, v2 (B, k_groups, kv_cap, D): the 4-slot fp cache; rows
 *          offset .. offset + S - 1 are written (k roped)
 *   y_origin (B, q_groups*gr, S, 2D) = [softmax(q1 k1^T) V1 || .. V2]
 *   y_noise  (B, q_groups, S, 2D)    = the same for q2 over k2
 * q and k are roped at positions offset + s exactly as motif_rope_split4
 * rounds them, so the cache rows equal its output bit for bit.  Query row
 * s sees cache rows [0, offset + s] (bottom-right causal).  fp32
 * accumulation.  q_groups % k_groups == 0.  fp16/bf16 at D = 128 only;
 * other shapes return MOTIF_ERR_UNSUPPORTED (compose motif_rope_split4 and
 * motif_sdpa_dual_v_rows).  workspace: motif_gda_prefill_workspace_bytes
 * (0 when the rows are not split).
 * ------------------------------------------------------------------------ */
size_t motif_gda_prefill_workspace_bytes(int B, int S, int q_groups, int gr, int k_groups, int D,
                                         int kv_len);
int motif_gda_prefill_proj(const void* q_proj, const void* k_proj, const void* v_proj, void* k1,
                           void* k2, void* v1, void* v2, void* y_origin, void* y_noise, int dtype,
                           int B, int S, int q_groups, int gr, int k_groups, int D, int kv_cap,
                           int offset, float scale, float theta, int origin_first,
                           void* workspace, size_t workspace_bytes, void* stream);
/* With RoPE scaling (see motif_rope_split4_scaled). */
int motif_gda_prefill_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                  void* k1, void* k2, void* v1, void* v2, void* y_origin,
                                  void* y_noise, int dtype, int B, int S, int q_groups, int gr,
                                  int k_groups, int D, int kv_cap, int offset, float scale,
                                  float theta, float position_scale, int origin_first,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ *
 * MLX affine quantisation (mx.quantize, mode "affine") of `rows` rows of D
 * values: data (rows, D*bits/32) uint32, scales/biases (rows, D/group_size)
 * in dtype.  The reference calls mx.quantize at cache.py:498 and
 * cache.py:399-402.  bits in {4,8}, group_size in {32,64,128},
 * D % group_size == 0.
 * ------------------------------------------------------------------------ */
int motif_quantize(const void* x, uint32_t* data, void* scales, void* biases, int dtype,
                   int64_t rows, int D, int bits, int group_size, void* stream);

/* Dequantisation y = dtype(float(scale) * u + float(bias)); replaces the
 * _dequant_probe kernel (src/mlx_motif/kernels/mlp.py:176-255) and serves the
 * dequant bridge (cache.py:448-465). */
int motif_dequantize(const uint32_t* data, const void* scales, const void* biases, void* y,
                     int dtype, int64_t rows, int D, int bits, int group_size, void* stream);

/* ------------------------------------------------------------------------ *
 * Batched 4-slot quantised cache write in ONE dispatch: quantise rows
 * [0,S) of k1,k2,v1,v2 (each (B,H,S,D) dtype) and store them at rows
 * [offset, offset+S) of the four cache triples, each of capacity kv_cap:
 *   data[i] (B,H,kv_cap,D*bits/32) uint32, scales[i]/biases[i]
 *   (B,H,kv_cap,D/group_size) dtype; i = 0..3 for k1,k2,v1,v2.
 * Replaces MotifGroupedQuantizedKVCache._update_4 (cache.py:485-512:
 * concat + one mx.quantize + 12 slice writes).  Requires
 * offset + S <= kv_cap (the host grows capacity first, cache.py:245-265).
 * ------------------------------------------------------------------------ */
int motif_quant_write4(const void* k1, const void* k2, const void* v1, const void* v2,
                       uint32_t* const data[4], void* const scales[4], void* const biases[4],
                       int dtype, int B, int H, int S, int D, int kv_cap, int offset, int bits,
                       int group_size, void* stream);

/* ------------------------------------------------------------------------ *
 * Fused GDA epilogue on split inputs (gda_post_split, gda.py:223-282):
 *   d = o[b,h,s,:] - lambda * n[b,h/gr,s,:]
 *   y = dtype(d * rsqrt(mean(d^2) + eps) * w * one_minus_lambda_init)
 * o (B,q_origin,S,C), n (B,q_groups,S,C), w (C) dtype, y like o.
 * lambda_full: device pointer to ONE fp32 value (no host sync).
 * Contract (gda.py:248): q_origin == q_groups * gr.
 * ------------------------------------------------------------------------ */
int motif_gda_post_split(const void* attn_o, const void* attn_n, const void* subln_w, void* y,
                         int dtype, int B, int q_origin, int q_groups, int gr, int S, int C,
                         const float* lambda_full, float one_minus_lambda_init, float eps,
                         void* stream);

/* Same epilogue on the merged layout (gda_post, gda.py:285-341): merged is
 * (B, q_groups*gr + q_groups, S, C); noise head of origin head h is
 * q_groups*gr + h/gr. */
int motif_gda_post(const void* merged, const void* subln_w, void* y, int dtype, int B,
                   int q_groups, int gr, int S, int C, const float* lambda_full,
                   float one_minus_lambda_init, float eps, void* stream);

/* ------------------------------------------------------------------------ *
 * One GDA decode-attention step of a layer over the fp16/bf16/fp32 4-slot
 * cache: the origin pass sdpa_dual_v(q1, k1, v1, v2), the noise pass
 * sdpa_dual_v(q2, k2, v1, v2) and gda_post_split on their outputs.
 * Replaces the DUAL_V caller sequence of src/mlx_motif/model.py:749-768
 * (two sdpa_dual_v calls and gda_post_split); the reference has no single
 * kernel for it.  For the fp16 or bf16 cache at D = 128 it runs as two launches:
 * one attention launch reads each KV head's k1, k2, v1 and v2 rows once for
 * both passes (4 cache streams instead of the calls' 6), and the split merge
 * applies the epilogue.  Other dtypes and head dims compose the separate
 * calls on the device.
 *   q1 (B, Hkv*gr, 1, D), q2 (B, Hkv, 1, D)          dtype
 *   k1, k2, v1, v2 (B, Hkv, kv_cap, D)               dtype
 *   subln_w (2D) dtype; lambda_full: device pointer to ONE fp32 value
 *   y (B, Hkv*gr, 1, 2D)                             dtype
 * Origin head h pairs with noise head h / gr (gda.py:248).  The attention
 * outputs are rounded to dtype before the epilogue, as the reference's are.
 * Workspace (this entry point and motif_gda_decode_q):
 * motif_gda_decode_workspace_bytes(B, Hkv, gr, kv_len, D) bytes, 256-byte
 * aligned, zeroed before its first use.
 * ------------------------------------------------------------------------ */
size_t motif_gda_decode_workspace_bytes(int B, int Hkv, int gr, int kv_len, int D);

int motif_gda_decode(const void* q1, const void* q2, const void* k1, const void* k2,
                     const void* v1, const void* v2, const void* subln_w,
                     const float* lambda_full, float one_minus_lambda_init, float eps, void* y,
                     int dtype, int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                     float scale, void* workspace, size_t workspace_bytes, void* stream);

/* Same step over the packed MLX-affine q4/q8 cache (QUANT_SDPA path of
 * model.py:717-748: two sdpa_dual_v_q4 calls + gda_post_split).  Each slot is
 * a (data, scales, biases) triple laid out as for motif_sdpa_dual_v_q.  The
 * fused launch covers fp16 and bf16 activations, scales and biases at D = 128
 * when (gr + 1) rounded up to a power of two, times D / group_size, is at
 * most 16; other shapes compose the separate calls on the device.  Contract
 * as motif_sdpa_dual_v_q. */
int motif_gda_decode_q(const void* q1, const void* q2, const uint32_t* k1_data,
                       const void* k1_scales, const void* k1_biases, const uint32_t* k2_data,
                       const void* k2_scales, const void* k2_biases, const uint32_t* v1_data,
                       const void* v1_scales, const void* v1_biases, const uint32_t* v2_data,
                       const void* v2_scales, const void* v2_biases, const void* subln_w,
                       const float* lambda_full, float one_minus_lambda_init, float eps, void* y,
                       int dtype, int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                       int bits, int group_size, float scale, void* workspace,
                       size_t workspace_bytes, void* stream);

/* The same step for any noise-head count: q1 (B, Hq1, 1, D) origin queries
 * and q2 (B, Hq2, 1, D) noise queries over Hkv KV heads, each pass a GQA
 * sdpa_dual_v call (attention.py:190-260, native GQA, so Hkv divides Hq2)
 * and gda_post_split pairing origin head h with noise head h / gr,
 * gr = Hq1 / Hq2 (gda.py:223-282, q_origin == q_groups * gr at gda.py:248).
 * motif_gda_decode / motif_gda_decode_append are the case Hq2 == Hkv (the
 * 12.7B layout, model.py:749-768); Hq2 > Hkv is e.g. 8 origin and 8 noise
 * heads over 4 KV heads.  k1_new .. v2_new: all four null (no cache write)
 * or all four set (the token's rows, written at row kv_len - 1 first, as
 * the _append entry points do).  The fused launch takes the G1 = Hq1 / Hkv
 * origin and G2 = Hq2 / Hkv noise heads of a KV head as G1 + G2 <= 16
 * columns (packed cache: that sum rounded up to a power of two, times
 * D / group_size, <= 16); other shapes compose the separate calls on the
 * device.  Workspace: motif_gda_decode_heads_workspace_bytes(B, Hq1, Hq2,
 * Hkv, kv_len, D) bytes (0 when Hkv does not divide Hq2 or Hq2 does not
 * divide Hq1), 256-byte aligned, zeroed before its first use.  Contract
 * otherwise as motif_gda_decode / motif_gda_decode_q. */
size_t motif_gda_decode_heads_workspace_bytes(int B, int Hq1, int Hq2, int Hkv, int kv_len,
                                              int D);
int motif_gda_decode_heads(const void* q1, const void* q2, const void* k1_new,
                           const void* k2_new, const void* v1_new, const void* v2_new, void* k1,
                           void* k2, void* v1, void* v2, const void* subln_w,
                           const float* lambda_full, float one_minus_lambda_init, float eps,
                           void* y, int dtype, int B, int Hq1, int Hq2, int Hkv, int D,
                           int kv_cap, int kv_len, float scale, void* workspace,
                           size_t workspace_bytes, void* stream);
int motif_gda_decode_q_heads(const void* q1, const void* q2, const void* k1_new,
                             const void* k2_new, const void* v1_new, const void* v2_new,
                             uint32_t* k1_data, void* k1_scales, void* k1_biases,
                             uint32_t* k2_data, void* k2_scales, void* k2_biases,
                             uint32_t* v1_data, void* v1_scales, void* v1_biases,
                             uint32_t* v2_data, void* v2_scales, void* v2_biases,
                             const void* subln_w, const float* lambda_full,
                             float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                             int Hq1, int Hq2, int Hkv, int D, int kv_cap, int kv_len, int bits,
                             int group_size, float scale, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Decode step with append: one call per layer for a decode token (no single
 * counterpart in the reference, whose step is the cache write
 * MotifGroupedKVCache.update_and_fetch_4 / the quantized cache's
 * update_and_fetch_4_quantized, src/mlx_motif/cache.py:337, 467, followed by
 * the calls above).  Writes the new token's rows k1_new, k2_new,
 * v1_new, v2_new (each (B, Hkv, 1, D) dtype) at row kv_len - 1 of the four
 * slots -- quantised as motif_quant_write4 does for the packed cache -- and
 * then runs the step over kv_len rows.  kv_len counts the new row (>= 1).
 * When the step is fused, the write happens inside the attention launch:
 * the one wave whose tiles include row kv_len - 1 of a KV head stores that
 * head's rows before it loads them.  Otherwise the row is written first
 * (a row copy, or motif_quant_write4) and the separate calls follow. */
int motif_gda_decode_append(const void* q1, const void* q2, const void* k1_new,
                            const void* k2_new, const void* v1_new, const void* v2_new,
                            void* k1, void* k2, void* v1, void* v2, const void* subln_w,
                            const float* lambda_full, float one_minus_lambda_init, float eps,
                            void* y, int dtype, int B, int Hkv, int gr, int D, int kv_cap,
                            int kv_len, float scale, void* workspace, size_t workspace_bytes,
                            void* stream);

/* The same decode step from the projection outputs, RoPE included: the
 * layer's whole decode attention in the attention launch plus the merge.
 * Replaces, for one decode token, the rope calls (model.py:590-594), the
 * q/k/v head splits (model.py:620-629, 669-679), update_and_fetch_4
 * (cache.py:337) and the three calls (model.py:749-768).
 *   q_proj (B, 1, Hkv*(gr+1)*D): heads g*(gr+1)+j (origin j < gr, noise
 *          j = gr), or with origin_first the Hkv*gr origin heads first
 *   k_proj (B, 1, 2*Hkv*D): k1[g] = head 2g, k2[g] = head 2g+1 (k_ratio 1)
 *   v_proj (B, 1, 2*Hkv*D): v1[g] = head 2g, v2[g] = head 2g+1
 * q and the k rows are roped at position kv_len - 1 exactly as
 * motif_rope_split4 does (same rounding), the four rows are written at row
 * kv_len - 1, and y is what motif_rope_split4 + motif_gda_decode give, bit
 * for bit.  fp16/bf16 cache at D = 128 with gr + 1 <= 16 only; other shapes
 * return MOTIF_ERR_UNSUPPORTED (compose those two calls instead). */
int motif_gda_decode_proj(const void* q_proj, const void* k_proj, const void* v_proj, void* k1,
                          void* k2, void* v1, void* v2, const void* subln_w,
                          const float* lambda_full, float one_minus_lambda_init, float eps,
                          void* y, int dtype, int B, int Hkv, int gr, int D, int kv_cap,
                          int kv_len, float scale, float theta, int origin_first,
                          void* workspace, size_t workspace_bytes, void* stream);
/* With RoPE scaling (see motif_rope_split4_scaled). */
int motif_gda_decode_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                 void* k1, void* k2, void* v1, void* v2, const void* subln_w,
                                 const float* lambda_full, float one_minus_lambda_init,
                                 float eps, void* y, int dtype, int B, int Hkv, int gr, int D,
                                 int kv_cap, int kv_len, float scale, float theta,
                                 float position_scale, int origin_first, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* The same from the projection outputs over the packed cache: q and the k
 * rows roped as motif_rope_split4 rounds them (fp16), the four rows
 * quantised into row kv_len - 1 as motif_quant_write4 does; y equals
 * motif_rope_split4 + motif_gda_decode_q_append bit for bit.  fp16 scales,
 * D = 128, (gr + 1 columns) x (D / group_size) <= 16; other shapes return
 * MOTIF_ERR_UNSUPPORTED. */
int motif_gda_decode_q_proj(const void* q_proj, const void* k_proj, const void* v_proj,
                            uint32_t* k1_data, void* k1_scales, void* k1_biases,
                            uint32_t* k2_data, void* k2_scales, void* k2_biases,
                            uint32_t* v1_data, void* v1_scales, void* v1_biases,
                            uint32_t* v2_data, void* v2_scales, void* v2_biases,
                            const void* subln_w, const float* lambda_full,
                            float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                            int Hkv, int gr, int D, int kv_cap, int kv_len, int bits,
                            int group_size, float scale, float theta, int origin_first,
                            void* workspace, size_t workspace_bytes, void* stream);
/* With RoPE scaling (see motif_rope_split4_scaled). */
int motif_gda_decode_q_proj_scaled(const void* q_proj, const void* k_proj, const void* v_proj,
                                   uint32_t* k1_data, void* k1_scales, void* k1_biases,
                                   uint32_t* k2_data, void* k2_scales, void* k2_biases,
                                   uint32_t* v1_data, void* v1_scales, void* v1_biases,
                                   uint32_t* v2_data, void* v2_scales, void* v2_biases,
                                   const void* subln_w, const float* lambda_full,
                                   float one_minus_lambda_init, float eps, void* y, int dtype,
                                   int B, int Hkv, int gr, int D, int kv_cap, int kv_len,
                                   int bits, int group_size, float scale, float theta,
                                   float position_scale, int origin_first, void* workspace,
                                   size_t workspace_bytes, void* stream);

int motif_gda_decode_q_append(const void* q1, const void* q2, const void* k1_new,
                              const void* k2_new, const void* v1_new, const void* v2_new,
                              uint32_t* k1_data, void* k1_scales, void* k1_biases,
                              uint32_t* k2_data, void* k2_scales, void* k2_biases,
                              uint32_t* v1_data, void* v1_scales, void* v1_biases,
                              uint32_t* v2_data, void* v2_scales, void* v2_biases,
                              const void* subln_w, const float* lambda_full,
                              float one_minus_lambda_init, float eps, void* y, int dtype, int B,
                              int Hkv, int gr, int D, int kv_cap, int kv_len, int bits,
                              int group_size, float scale, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ *
 * Fused PolyNorm (polynorm, src/mlx_motif/kernels/mlp.py:119-157):
 *   y = w0*x^3*rsqrt(mean(x^6)+eps) + w1*x^2*rsqrt(mean(x^4)+eps)
 *     + w2*x*rsqrt(mean(x^2)+eps) + b
 * over the last axis of x (rows, D); weight (3) and bias (1) are dtype device
 * arrays.  x is read from HBM once.
 * ------------------------------------------------------------------------ */
int motif_polynorm(const void* x, const void* weight, const void* bias, void* y, int dtype,
                   int64_t rows, int D, float eps, void* stream);

/* ------------------------------------------------------------------------ *
 * Tuning knobs of the split-KV kernels (process-wide; for benchmarks and
 * sweeps, not needed for correct use).  key: "rows_per_split",
 * "waves_per_wg" (also the block size of the LDS-shared-tile multi-row
 * kernel), "min_wgs" (value 0 restores the default), "mfma" (1, the
 * default: matrix-core kernels where compiled; 0: VALU kernels only),
 * "fused_merge" (0, the default: a second launch combines the splits; 1: the
 * last workgroup to finish combines them inside the attention launch),
 * "qpair" (packed caches at head_dim 128, group size 64/128: 1, the
 * default, runs bf16 activations over 4-bit caches on the paired-tile
 * kernel and every other call on the per-tile kernel; 2 runs every such
 * call on the paired-tile kernel; 0 none), "qslab" (packed-cache
 * verify slabs of 17..64 virtual heads per KV head: 2, the default, runs 8-
 * and 4-bit slabs on the kernel that dequantises each tile once into LDS;
 * 1 only 8-bit slabs; 0 neither), "waves_per_wg" 4 also selects that
 * kernel's 4-wave variant, "qslab_ws" (1, the default: its 8-wave variant
 * runs four producer waves beside four consumer waves; 0: every wave does
 * both), "qslab_sets" (2, the default: its producers hold two steps of
 * packed data in registers; 3: three, one more step of loads in flight),
 * "merge_rows" (1, the default: a merge launch of at least 2048
 * partial rows runs one wave per row; 0: one wave per row slice),
 * "prefill_ncb" (column blocks of 16 virtual heads per wave of the 8-wave
 * shared-tile kernels: 0, the default, takes 2 from 2048 virtual heads per
 * KV head over at least 2048 rows, else 1; 1 or 2 forces it),
 * "prefill_min_heads" (0, the default: multi-row fp16/bf16 calls take the
 * shared-tile kernel from 64 virtual heads per KV head, or from 17 over 2048
 * or more rows; n > 0: from n heads),
 * "poly_rows" (workgroups per CU of the persistent PolyNorm kernel for 16-bit
 * rows of 2056..16384 values; 0, the default, sizes it by register use).
 * Returns MOTIF_OK or MOTIF_ERR_CONTRACT for an unknown key or value.
 * ------------------------------------------------------------------------ */
int motif_set_tuning(const char* key, int value);

/* ------------------------------------------------------------------------ *
 * Host-only self-check of the launch planners; no reference counterpart.
 * Walks every planner over decode, slab and prefill shapes without any HIP
 * call and checks that each plan of more than one split gets a workspace
 * holding its counters and partials, that the kernels would receive non-null
 * partial buffers inside it, that a missing workspace is refused before any
 * launch, and that motif_sdpa_workspace_bytes covers every plan it sizes.
 * Returns MOTIF_OK, or MOTIF_ERR_INTERNAL with the failing plan in
 * motif_last_error().  For tests and for callers that change the tuning.
 * ------------------------------------------------------------------------ */
int motif_plan_selfcheck(void);

#ifdef __cplusplus
}
#endif

#endif /* MOTIF_HIP_H */
