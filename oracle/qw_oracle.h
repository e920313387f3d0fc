/*
 * qw_oracle.h -- CPU oracle for the projection-matmul path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg load it.  Every function is a
 * scalar restatement of a reference CPU operator (file:line cited at each
 * definition in qw_oracle.c), or an FP64 ground truth used to bound the error
 * of the GPU kernels.
 *
 * Conventions (identical to the reference CPU operators):
 *   - weights are row-major W[out][in]  (N rows of K elements);
 *   - activations are row-major x[M][K], outputs y[M][N];
 *   - y[m][o] = sum_k W[o][k] * x[m][k], FP32 accumulated in ascending k.
 *
 * Each function is pinned by tests/test_oracle.py: against the reference's
 * own CPU operators (oracle/_ref), the committed golden vectors in
 * tests/golden/, closed forms and FP64 brute force.
 */
#ifndef QW_ORACLE_H
#define QW_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats (round-to-nearest-even, as torch / HIP intrinsics) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n);
void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

/* ---- projections ---- */
/* FP32 sequential-k matvec over M rows: y[m][o] = sum_k W[o][k]*x[m][k]. */
void orc_linear_f32(const float* W, const float* x, float* y, int M, int N, int K);
/* FP64 ground truth on the same FP32 inputs. */
void orc_linear_f64(const float* W, const float* x, double* y, int M, int N, int K);

/* ---- INT8 weight-only ---- */
/* Per-output-row symmetric quantization: s=max|w|/127 (1.0 if <=1e-8),
 * q=clamp(roundf(w/s),-127,127). */
void orc_quantize_rowscale(const float* W, int8_t* q, float* s, int N, int K);
/* Dequant-then-matmul: y[m][o] = sum_k (q[o][k]*s[o]) * x[m][k]. */
void orc_linear_int8_dequant(const int8_t* q, const float* s, const float* x, float* y,
                             int M, int N, int K);
/* FP64 ground truth: y = s[o] * sum_k q[o][k]*x[m][k]. */
void orc_linear_int8_f64(const int8_t* q, const float* s, const float* x, double* y,
                         int M, int N, int K);

/* ---- epilogue pieces ---- */
float orc_silu(float x);
/* RMSNorm with the Qwen3.5 (1+w) convention, eps given. */
void orc_rmsnorm(const float* x, const float* w, float* y, int M, int K, float eps);
void orc_rmsnorm_f64(const float* x, const float* w, double* y, int M, int K, double eps);
/* residual_out = residual_in + a ; normed = RMSNorm(residual_out). */
void orc_residual_rmsnorm(const float* residual_in, const float* a, const float* w,
                          float* residual_out, float* normed, int M, int K, float eps);

/* ---- MLP block ---- */
/* y[m] = Wd . (silu(Wg.x) * (Wu.x)), FP32, sequential k. */
void orc_mlp(const float* Wg, const float* Wu, const float* Wd, const float* x, float* y,
             int M, int H, int I);
/* FP64 ground truth of the same. */
void orc_mlp_f64(const float* Wg, const float* Wu, const float* Wd, const float* x, double* y,
                 int M, int H, int I);
/* Decoder-layer MLP half: h = residual; y = h + MLP(RMSNorm(h)). */
void orc_mlp_block(const float* Wg, const float* Wu, const float* Wd, const float* gamma,
                   const float* x, float* y, int M, int H, int I, float eps);
void orc_mlp_block_f64(const float* Wg, const float* Wu, const float* Wd, const float* gamma,
                       const float* x, double* y, int M, int H, int I, double eps);

/* ---- full attention Q+gate de-interleave ---- */
/* q_raw[m][H*2D] -> q[m][H*D], gate[m][H*D]: head h rows [h*2D,h*2D+D) are Q. */
void orc_split_q_gate(const float* q_raw, float* q, float* gate, int M, int heads, int head_dim);

/* ---- lm_head + greedy argmax ---- */
/* index of the first maximum (std::max_element semantics). */
int32_t orc_argmax_first(const float* v, int64_t n);
/* logits = E . h (FP32 sequential k), ids[m] = first argmax, maxv[m] = its logit. */
void orc_lmhead_argmax(const float* E, const float* h, int32_t* ids, float* maxv,
                       int M, int V, int K);
/* Same over bf16 inputs (E and h given as bf16 bits), FP32 accumulate. */
void orc_lmhead_argmax_bf16(const uint16_t* E, const uint16_t* h, int32_t* ids, float* maxv,
                            int M, int V, int K);
/* INT8 per-row-scaled E: logits = s[v]*sum_k q[v][k]*h[m][k] (FP32). */
void orc_lmhead_argmax_int8(const int8_t* q, const float* s, const float* h, int32_t* ids,
                            float* maxv, int M, int V, int K);

/* ---- seeded synthetic generator (mt19937-64 + Box-Muller) ---- */
/* raw MT19937-64 stream (first n outputs after seeding) */
void orc_mt64_raw(uint64_t seed, uint64_t* out, int64_t n);
void orc_fill_normal(float* dst, int64_t n, uint64_t seed, float mean, float std);
void orc_fill_uniform(float* dst, int64_t n, uint64_t seed, float lo, float hi);
void orc_fill_int8_uniform(int8_t* dst, int64_t n, uint64_t seed, int lo, int hi);

/* Gated-DeltaNet decode step between the projections
 * (language_linear_attn.cpp:143-256); see qw_oracle.c. */
void orc_gdn_step(int B, int nh, int kd, int vd, int K, const float* mixed, const float* a, const float* b,
                  const float* z, const float* conv_w, const float* A_log, const float* dt_bias,
                  const float* norm_w, float* conv_state, float* rec_state, float* out);

/* ---- gated full attention between the projections
 * (language_full_attn.cpp:117-216; INT8 KV recipe full_attention_cuda.cu:75-155) ---- */
/* Per-head RMSNorm (1 + w) of q [nh][hd] and k [nkv][hd] in place, then RoPE on
 * the first rotary_dim dims (interleaved pairs) at `position`. */
void orc_attn_norm_rope(float* q, float* k, int nh, int nkv, int hd, int rotary_dim, float theta,
                        const float* q_norm_w, const float* k_norm_w, int position);
/* Symmetric INT8 of one head vector: scale = max|x| / 127 (1 when <= 1e-8),
 * q = clamp(round_half_away(x / scale), -127, 127). */
void orc_kv_quant_int8(const float* x, int hd, int8_t* q, float* scale);
/* One query token over a cache of `len` tokens (FP32, [len][nkv][hd]), GQA
 * head h -> kv head h / (nh / nkv), scale 1/sqrt(hd), exact softmax, then
 * out *= sigmoid(gate).  q, gate, out: [nh][hd]. */
void orc_attn_token(const float* q, const float* gate, const float* kc, const float* vc, int len, int nh,
                    int nkv, int hd, float* out);
/* T tokens of one sequence at positions pos0 .. pos0+T-1: norm + RoPE, append
 * to the cache (cache_int8: INT8 with per-(token, kv head) scales, else FP32),
 * attention over positions 0 .. p (causal), gate.  q, gate: [T][nh][hd] raw
 * projections (after the Q/gate split); k, v: [T][nkv][hd].  Caches are
 * [capacity][nkv][hd] (kc/vc FP32 or int8_t), scales [capacity][nkv]. */
void orc_full_attn_seq(int T, int pos0, int nh, int nkv, int hd, int rotary_dim, float theta,
                       const float* q_norm_w, const float* k_norm_w, const float* q, const float* gate,
                       const float* k, const float* v, int cache_int8, void* kc, void* vc, float* ks, float* vs,
                       float* out);


#ifdef __cplusplus
}
#endif
#endif

