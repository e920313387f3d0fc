/*
 * qw_oracle.c -- scalar CPU restatement of the reference projection operators.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker used by tests/, by the
 * smoke() entry point and by bench.py's cpu_baseline leg.  The product path
 * (the HIP library) never links or calls it.
 *
 * Build: oracle/Makefile  (gcc -O2 -ffp-contract=off, like the reference's
 * CMakeLists.txt:47 "-O2", no SIMD intrinsics, single thread).
 *
 * Reference files followed (paths relative to the reference repository):
 *   linear/matvec   src/backend/cpu/core/attention/language_linear_attn.cpp:33-42
 *                   src/backend/cpu/core/heads/lm_head.cpp:24-39
 *   MLP             src/backend/cpu/core/mlp/language_mlp.cpp:7-9,53-91,93-127
 *   RMSNorm (1+w)   src/backend/cpu/core/common/language_common.cpp:21-78
 *   residual adds   src/backend/cpu/core/common/language_backbone.cpp:76-88
 *   Q/gate split    src/backend/cpu/core/attention/language_full_attn.cpp:127-140
 *   INT8 recipe     src/backend/cuda/kernels/mlp_cuda.cu:22-39
 *   greedy argmax   src/backend/cpu/core/heads/sampler.cpp:41-43
 */
#include "qw_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* number formats                                                            */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;                                  /* round to nearest even */
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

/* IEEE binary16, round to nearest even, with subnormals and overflow to inf. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (absu > 0x7f800000u ? 0x200u : 0u));
    if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);        /* >= 65520 rounds to inf */
    if (absu < 0x38800000u) {                                          /* result is subnormal */
        /* value = absf; subnormal unit is 2^-24 */
        float a = u2f(absu);
        float scaled = a * 16777216.0f;                                /* exact: a * 2^24 */
        /* round half to even on an exact float (scaled < 1024, representable) */
        float fl = floorf(scaled);
        float rem = scaled - fl;
        uint32_t m = (uint32_t)fl;
        if (rem > 0.5f || (rem == 0.5f && (m & 1u))) m += 1u;
        return (uint16_t)(sign | m);
    }
    uint32_t exp = (absu >> 23) - 127 + 15;
    uint32_t mant = absu & 0x7fffffu;
    uint32_t res = (exp << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (res & 1u))) res += 1u;
    return (uint16_t)(sign | res);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);                  /* mant * 2^-24 */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

void orc_f32_to_bf16_n(const float* s, uint16_t* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_bf16(s[i]); }
void orc_bf16_to_f32_n(const uint16_t* s, float* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_bf16_to_f32(s[i]); }
void orc_f32_to_f16_n(const float* s, uint16_t* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_f16(s[i]); }
void orc_f16_to_f32_n(const uint16_t* s, float* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f16_to_f32(s[i]); }

/* ------------------------------------------------------------------------ */
/* projections                                                               */
/* ------------------------------------------------------------------------ */

/* LinearAttention::linear (language_linear_attn.cpp:33-42) and LMHead::forward
 * (lm_head.cpp:30-36): for each output row, a dot of the weight row with the
 * input, accumulated in FP32 in ascending k.  M rows are processed one after
 * another, as MLP::forward_batch does (language_mlp.cpp:93-127). */
void orc_linear_f32(const float* W, const float* x, float* y, int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        for (int o = 0; o < N; ++o) {
            const float* w = W + (int64_t)o * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += w[k] * xm[k];
            y[(int64_t)m * N + o] = acc;
        }
    }
}

void orc_linear_f64(const float* W, const float* x, double* y, int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        for (int o = 0; o < N; ++o) {
            const float* w = W + (int64_t)o * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)w[k] * (double)xm[k];
            y[(int64_t)m * N + o] = acc;
        }
    }
}

/* quantize_fp32_to_int8_kernel (mlp_cuda.cu:22-39): per output row,
 * s = max|w| / 127, replaced by 1.0 when s <= 1e-8; q = clamp(roundf(w / s)).
 * roundf rounds half away from zero.  The division is by the stored scale, as
 * the kernel reads scale[row] back before dividing (mlp_cuda.cu:36). */
void orc_quantize_rowscale(const float* W, int8_t* q, float* s, int N, int K) {
    for (int o = 0; o < N; ++o) {
        const float* w = W + (int64_t)o * K;
        float mx = 0.0f;
        for (int k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(w[k]));
        float sc = mx / 127.0f;
        sc = (sc > 1e-8f) ? sc : 1.0f;
        s[o] = sc;
        for (int k = 0; k < K; ++k) {
            float v = w[k] / sc;
            v = fmaxf(-127.0f, fminf(127.0f, roundf(v)));
            q[(int64_t)o * K + k] = (int8_t)v;
        }
    }
}

/* Dequant-then-matmul: the weight is reconstructed as q*s in FP32 and the dot
 * runs in ascending k, the FP32 restatement of the INT8 GEMV's math
 * (mlp_cuda.cu:158-180 intends y = s[o] * sum q*x). */
void orc_linear_int8_dequant(const int8_t* q, const float* s, const float* x, float* y,
                             int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        for (int o = 0; o < N; ++o) {
            const int8_t* qo = q + (int64_t)o * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += ((float)qo[k] * s[o]) * xm[k];
            y[(int64_t)m * N + o] = acc;
        }
    }
}

void orc_linear_int8_f64(const int8_t* q, const float* s, const float* x, double* y,
                         int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        for (int o = 0; o < N; ++o) {
            const int8_t* qo = q + (int64_t)o * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)qo[k] * (double)xm[k];
            y[(int64_t)m * N + o] = acc * (double)s[o];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* epilogue pieces                                                           */
/* ------------------------------------------------------------------------ */

/* language_mlp.cpp:7-9 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* RMSNorm::forward_batch (language_common.cpp:56-78): rms = sqrt(mean(x^2)+eps),
 * y = (x / rms) * (1 + w). */
void orc_rmsnorm(const float* x, const float* w, float* y, int M, int K, float eps) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        float ss = 0.0f;
        for (int k = 0; k < K; ++k) ss += xm[k] * xm[k];
        float rms = sqrtf(ss / (float)K + eps);
        for (int k = 0; k < K; ++k) y[(int64_t)m * K + k] = (xm[k] / rms) * (1.0f + w[k]);
    }
}

void orc_rmsnorm_f64(const float* x, const float* w, double* y, int M, int K, double eps) {
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * K;
        double ss = 0.0;
        for (int k = 0; k < K; ++k) ss += (double)xm[k] * (double)xm[k];
        double rms = sqrt(ss / (double)K + eps);
        for (int k = 0; k < K; ++k) y[(int64_t)m * K + k] = ((double)xm[k] / rms) * (1.0 + (double)w[k]);
    }
}

/* LanguageLayer::forward (language_backbone.cpp:76-81): h = input + attn_out,
 * then the post-attention RMSNorm of h. */
void orc_residual_rmsnorm(const float* residual_in, const float* a, const float* w,
                          float* residual_out, float* normed, int M, int K, float eps) {
    for (int64_t i = 0; i < (int64_t)M * K; ++i) residual_out[i] = residual_in[i] + a[i];
    orc_rmsnorm(residual_out, w, normed, M, K, eps);
}

/* ------------------------------------------------------------------------ */
/* MLP                                                                       */
/* ------------------------------------------------------------------------ */

/* MLP::forward / forward_batch (language_mlp.cpp:53-127): gate and up dots in
 * one loop over k, gate[i] = silu(g), hidden = gate*up, then the down dot. */
void orc_mlp(const float* Wg, const float* Wu, const float* Wd, const float* x, float* y,
             int M, int H, int I) {
    float* gate = (float*)malloc(sizeof(float) * (size_t)I);
    float* up = (float*)malloc(sizeof(float) * (size_t)I);
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * H;
        for (int i = 0; i < I; ++i) {
            float g = 0.0f, u = 0.0f;
            for (int j = 0; j < H; ++j) {
                float xv = xm[j];
                g += Wg[(int64_t)i * H + j] * xv;
                u += Wu[(int64_t)i * H + j] * xv;
            }
            gate[i] = orc_silu(g);
            up[i] = u;
        }
        for (int i = 0; i < I; ++i) gate[i] = gate[i] * up[i];
        for (int o = 0; o < H; ++o) {
            float acc = 0.0f;
            for (int j = 0; j < I; ++j) acc += Wd[(int64_t)o * I + j] * gate[j];
            y[(int64_t)m * H + o] = acc;
        }
    }
    free(gate);
    free(up);
}

void orc_mlp_f64(const float* Wg, const float* Wu, const float* Wd, const float* x, double* y,
                 int M, int H, int I) {
    double* hid = (double*)malloc(sizeof(double) * (size_t)I);
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (int64_t)m * H;
        for (int i = 0; i < I; ++i) {
            double g = 0.0, u = 0.0;
            for (int j = 0; j < H; ++j) {
                g += (double)Wg[(int64_t)i * H + j] * (double)xm[j];
                u += (double)Wu[(int64_t)i * H + j] * (double)xm[j];
            }
            hid[i] = g / (1.0 + exp(-g)) * u;
        }
        for (int o = 0; o < H; ++o) {
            double acc = 0.0;
            for (int j = 0; j < I; ++j) acc += (double)Wd[(int64_t)o * I + j] * hid[j];
            y[(int64_t)m * H + o] = acc;
        }
    }
    free(hid);
}

/* Second half of LanguageLayer::forward (language_backbone.cpp:81-88):
 * h2 = post_layernorm(h), out = h + mlp(h2). */
void orc_mlp_block(const float* Wg, const float* Wu, const float* Wd, const float* gamma,
                   const float* x, float* y, int M, int H, int I, float eps) {
    float* xn = (float*)malloc(sizeof(float) * (size_t)M * H);
    orc_rmsnorm(x, gamma, xn, M, H, eps);
    orc_mlp(Wg, Wu, Wd, xn, y, M, H, I);
    for (int64_t i = 0; i < (int64_t)M * H; ++i) y[i] = x[i] + y[i];
    free(xn);
}

void orc_mlp_block_f64(const float* Wg, const float* Wu, const float* Wd, const float* gamma,
                       const float* x, double* y, int M, int H, int I, double eps) {
    double* xn = (double*)malloc(sizeof(double) * (size_t)M * H);
    double* hid = (double*)malloc(sizeof(double) * (size_t)I);
    orc_rmsnorm_f64(x, gamma, xn, M, H, eps);
    for (int m = 0; m < M; ++m) {
        const double* xm = xn + (int64_t)m * H;
        for (int i = 0; i < I; ++i) {
            double g = 0.0, u = 0.0;
            for (int j = 0; j < H; ++j) {
                g += (double)Wg[(int64_t)i * H + j] * xm[j];
                u += (double)Wu[(int64_t)i * H + j] * xm[j];
            }
            hid[i] = g / (1.0 + exp(-g)) * u;
        }
        for (int o = 0; o < H; ++o) {
            double acc = 0.0;
            for (int j = 0; j < I; ++j) acc += (double)Wd[(int64_t)o * I + j] * hid[j];
            y[(int64_t)m * H + o] = (double)x[(int64_t)m * H + o] + acc;
        }
    }
    free(hid);
    free(xn);
}

/* ------------------------------------------------------------------------ */
/* full attention Q / gate                                                   */
/* ------------------------------------------------------------------------ */

/* FullAttention::forward (language_full_attn.cpp:133-140): q_proj output of
 * 2*heads*D rows; per head h, rows [h*2D, h*2D+D) are Q, the next D the gate. */
void orc_split_q_gate(const float* q_raw, float* q, float* gate, int M, int heads, int D) {
    for (int m = 0; m < M; ++m) {
        const float* r = q_raw + (int64_t)m * heads * 2 * D;
        for (int h = 0; h < heads; ++h)
            for (int d = 0; d < D; ++d) {
                q[(int64_t)m * heads * D + h * D + d] = r[h * 2 * D + d];
                gate[(int64_t)m * heads * D + h * D + d] = r[h * 2 * D + D + d];
            }
    }
}

/* ------------------------------------------------------------------------ */
/* lm_head + greedy argmax                                                   */
/* ------------------------------------------------------------------------ */

/* Sampler::sample_greedy (sampler.cpp:41-43): std::max_element, which returns
 * the first element that no later element exceeds -- the lowest index wins a
 * tie. */
int32_t orc_argmax_first(const float* v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[best] < v[i]) best = i;
    return (int32_t)best;
}

static void lmhead_rows(const float* logits, int32_t* ids, float* maxv, int m, int V) {
    int32_t id = orc_argmax_first(logits, V);
    ids[m] = id;
    if (maxv) maxv[m] = logits[id];
}

/* LMHead::forward (lm_head.cpp:24-39) followed by greedy sampling. */
void orc_lmhead_argmax(const float* E, const float* h, int32_t* ids, float* maxv,
                       int M, int V, int K) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)V);
    for (int m = 0; m < M; ++m) {
        orc_linear_f32(E, h + (int64_t)m * K, logits, 1, V, K);
        lmhead_rows(logits, ids, maxv, m, V);
    }
    free(logits);
}

/* The same with the tied matrix and the hidden state held in bf16, as
 * CudaLMHead does (lm_head_cuda.cu:177-180 converts E, :198-210 converts the
 * input); products and sums in FP32. */
void orc_lmhead_argmax_bf16(const uint16_t* E, const uint16_t* h, int32_t* ids, float* maxv,
                            int M, int V, int K) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)V);
    float* hf = (float*)malloc(sizeof(float) * (size_t)K);
    for (int m = 0; m < M; ++m) {
        for (int k = 0; k < K; ++k) hf[k] = orc_bf16_to_f32(h[(int64_t)m * K + k]);
        for (int v = 0; v < V; ++v) {
            const uint16_t* e = E + (int64_t)v * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += orc_bf16_to_f32(e[k]) * hf[k];
            logits[v] = acc;
        }
        lmhead_rows(logits, ids, maxv, m, V);
    }
    free(hf);
    free(logits);
}

void orc_lmhead_argmax_int8(const int8_t* q, const float* s, const float* h, int32_t* ids,
                            float* maxv, int M, int V, int K) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)V);
    for (int m = 0; m < M; ++m) {
        orc_linear_int8_dequant(q, s, h + (int64_t)m * K, logits, 1, V, K);
        lmhead_rows(logits, ids, maxv, m, V);
    }
    free(logits);
}

/* ------------------------------------------------------------------------ */
/* seeded generator: MT19937-64 (Matsumoto & Nishimura, 2000) + Box-Muller    */
/* ------------------------------------------------------------------------ */

typedef struct { uint64_t mt[312]; int idx; } mt64;

static void mt64_seed(mt64* g, uint64_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

static uint64_t mt64_next(mt64* g) {
    static const uint64_t UM = 0xFFFFFFFF80000000ULL, LM = 0x7FFFFFFFULL;
    static const uint64_t MATRIX_A = 0xB5026F5AA96619E9ULL;
    if (g->idx >= 312) {
        for (int i = 0; i < 312; ++i) {
            uint64_t x = (g->mt[i] & UM) | (g->mt[(i + 1) % 312] & LM);
            uint64_t xa = x >> 1;
            if (x & 1ULL) xa ^= MATRIX_A;
            g->mt[i] = g->mt[(i + 156) % 312] ^ xa;
        }
        g->idx = 0;
    }
    uint64_t x = g->mt[g->idx++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= (x >> 43);
    return x;
}

void orc_mt64_raw(uint64_t seed, uint64_t* out, int64_t n) {
    mt64 g;
    mt64_seed(&g, seed);
    for (int64_t i = 0; i < n; ++i) out[i] = mt64_next(&g);
}

/* uniform double in (0, 1): 53 random bits, offset by half an ulp */
static double mt64_unit(mt64* g) {
    return ((double)(mt64_next(g) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(float* dst, int64_t n, uint64_t seed, float mean, float std) {
    mt64 g;
    mt64_seed(&g, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = mt64_unit(&g), u2 = mt64_unit(&g);
        double r = sqrt(-2.0 * log(u1));
        dst[i] = (float)(mean + std * r * cos(two_pi * u2));
        if (i + 1 < n) dst[i + 1] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

void orc_fill_uniform(float* dst, int64_t n, uint64_t seed, float lo, float hi) {
    mt64 g;
    mt64_seed(&g, seed);
    for (int64_t i = 0; i < n; ++i) dst[i] = (float)(lo + (hi - lo) * mt64_unit(&g));
}

void orc_fill_int8_uniform(int8_t* dst, int64_t n, uint64_t seed, int lo, int hi) {
    mt64 g;
    mt64_seed(&g, seed);
    uint64_t span = (uint64_t)(hi - lo + 1);
    for (int64_t i = 0; i < n; ++i) dst[i] = (int8_t)(lo + (int)(mt64_next(&g) % span));
}

/* ------------------------------------------------------------------------
 * Gated-DeltaNet decode step: everything between the input projections and
 * the out projection of LinearAttention::forward
 * (src/backend/cpu/core/attention/language_linear_attn.cpp:143-256), in that
 * file's operation order, one token per sequence for B sequences:
 *   1. causal conv1d over the conv_dim = 2*nh*kd + nh*vd QKV channels with
 *      the reference's tap order (w[d][K-1] on the current input, w[d][j] on
 *      conv_state[d][j], j < K-1, state[d][0] the newest), SiLU; then the
 *      state shift (:144-157);
 *   2. beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias) (:166-174);
 *   3. per head: q /= sqrt(sum q^2 + 1e-6) then * 1/sqrt(kd); k likewise
 *      without the scale (:176-200);
 *   4. per head the delta rule on S[kd][vd]: S *= exp(g); kv = S^T k;
 *      delta = (v - kv) * beta; S += k delta^T; o = S^T q (:202-234);
 *   5. per head RMSNorm of o (eps 1e-6) times norm_w, times SiLU(z) (:236-251).
 * Layouts: mixed [B][conv_dim], a/b [B][nh], z [B][nh*vd], conv_w
 * [conv_dim][K], conv_state [B][conv_dim][K-1], rec_state [B][nh][kd][vd],
 * out [B][nh*vd].  The states are updated in place.
 * ------------------------------------------------------------------------ */
static float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
static float orc_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

void orc_gdn_step(int B, int nh, int kd, int vd, int K, const float* mixed, const float* a, const float* b,
                  const float* z, const float* conv_w, const float* A_log, const float* dt_bias,
                  const float* norm_w, float* conv_state, float* rec_state, float* out) {
    const int conv_dim = 2 * nh * kd + nh * vd;
    const int sl = K - 1;
    float* co = (float*)malloc(sizeof(float) * (size_t)conv_dim);
    float* kv = (float*)malloc(sizeof(float) * (size_t)vd);
    float* de = (float*)malloc(sizeof(float) * (size_t)vd);
    const float q_scale = 1.0f / sqrtf((float)kd);
    for (int bi = 0; bi < B; ++bi) {
        const float* mx = mixed + (size_t)bi * conv_dim;
        float* cs = conv_state + (size_t)bi * conv_dim * sl;
        for (int d = 0; d < conv_dim; ++d) {
            float sum = conv_w[(size_t)d * K + (K - 1)] * mx[d];
            for (int j = 0; j < sl; ++j) sum += conv_w[(size_t)d * K + j] * cs[(size_t)d * sl + j];
            co[d] = orc_silu(sum);
        }
        for (int d = 0; d < conv_dim; ++d) {
            for (int j = sl - 1; j > 0; --j) cs[(size_t)d * sl + j] = cs[(size_t)d * sl + j - 1];
            if (sl > 0) cs[(size_t)d * sl] = mx[d];
        }
        float* q = co;
        float* k = co + nh * kd;
        const float* v = co + 2 * nh * kd;
        float* o = out + (size_t)bi * nh * vd;
        const float* zz = z + (size_t)bi * nh * vd;
        for (int h = 0; h < nh; ++h) {
            float ql = 0.0f, kl = 0.0f;
            for (int d = 0; d < kd; ++d) ql += q[h * kd + d] * q[h * kd + d];
            ql = sqrtf(ql + 1e-6f);
            for (int d = 0; d < kd; ++d) q[h * kd + d] = q[h * kd + d] / ql * q_scale;
            for (int d = 0; d < kd; ++d) kl += k[h * kd + d] * k[h * kd + d];
            kl = sqrtf(kl + 1e-6f);
            for (int d = 0; d < kd; ++d) k[h * kd + d] = k[h * kd + d] / kl;
        }
        for (int h = 0; h < nh; ++h) {
            const float beta = orc_sigmoid(b[(size_t)bi * nh + h]);
            const float g = -expf(A_log[h]) * orc_softplus(a[(size_t)bi * nh + h] + dt_bias[h]);
            const float gt = expf(g);
            float* S = rec_state + ((size_t)bi * nh + h) * kd * vd;
            for (int i = 0; i < kd * vd; ++i) S[i] *= gt;
            for (int c = 0; c < vd; ++c) {
                float acc = 0.0f;
                for (int r = 0; r < kd; ++r) acc += S[r * vd + c] * k[h * kd + r];
                kv[c] = acc;
            }
            for (int c = 0; c < vd; ++c) de[c] = (v[h * vd + c] - kv[c]) * beta;
            for (int r = 0; r < kd; ++r)
                for (int c = 0; c < vd; ++c) S[r * vd + c] += k[h * kd + r] * de[c];
            for (int c = 0; c < vd; ++c) {
                float acc = 0.0f;
                for (int r = 0; r < kd; ++r) acc += S[r * vd + c] * q[h * kd + r];
                o[h * vd + c] = acc;
            }
        }
        for (int h = 0; h < nh; ++h) {
            float var = 0.0f;
            for (int c = 0; c < vd; ++c) var += o[h * vd + c] * o[h * vd + c];
            var /= (float)vd;
            const float inv = 1.0f / sqrtf(var + 1e-6f);
            for (int c = 0; c < vd; ++c) o[h * vd + c] = o[h * vd + c] * inv * norm_w[c];
        }
        for (int i = 0; i < nh * vd; ++i) o[i] = o[i] * orc_silu(zz[i]);
    }
    free(co);
    free(kv);
    free(de);
}

/* ===== gated full attention (language_full_attn.cpp:117-216) ===== */

/* FullAttention::rms_normalize (language_full_attn.cpp:77-86) */
static void orc_attn_rmsnorm(float* x, int n, const float* w) {
    float sum_sq = 0.0f;
    for (int i = 0; i < n; ++i) sum_sq += x[i] * x[i];
    const float rms = sqrtf(sum_sq / n + 1e-6f);
    for (int i = 0; i < n; ++i) x[i] = x[i] / rms * (1.0f + w[i]);
}

/* per-head norms (language_full_attn.cpp:156-161) and FullAttention::apply_rope
 * (language_full_attn.cpp:88-108) */
void orc_attn_norm_rope(float* q, float* k, int nh, int nkv, int hd, int rotary_dim, float theta,
                        const float* q_norm_w, const float* k_norm_w, int position) {
    for (int h = 0; h < nh; ++h) orc_attn_rmsnorm(q + (size_t)h * hd, hd, q_norm_w);
    for (int h = 0; h < nkv; ++h) orc_attn_rmsnorm(k + (size_t)h * hd, hd, k_norm_w);
    for (int d = 0; d < rotary_dim; d += 2) {
        const float freq = 1.0f / powf(theta, (float)d / rotary_dim);
        const float angle = position * freq;
        const float c = cosf(angle), s = sinf(angle);
        for (int h = 0; h < nh; ++h) {
            const float q0 = q[h * hd + d], q1 = q[h * hd + d + 1];
            q[h * hd + d] = q0 * c - q1 * s;
            q[h * hd + d + 1] = q0 * s + q1 * c;
        }
        for (int h = 0; h < nkv; ++h) {
            const float k0 = k[h * hd + d], k1 = k[h * hd + d + 1];
            k[h * hd + d] = k0 * c - k1 * s;
            k[h * hd + d + 1] = k0 * s + k1 * c;
        }
    }
}

/* the INT8 KV-cache write of fused_kv_cache_int8_kernel
 * (full_attention_cuda.cu:130-150): absmax / 127 per head, 1 when tiny,
 * roundf (half away from zero), clamp to +-127 */
void orc_kv_quant_int8(const float* x, int hd, int8_t* q, float* scale) {
    float m = 0.0f;
    for (int d = 0; d < hd; ++d) m = fmaxf(m, fabsf(x[d]));
    float s = m / 127.0f;
    s = s > 1e-8f ? s : 1.0f;
    for (int d = 0; d < hd; ++d) q[d] = (int8_t)fmaxf(-127.0f, fminf(127.0f, roundf(x[d] / s)));
    *scale = s;
}

/* the attention and gate of FullAttention::forward (language_full_attn.cpp:165-207) */
void orc_attn_token(const float* q, const float* gate, const float* kc, const float* vc, int len, int nh,
                    int nkv, int hd, float* out) {
    const int group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    float* w = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    for (int h = 0; h < nh; ++h) {
        const int g = h / group;
        float* o = out + (size_t)h * hd;
        for (int d = 0; d < hd; ++d) o[d] = 0.0f;
        for (int t = 0; t < len; ++t) {
            const float* kp = kc + ((size_t)t * nkv + g) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += q[(size_t)h * hd + d] * kp[d];
            w[t] = dot * scale;
        }
        float mx = w[0];
        for (int t = 1; t < len; ++t) mx = fmaxf(mx, w[t]);
        float sum = 0.0f;
        for (int t = 0; t < len; ++t) {
            w[t] = expf(w[t] - mx);
            sum += w[t];
        }
        for (int t = 0; t < len; ++t) w[t] /= sum;
        for (int t = 0; t < len; ++t) {
            const float* vp = vc + ((size_t)t * nkv + g) * hd;
            for (int d = 0; d < hd; ++d) o[d] += w[t] * vp[d];
        }
        for (int d = 0; d < hd; ++d) o[d] *= 1.0f / (1.0f + expf(-gate[(size_t)h * hd + d]));
    }
    free(w);
}

/* FullAttention::forward over consecutive positions (forward_sequence,
 * language_full_attn.cpp:219-250), between the projections; the INT8 cache
 * variant stores what fused_kv_cache_int8_kernel stores and reads each token
 * back with its own scale */
void orc_full_attn_seq(int T, int pos0, int nh, int nkv, int hd, int rotary_dim, float theta,
                       const float* q_norm_w, const float* k_norm_w, const float* q, const float* gate,
                       const float* k, const float* v, int cache_int8, void* kc, void* vc, float* ks, float* vs,
                       float* out) {
    const size_t qn = (size_t)nh * hd, kn = (size_t)nkv * hd;
    float* qb = (float*)malloc(sizeof(float) * qn);
    float* kb = (float*)malloc(sizeof(float) * kn);
    const int len_max = pos0 + T;
    float* kf = cache_int8 ? (float*)malloc(sizeof(float) * (size_t)len_max * kn) : NULL;
    float* vf = cache_int8 ? (float*)malloc(sizeof(float) * (size_t)len_max * kn) : NULL;
    for (int t = 0; t < T; ++t) {
        const int pos = pos0 + t;
        memcpy(qb, q + (size_t)t * qn, sizeof(float) * qn);
        memcpy(kb, k + (size_t)t * kn, sizeof(float) * kn);
        orc_attn_norm_rope(qb, kb, nh, nkv, hd, rotary_dim, theta, q_norm_w, k_norm_w, pos);
        const float* vt = v + (size_t)t * kn;
        if (cache_int8) {
            int8_t* kq = (int8_t*)kc;
            int8_t* vq = (int8_t*)vc;
            for (int h = 0; h < nkv; ++h) {
                orc_kv_quant_int8(kb + (size_t)h * hd, hd, kq + ((size_t)pos * nkv + h) * hd, ks + (size_t)pos * nkv + h);
                orc_kv_quant_int8(vt + (size_t)h * hd, hd, vq + ((size_t)pos * nkv + h) * hd, vs + (size_t)pos * nkv + h);
            }
            for (int p = 0; p <= pos; ++p)
                for (int h = 0; h < nkv; ++h)
                    for (int d = 0; d < hd; ++d) {
                        const size_t i = ((size_t)p * nkv + h) * hd + d;
                        kf[i] = (float)kq[i] * ks[(size_t)p * nkv + h];
                        vf[i] = (float)vq[i] * vs[(size_t)p * nkv + h];
                    }
            orc_attn_token(qb, gate + (size_t)t * qn, kf, vf, pos + 1, nh, nkv, hd, out + (size_t)t * qn);
        } else {
            memcpy((float*)kc + (size_t)pos * kn, kb, sizeof(float) * kn);
            memcpy((float*)vc + (size_t)pos * kn, vt, sizeof(float) * kn);
            orc_attn_token(qb, gate + (size_t)t * qn, (const float*)kc, (const float*)vc, pos + 1, nh, nkv, hd,
                           out + (size_t)t * qn);
        }
    }
    free(qb);
    free(kb);
    free(kf);
    free(vf);
}
