// ref_shim.cpp -- extern "C" entry points over the reference's own CPU operator
// classes, compiled together with the reference sources where they lie under
// /root/reference (see oracle/Makefile).  TEST INFRASTRUCTURE ONLY: the result,
// oracle/_ref/libqwref.so, validates the oracle restatement in this container.
//
// Classes used (reference repository paths):
//   qwen::LMHead   src/backend/cpu/core/heads/lm_head.hpp:7-33   (generic W.x)
//   qwen::MLP      src/backend/cpu/core/mlp/language_mlp.hpp:7-36
//   qwen::Sampler  src/backend/cpu/core/heads/sampler.hpp        (GREEDY)
//   qwen::RMSNorm  src/backend/cpu/core/common/language_common.hpp:9-33
//   qwen::LinearAttention  src/backend/cpu/core/attention/language_linear_attn.hpp:7-90
//   qwen::FullAttention, qwen::KVCache  src/backend/cpu/core/attention/language_full_attn.hpp:8-124
#include <chrono>
#include <exception>
#include <vector>

#include "language_full_attn.hpp"
#include "language_linear_attn.hpp"
#include "language_mlp.hpp"
#include "language_common.hpp"
#include "lm_head.hpp"
#include "sampler.hpp"

extern "C" {

// y[m][o] = W[o] . x[m] through LMHead::forward (a plain FP32 row-dot loop).
int ref_linear(const float* W, const float* x, float* y, int M, int N, int K) {
    try {
        qwen::LMHead head(K, N);
        head.set_weight(std::vector<float>(W, W + (size_t)N * K));
        for (int m = 0; m < M; ++m) {
            std::vector<float> in(x + (size_t)m * K, x + (size_t)(m + 1) * K);
            std::vector<float> out = head.forward(in);
            for (int o = 0; o < N; ++o) y[(size_t)m * N + o] = out[o];
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_mlp(const float* Wg, const float* Wu, const float* Wd, const float* x, float* y,
            int M, int H, int I) {
    try {
        qwen::MLP mlp(H, I);
        mlp.set_weights(std::vector<float>(Wg, Wg + (size_t)I * H),
                        std::vector<float>(Wu, Wu + (size_t)I * H),
                        std::vector<float>(Wd, Wd + (size_t)H * I));
        mlp.forward_batch(x, y, M);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_greedy(const float* logits, int n) {
    try {
        qwen::Sampler s(n, qwen::SamplingStrategy::GREEDY);
        return s.sample(std::vector<float>(logits, logits + n));
    } catch (const std::exception&) {
        return -1;
    }
}

// Timing leg of the CPU baseline: builds the reference MLP once and runs
// MLP::forward_batch `iters` times; returns the elapsed seconds (or -1).
double ref_mlp_time(const float* Wg, const float* Wu, const float* Wd, const float* x, float* y,
                    int M, int H, int I, int iters) {
    try {
        qwen::MLP mlp(H, I);
        mlp.set_weights(std::vector<float>(Wg, Wg + (size_t)I * H),
                        std::vector<float>(Wu, Wu + (size_t)I * H),
                        std::vector<float>(Wd, Wd + (size_t)H * I));
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) mlp.forward_batch(x, y, M);
        auto t1 = std::chrono::steady_clock::now();
        return std::chrono::duration<double>(t1 - t0).count();
    } catch (const std::exception&) {
        return -1.0;
    }
}

// Timing leg for the lm_head: LMHead::forward + greedy Sampler, `iters` times.
double ref_lmhead_time(const float* E, const float* h, int V, int K, int iters, int* id_out) {
    try {
        qwen::LMHead head(K, V);
        head.set_weight(std::vector<float>(E, E + (size_t)V * K));
        qwen::Sampler s(V, qwen::SamplingStrategy::GREEDY);
        std::vector<float> in(h, h + K);
        auto t0 = std::chrono::steady_clock::now();
        int id = -1;
        for (int i = 0; i < iters; ++i) id = s.sample(head.forward(in));
        auto t1 = std::chrono::steady_clock::now();
        if (id_out) *id_out = id;
        return std::chrono::duration<double>(t1 - t0).count();
    } catch (const std::exception&) {
        return -1.0;
    }
}

// Returns 0 if RMSNorm(K, eps) constructs, -1 if its constructor throws.
int ref_rmsnorm(const float* x, const float* w, float* y, int M, int K, float eps) {
    try {
        qwen::RMSNorm norm(K, eps);
        norm.set_weight(std::vector<float>(w, w + K));
        norm.forward_batch(x, y, M);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// T tokens of one sequence through LinearAttention::forward (the whole
// Gated-DeltaNet layer: projections, conv, gates, delta rule, norm-gate, out
// projection), starting from the given conv state [conv_dim][K-1] and
// recurrent state [nh][kd*vd]; both are returned updated.
int ref_linear_attn(const float* x, float* y, int T, int H, int nh, int kd, int vd, int K,
                    const float* Wqkv, const float* Wa, const float* Wb, const float* Wz,
                    const float* conv_w, const float* A_log, const float* dt_bias, const float* norm_w,
                    const float* Wout, float* conv_state, float* rec_state) {
    try {
        const int conv_dim = 2 * nh * kd + nh * vd;
        qwen::LinearAttention la(H, nh, kd, vd, K);
        la.set_weights(std::vector<float>(Wqkv, Wqkv + (size_t)conv_dim * H),
                       std::vector<float>(Wa, Wa + (size_t)nh * H), std::vector<float>(Wb, Wb + (size_t)nh * H),
                       std::vector<float>(Wz, Wz + (size_t)nh * vd * H),
                       std::vector<float>(conv_w, conv_w + (size_t)conv_dim * K),
                       std::vector<float>(A_log, A_log + nh), std::vector<float>(dt_bias, dt_bias + nh),
                       std::vector<float>(norm_w, norm_w + vd),
                       std::vector<float>(Wout, Wout + (size_t)H * nh * vd));
        qwen::LinearAttnState st;
        st.reset(nh, kd, vd, K);
        for (int d = 0; d < conv_dim; ++d)
            for (int j = 0; j < K - 1; ++j) st.conv_state[d][j] = conv_state[(size_t)d * (K - 1) + j];
        for (int h = 0; h < nh; ++h)
            for (int i = 0; i < kd * vd; ++i) st.recurrent_state[h][i] = rec_state[(size_t)h * kd * vd + i];
        for (int t = 0; t < T; ++t) {
            std::vector<float> in(x + (size_t)t * H, x + (size_t)(t + 1) * H);
            std::vector<float> out = la.forward(in, st);
            for (int i = 0; i < H; ++i) y[(size_t)t * H + i] = out[i];
        }
        for (int d = 0; d < conv_dim; ++d)
            for (int j = 0; j < K - 1; ++j) conv_state[(size_t)d * (K - 1) + j] = st.conv_state[d][j];
        for (int h = 0; h < nh; ++h)
            for (int i = 0; i < kd * vd; ++i) rec_state[(size_t)h * kd * vd + i] = st.recurrent_state[h][i];
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

/* FullAttention::forward_sequence-style run from an empty cache: token t at
 * position t (language_full_attn.cpp:117-216).  x [T][H] -> y [T][H]. */
int ref_full_attn(const float* x, float* y, int T, int H, int nh, int nkv, int qhd, int kvhd, float theta,
                  float partial, const float* Wq, const float* Wk, const float* Wv, const float* qn,
                  const float* kn, const float* Wo) {
    try {
        qwen::FullAttention fa(H, nh, nkv, qhd, kvhd, theta, partial);
        fa.set_weights(std::vector<float>(Wq, Wq + (size_t)nh * qhd * 2 * H),
                       std::vector<float>(Wk, Wk + (size_t)nkv * kvhd * H),
                       std::vector<float>(Wv, Wv + (size_t)nkv * kvhd * H), std::vector<float>(qn, qn + kvhd),
                       std::vector<float>(kn, kn + kvhd), std::vector<float>(Wo, Wo + (size_t)H * nh * kvhd));
        qwen::KVCache cache;
        cache.reset(1, nkv, kvhd, T);
        for (int t = 0; t < T; ++t) {
            std::vector<float> in(x + (size_t)t * H, x + (size_t)(t + 1) * H);
            std::vector<float> out = fa.forward(in, cache, 0, t);
            for (int i = 0; i < H; ++i) y[(size_t)t * H + i] = out[i];
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

}  // extern "C"
