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
#include <chrono>
#include <exception>
#include <vector>

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

}  // extern "C"
