// qw_norm.hip -- RMSNorm (Qwen3.5 "(1+w)" form), fused residual add + RMSNorm,
// and the element-wise SiLU*mul.
//
// y = x / sqrt(mean(x^2) + eps) * (1 + w)   (language_common.cpp:21-36,
// rmsnorm_cuda.cu:39-100); the residual variant first forms r = a + b and
// writes it back (rmsnorm_cuda.cu:103-170, fused_kernels.cu:23-65).
// One 256-thread workgroup per token row; the row stays in registers between
// the reduction and the scaling pass, so each element is read once.
#include "qw_device.hpp"
#include "qw_kernels.hpp"

namespace qwk {

constexpr int NORM_MAX_PER_THREAD = 16;  // K <= 4096

__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, int xdt, const void* add,
                                                      void* sum_out, const float* gamma, float eps,
                                                      void* y, int ydt, int K, int ldx, int ldy) {
    __shared__ float red[4];
    const int64_t row = (int64_t)blockIdx.x * ldx;
    const int64_t yrow = (int64_t)blockIdx.x * ldy;
    float v[NORM_MAX_PER_THREAD];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_MAX_PER_THREAD; ++i) {
        const int k = threadIdx.x + i * 256;
        v[i] = 0.0f;
        if (k < K) {
            float f = load_act(x, xdt, row + k);
            if (add) {
                f += load_act(add, xdt, row + k);
                store_act(sum_out, xdt, row + k, f);
                // later reads use the value as stored
                f = load_act(sum_out, xdt, row + k);
            }
            v[i] = f;
            ss += f * f;
        }
    }
    // wave reduction (fixed order), then across the four waves
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
    for (int i = 0; i < NORM_MAX_PER_THREAD; ++i) {
        const int k = threadIdx.x + i * 256;
        if (k < K) store_act(y, ydt, yrow + k, v[i] * inv * (1.0f + gamma[k]));
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const void* g, const void* u, void* h, int dt,
                                                       int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) store_act(h, dt, i, silu_f(load_act(g, dt, i)) * load_act(u, dt, i));
}

hipError_t launch_rmsnorm(const void* x, int xdt, const void* add, void* sum_out,
                          const float* gamma, float eps, void* y, int ydt, int M, int K,
                          hipStream_t stream) {
    if (K > NORM_MAX_PER_THREAD * 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, stream, x, xdt, add, sum_out, gamma,
                       eps, y, ydt, K, K, K);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_ld(const void* x, int xdt, int ldx, const float* gamma, float eps, void* y, int ydt,
                             int ldy, int M, int K, hipStream_t stream) {
    if (K > NORM_MAX_PER_THREAD * 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, stream, x, xdt, nullptr, nullptr, gamma, eps, y, ydt,
                       K, ldx, ldy);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const void* g, const void* u, void* h, int dt, int64_t n,
                           hipStream_t stream) {
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, g, u, h, dt, n);
    return hipGetLastError();
}

}  // namespace qwk
