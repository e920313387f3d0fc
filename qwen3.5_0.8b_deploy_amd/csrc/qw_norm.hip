// qw_norm.hip -- RMSNorm (Qwen3.5 "(1+w)" form), fused residual add + RMSNorm,
// and the element-wise SiLU*mul.
//
// y = x / sqrt(mean(x^2) + eps) * (1 + w)   (language_common.cpp:21-36,
// rmsnorm_cuda.cu:39-100); the residual variant first forms r = a + b and
// writes it back (rmsnorm_cuda.cu:103-170, fused_kernels.cu:23-65).
// One 256-thread workgroup per token row; the row stays in registers between
// the reduction and the scaling pass, so each element is read once.
#include <algorithm>

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
        if (k < K) store_act(y, ydt, yrow + k, v[i] * inv * (gamma ? 1.0f + gamma[k] : 1.0f));
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const void* g, const void* u, void* h, int dt,
                                                       int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) store_act(h, dt, i, silu_f(load_act(g, dt, i)) * load_act(u, dt, i));
}

// Row-wise greedy argmax over materialized logits (GpuGreedyArgmaxSampler,
// gpu_sampler_argmax.cu:14-93, without its host-side second stage): grid
// (nblk, M); each workgroup scans a contiguous slice of one row, reduces
// (logit, index) keys across its waves and merges them into keys[m] with a
// 64-bit atomic max (lowest index on ties, std::max_element's rule); the last
// workgroup decodes every row and resets the keys and the counter.
__global__ __launch_bounds__(256) void argmax_rows_kernel(const void* logits, int dt, int V, int64_t ld,
                                                          unsigned long long* keys, unsigned* done,
                                                          int32_t* ids, float* maxv, int M) {
    __shared__ unsigned long long wbest[4];
    __shared__ int last;
    const int m = blockIdx.y;
    const int per = (V + gridDim.x - 1) / gridDim.x;
    const int v0 = blockIdx.x * per;
    const int v1 = min(V, v0 + per);
    unsigned long long best = 0ull;
    for (int v = v0 + threadIdx.x; v < v1; v += 256) {
        const unsigned long long k = argmax_key(load_act(logits, dt, (int64_t)m * ld + v), (uint32_t)v);
        best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wbest[0];
        for (int w = 1; w < 4; ++w) b = wbest[w] > b ? wbest[w] : b;
        if (b) __hip_atomic_fetch_max(&keys[m], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned old = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (old == total - 1) ? 1 : 0;
    }
    __syncthreads();
    if (last) {
        for (int r = threadIdx.x; r < M; r += 256) {
            const unsigned long long k = __hip_atomic_exchange(&keys[r], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ids[r] = (int32_t)key_index(k);
            if (maxv) maxv[r] = key_value(k);
        }
        if (threadIdx.x == 0) __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t launch_argmax_rows(const void* logits, int dt, int M, int V, int64_t ld, unsigned long long* keys,
                              unsigned* done, int32_t* ids, float* maxv, hipStream_t stream) {
    int nblk = (V + 2047) / 2048;
    const int cap = std::max(1, 1024 / M);
    nblk = std::max(1, std::min(nblk, cap));
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(nblk, M), dim3(256), 0, stream, logits, dt, V, ld, keys, done, ids,
                       maxv, M);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const void* x, int xdt, const void* add, void* sum_out,
                          const float* gamma, float eps, void* y, int ydt, int M, int K,
                          hipStream_t stream) {
    if (K > NORM_MAX_PER_THREAD * 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, stream, x, xdt, add, sum_out, gamma,
                       eps, y, ydt, K, K, K);
    return hipGetLastError();
}

// 16-bit rows with K % 8 == 0: one wave per row, 16-byte loads and stores,
// the row in registers (up to 8 chunks of 512), the sum of squares reduced
// within the wave (fixed order).  Four rows per workgroup.
template <int XDT, int YDT>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const uint16_t* x, int ldx, const float* gamma, float eps,
                                                          uint16_t* y, int ldy, int M, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const uint16_t* xr = x + (int64_t)row * ldx;
    uint16_t* yr = y + (int64_t)row * ldy;
    u32x4 v[8];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int k = c * 512 + lane * 8;
        v[c] = u32x4{0u, 0u, 0u, 0u};
        if (k < K) v[c] = *reinterpret_cast<const u32x4*>(xr + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t h = (v[c][e >> 1] >> (16 * (e & 1))) & 0xffffu;
            const float f = XDT == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
            ss += f * f;
        }
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int k = c * 512 + lane * 8;
        if (k >= K) continue;
        f32x4 g0 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
        if (gamma) {
            g0 = *reinterpret_cast<const f32x4*>(gamma + k);
            g1 = *reinterpret_cast<const f32x4*>(gamma + k + 4);
        }
        u32x4 o;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            uint32_t w = 0;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int e = 2 * e2 + h2;
                const uint32_t hb = (v[c][e2] >> (16 * h2)) & 0xffffu;
                const float f = XDT == DT_BF16 ? bf16_bits_to_f32(hb) : f16_bits_to_f32(hb);
                const float r = f * inv * (1.0f + (e < 4 ? g0[e & 3] : g1[e & 3]));
                w |= (YDT == DT_BF16 ? f32_to_bf16_bits(r) : f32_to_f16_bits(r)) << (16 * h2);
            }
            o[e2] = w;
        }
        *reinterpret_cast<u32x4*>(yr + k) = o;
    }
}

hipError_t launch_rmsnorm_ld(const void* x, int xdt, int ldx, const float* gamma, float eps, void* y, int ydt,
                             int ldy, int M, int K, hipStream_t stream) {
    const bool h16 = (xdt == DT_BF16 || xdt == DT_F16) && (ydt == DT_BF16 || ydt == DT_F16);
    if (h16 && K % 8 == 0 && K <= 4096 && ldx % 8 == 0 && ldy % 8 == 0 && ((uintptr_t)x & 15) == 0 &&
        ((uintptr_t)y & 15) == 0 && ((uintptr_t)gamma & 15) == 0) {
        const dim3 grid((M + 3) / 4);
        auto go = [&](auto k) {
            hipLaunchKernelGGL(k, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x), ldx, gamma, eps,
                               static_cast<uint16_t*>(y), ldy, M, K);
        };
        if (xdt == DT_BF16) {
            if (ydt == DT_BF16) go(rmsnorm_vec_kernel<DT_BF16, DT_BF16>);
            else go(rmsnorm_vec_kernel<DT_BF16, DT_F16>);
        } else {
            if (ydt == DT_BF16) go(rmsnorm_vec_kernel<DT_F16, DT_BF16>);
            else go(rmsnorm_vec_kernel<DT_F16, DT_F16>);
        }
        return hipGetLastError();
    }
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
