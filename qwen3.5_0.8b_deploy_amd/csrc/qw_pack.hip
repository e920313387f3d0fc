// qw_pack.hip -- weight packer: dtype conversion, INT8 row quantization, and
// re-layout of W[N][K] into the gfx950 MFMA tile order described in
// qw_device.hpp.  Runs once per weight at load time (the role of
// CudaMLP::set_weights + quantize_fp32_to_int8_kernel, mlp_cuda.cu:22-39,
// 261-293, and of the host FP32->BF16 loops of lm_head_cuda.cu:177-180 and
// linear_attention_cuda.cu:412-466).
#include "qw_device.hpp"
#include "qw_kernels.hpp"

namespace qwk {

template <int WF>
__device__ __forceinline__ int64_t packed_offset(int pt, int r, int k, int ksteps) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int ES = WF == WF_F32 ? 4 : (WF == WF_BF16 ? 2 : 1);
    const int ks = k / (4 * KE);
    const int rem = k - ks * 4 * KE;
    const int g = rem / KE;
    const int e = rem - g * KE;
    const int lane = r + 16 * g;
    return (((int64_t)pt * ksteps + ks) * 64 + lane) * 16 + e * ES;
}

__device__ __forceinline__ float load_src(const void* p, int dt, int64_t i) {
    if (dt == DT_I8) return (float)reinterpret_cast<const int8_t*>(p)[i];
    return load_act(p, dt, i);
}

// One workgroup per source row.
template <int WF>
__global__ __launch_bounds__(256) void pack_kernel(const void* src, int src_dt,
                                                   const float* src_scales, int K, uint8_t* dst,
                                                   float* dst_scales, int tile_mul, int tile_add) {
    constexpr int KE = WTraits<WF>::KE;
    const int o = blockIdx.x;
    const int t = o >> 4, r = o & 15;
    const int pt = t * tile_mul + tile_add;
    const int ksteps = K / (4 * KE);
    const int64_t row = (int64_t)o * K;

    if constexpr (WF == WF_I8) {
        __shared__ float red[256];
        float scale;
        if (src_dt == DT_I8) {
            scale = src_scales[o];
        } else {
            // per-row max |w| (order-independent, hence exact)
            float mx = 0.0f;
            for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(load_src(src, src_dt, row + k)));
            red[threadIdx.x] = mx;
            __syncthreads();
            for (int s = 128; s > 0; s >>= 1) {
                if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
                __syncthreads();
            }
            const float sc = red[0] / 127.0f;
            scale = (sc > 1e-8f) ? sc : 1.0f;
        }
        if (threadIdx.x == 0) dst_scales[pt * 16 + r] = scale;
        for (int k = threadIdx.x; k < K; k += 256) {
            int8_t q;
            if (src_dt == DT_I8) {
                q = reinterpret_cast<const int8_t*>(src)[row + k];
            } else {
                float v = load_src(src, src_dt, row + k) / scale;
                v = fmaxf(-127.0f, fminf(127.0f, roundf(v)));
                q = (int8_t)v;
            }
            dst[packed_offset<WF>(pt, r, k, ksteps)] = (uint8_t)q;
        }
    } else if constexpr (WF == WF_BF16) {
        for (int k = threadIdx.x; k < K; k += 256) {
            uint32_t h;
            if (src_dt == DT_BF16) h = reinterpret_cast<const unsigned short*>(src)[row + k];
            else h = f32_to_bf16_bits(load_src(src, src_dt, row + k));
            *reinterpret_cast<unsigned short*>(dst + packed_offset<WF>(pt, r, k, ksteps)) = (unsigned short)h;
        }
    } else {
        for (int k = threadIdx.x; k < K; k += 256) {
            *reinterpret_cast<float*>(dst + packed_offset<WF>(pt, r, k, ksteps)) = load_src(src, src_dt, row + k);
        }
    }
}

// One workgroup per stored row: packed -> row-major in the stored dtype.
template <int WF>
__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t* src, int K, void* dst,
                                                     int tile_mul, int tile_add) {
    constexpr int KE = WTraits<WF>::KE;
    const int o = blockIdx.x;
    const int t = o >> 4, r = o & 15;
    const int pt = t * tile_mul + tile_add;
    const int ksteps = K / (4 * KE);
    const int64_t row = (int64_t)o * K;
    for (int k = threadIdx.x; k < K; k += 256) {
        const uint8_t* p = src + packed_offset<WF>(pt, r, k, ksteps);
        if constexpr (WF == WF_I8) reinterpret_cast<int8_t*>(dst)[row + k] = (int8_t)*p;
        else if constexpr (WF == WF_BF16) reinterpret_cast<unsigned short*>(dst)[row + k] = *reinterpret_cast<const unsigned short*>(p);
        else reinterpret_cast<float*>(dst)[row + k] = *reinterpret_cast<const float*>(p);
    }
}

// W[o][k] *= (1 + gamma[k]) in place on the packed tile order (the RMSNorm
// weight folded into the consuming projection).  One thread per 16-byte lane
// chunk: chunk c of k-step ks of any tile holds k = ks*4*KE + g*KE + e,
// g = (c % 64) / 16.  BF16 results are rounded to nearest even.
__global__ __launch_bounds__(256) void fold_norm_kernel(uint8_t* w, int wf, int ksteps, int64_t chunks,
                                                        const float* gamma) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int lane = (int)(c & 63);
    const int ks = (int)((c >> 6) % ksteps);
    const int g = lane >> 4;
    u32x4* p = reinterpret_cast<u32x4*>(w) + c;
    u32x4 v = *p;
    if (wf == WF_BF16) {
        const int k0 = ks * 32 + g * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float lo = bf16_bits_to_f32(v[q] & 0xffffu) * (1.0f + gamma[k0 + 2 * q]);
            const float hi = bf16_bits_to_f32(v[q] >> 16) * (1.0f + gamma[k0 + 2 * q + 1]);
            v[q] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
        }
    } else {
        const int k0 = ks * 16 + g * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __float_as_uint(__uint_as_float(v[q]) * (1.0f + gamma[k0 + q]));
    }
    *p = v;
}

hipError_t launch_fold_norm(uint8_t* w, int wf, int phys_tiles, int ksteps, const float* gamma, hipStream_t stream) {
    if (wf != WF_BF16 && wf != WF_F32) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)phys_tiles * ksteps * 64;
    hipLaunchKernelGGL(fold_norm_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, w, wf, ksteps,
                       chunks, gamma);
    return hipGetLastError();
}

hipError_t launch_pack(const void* src, int src_dt, int wf, const float* src_scales, int N, int K,
                       uint8_t* dst, float* dst_scales, int tile_mul, int tile_add,
                       hipStream_t stream) {
    dim3 grid(N), block(256);
    switch (wf) {
        case WF_F32: hipLaunchKernelGGL(pack_kernel<WF_F32>, grid, block, 0, stream, src, src_dt, src_scales, K, dst, dst_scales, tile_mul, tile_add); break;
        case WF_BF16: hipLaunchKernelGGL(pack_kernel<WF_BF16>, grid, block, 0, stream, src, src_dt, src_scales, K, dst, dst_scales, tile_mul, tile_add); break;
        case WF_I8: hipLaunchKernelGGL(pack_kernel<WF_I8>, grid, block, 0, stream, src, src_dt, src_scales, K, dst, dst_scales, tile_mul, tile_add); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_unpack(const uint8_t* src, int wf, int n_rows, int K, void* dst, int tile_mul,
                         int tile_add, hipStream_t stream) {
    dim3 grid(n_rows), block(256);
    switch (wf) {
        case WF_F32: hipLaunchKernelGGL(unpack_kernel<WF_F32>, grid, block, 0, stream, src, K, dst, tile_mul, tile_add); break;
        case WF_BF16: hipLaunchKernelGGL(unpack_kernel<WF_BF16>, grid, block, 0, stream, src, K, dst, tile_mul, tile_add); break;
        case WF_I8: hipLaunchKernelGGL(unpack_kernel<WF_I8>, grid, block, 0, stream, src, K, dst, tile_mul, tile_add); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qwk
