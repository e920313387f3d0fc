// qw_attn.hip -- gated full attention between the projections for gfx950:
// per-head RMSNorm (1 + w) of q and k, partial RoPE, the KV-cache write
// (INT8 with one scale per token and KV head, or FP32), causal GQA attention
// over the cache, and the sigmoid gate.  B sequences of T new tokens each.
//
// Math (reference CPU operator, src/backend/cpu/core/attention/
// language_full_attn.cpp:77-108,156-207; INT8 cache recipe of
// fused_kv_cache_int8_kernel, full_attention_cuda.cu:75-155):
//   q_h = rmsnorm(q_h) * (1 + q_norm_w), k_g likewise, eps 1e-6
//   RoPE on dims d < rot, pairs (d, d+1): angle = pos / theta^(d / rot)
//   K/V INT8: scale = max|x| / 127 (1 when <= 1e-8), round half away, clamp 127
//   o_h = softmax(q_h . K_g^T / sqrt(hd)) V_g over positions 0 .. pos (causal),
//   g = h / (nh / nkv); out = o * sigmoid(gate)
//
// Three launches per segment of rows:
//   attn_prep     one workgroup per row: norms, RoPE, cache write, the
//                 normalized q to the workspace;
//   attn_split    (key split, KV head, row): the query heads of one KV group
//                 (one wave each) over one range of keys, online softmax,
//                 32-key tiles of K and V dequantized into LDS once for the
//                 whole group; a partial (o, max, sum) per split;
//   attn_combine  (row, head): merges the splits, gate, output.
// Splits are sized so that a step fills the chip: many for one long decode
// row, one per row for a prefill.  A token whose position lies outside the
// cache (or beyond the max_len the launch was sized for) writes nothing,
// outputs zeros and raises the context's device error flag.
#include "qw_stream.hpp"

namespace qwk {

constexpr int AT_KT = 32;  // keys per LDS tile

__device__ __forceinline__ float at_load(const void* p, int dt, int64_t i) {
    return dt == DT_F32 ? reinterpret_cast<const float*>(p)[i] : load_act(p, dt, i);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// ---------------------------------------------------------------------------
// prep: one workgroup (4 waves) per row; work items = nh q heads, nkv k
// heads, nkv v heads, one wave each; lane l holds dims [l*E, l*E + E).
template <int HD>
__global__ __launch_bounds__(256) void attn_prep(AttnArgs a) {
    constexpr int E = HD / 64;
    const int rl = blockIdx.x, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    // a position outside the cache, or past the keys the launch was sized for
    const bool ok = P >= 0 && P < a.cap && P < a.nsplit * a.split;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (!ok && threadIdx.x == 0) *a.err = 1u;
    const int items = a.nh + 2 * a.nkv;
    const int64_t row = (int64_t)r * a.ld_in;
    for (int it = wave; it < items; it += 4) {
        const bool isq = it < a.nh, isk = !isq && it < a.nh + a.nkv;
        const int h = isq ? it : (isk ? it - a.nh : it - a.nh - a.nkv);
        const void* src = isq ? a.q : (isk ? a.k : a.v);
        const int64_t base = row + (isq ? (int64_t)h * a.q_hs : (int64_t)h * HD) + lane * E;
        float x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = at_load(src, a.in_dt, base + e);
        if (isq || isk) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) ss += x[e] * x[e];
            ss = wave_sum(ss);
            const float rms = sqrtf(ss / (float)HD + 1e-6f);
            const float* w = isq ? a.qn_w : a.kn_w;
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = x[e] / rms * (1.0f + w[lane * E + e]);
#pragma unroll
            for (int e = 0; e < E; e += 2) {
                const int d = lane * E + e;
                if (d < a.rot) {
                    const float freq = 1.0f / powf(a.theta, (float)d / (float)a.rot);
                    const float ang = (float)P * freq;
                    const float c = cosf(ang), s = sinf(ang);
                    const float x0 = x[e], x1 = x[e + 1];
                    x[e] = x0 * c - x1 * s;
                    x[e + 1] = x0 * s + x1 * c;
                }
            }
        }
        if (isq) {
            float* dst = a.qn + ((int64_t)rl * a.nh + h) * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) dst[e] = x[e];
            continue;
        }
        if (!ok) continue;
        const int64_t slot = ((int64_t)b * a.cap + P) * a.nkv + h;
        if (a.kv_dt == DT_I8) {
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) m = fmaxf(m, fabsf(x[e]));
            m = wave_max(m);
            float sc = m / 127.0f;
            sc = sc > 1e-8f ? sc : 1.0f;
            int8_t* dst = reinterpret_cast<int8_t*>(isk ? a.kc : a.vc) + slot * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) dst[e] = (int8_t)fmaxf(-127.0f, fminf(127.0f, roundf(x[e] / sc)));
            if (lane == 0) (isk ? a.ks : a.vs)[slot] = sc;
        } else {
            float* dst = reinterpret_cast<float*>(isk ? a.kc : a.vc) + slot * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) dst[e] = x[e];
        }
    }
}

// ---------------------------------------------------------------------------
// split: (key split s, KV head g, row rl); wave w < G handles query head g*G + w.
template <int HD>
__global__ __launch_bounds__(256) void attn_split(AttnArgs a) {
    constexpr int E = HD / 64, KP = HD + 4;
    const int s = blockIdx.x, g = blockIdx.y, rl = blockIdx.z, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    const int L = (P >= 0 && P < a.cap && P < a.nsplit * a.split) ? P + 1 : 0;  // causal: keys 0 .. P
    const int k0 = s * a.split, k1 = min(k0 + a.split, L);
    if (k0 >= k1) return;  // uniform over the workgroup
    const int G = a.nh / a.nkv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = g * G + wave;

    __shared__ __attribute__((aligned(16))) float qs[4][HD];
    __shared__ __attribute__((aligned(16))) float Ks[AT_KT][KP], Vs[AT_KT][KP];

    for (int e = threadIdx.x; e < G * HD; e += 256) qs[e / HD][e % HD] = a.qn[((int64_t)rl * a.nh + g * G) * HD + e];
    const float scale = 1.0f / sqrtf((float)HD);
    float m = -INFINITY, l = 0.0f, o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
    const int kj = lane >> 1, half = lane & 1;  // score lane: key kj of the tile, half of the dims

    for (int kt = k0; kt < k1; kt += AT_KT) {
        const int n = min(AT_KT, k1 - kt);
        __syncthreads();  // the previous tile is consumed; qs is in place
        // K and V rows of the tile: 2 x n rows, 64 lanes x E dims per row
        for (int rr = threadIdx.x >> 6; rr < 2 * n; rr += 4) {
            const int j = rr >> 1;
            const bool isv = rr & 1;
            const int64_t slot = ((int64_t)b * a.cap + kt + j) * a.nkv + g;
            float* dst = (isv ? &Vs[j][0] : &Ks[j][0]) + lane * E;
            if (a.kv_dt == DT_I8) {
                const float sc = (isv ? a.vs : a.ks)[slot];
                const int8_t* src = reinterpret_cast<const int8_t*>(isv ? a.vc : a.kc) + slot * HD + lane * E;
#pragma unroll
                for (int e = 0; e < E; ++e) dst[e] = (float)src[e] * sc;
            } else {
                const float* src = reinterpret_cast<const float*>(isv ? a.vc : a.kc) + slot * HD + lane * E;
#pragma unroll
                for (int e = 0; e < E; ++e) dst[e] = src[e];
            }
        }
        __syncthreads();
        if (wave < G) {
            // scores: lane pair (kj, half) covers key kj
            float dot = 0.0f;
            if (kj < n) {
                const float* kr = &Ks[kj][half * (HD / 2)];
                const float* qr = &qs[wave][half * (HD / 2)];
#pragma unroll 8
                for (int d = 0; d < HD / 2; d += 4) {
                    const float4 kv = *reinterpret_cast<const float4*>(kr + d);
                    const float4 qv = *reinterpret_cast<const float4*>(qr + d);
                    dot += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
                }
            }
            dot += __shfl_xor(dot, 1);
            const float sc = kj < n ? dot * scale : -INFINITY;
            const float mt = wave_max(sc);
            const float mn = fmaxf(m, mt);
            const float corr = __expf(m - mn);  // m = -inf on the first tile: 0
            const float p = kj < n ? __expf(sc - mn) : 0.0f;
            l = l * corr + wave_sum(half == 0 ? p : 0.0f);
#pragma unroll
            for (int e = 0; e < E; ++e) o[e] *= corr;
            for (int j = 0; j < n; ++j) {
                const float pj = __shfl(p, 2 * j);
#pragma unroll
                for (int e = 0; e < E; ++e) o[e] += pj * Vs[j][lane * E + e];
            }
            m = mn;
        }
    }
    if (wave < G) {
        float* dst = a.part + (((int64_t)rl * a.nh + h) * a.nsplit + s) * (HD + 2);
#pragma unroll
        for (int e = 0; e < E; ++e) dst[lane * E + e] = o[e];
        if (lane == 0) {
            dst[HD] = m;
            dst[HD + 1] = l;
        }
    }
}

// ---------------------------------------------------------------------------
// combine: one wave per (row, head); merges the used splits, gate, output.
template <int HD>
__global__ __launch_bounds__(64) void attn_combine(AttnArgs a) {
    constexpr int E = HD / 64;
    const int rl = blockIdx.x, h = blockIdx.y, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    const int L = (P >= 0 && P < a.cap && P < a.nsplit * a.split) ? P + 1 : 0;
    const int lane = threadIdx.x;
    const int ns = (L + a.split - 1) / a.split;
    const float* pp = a.part + ((int64_t)rl * a.nh + h) * a.nsplit * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, pp[s * (HD + 2) + HD]);
    float l = 0.0f, o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
    for (int s = 0; s < ns; ++s) {
        const float w = __expf(pp[s * (HD + 2) + HD] - M);
        l += w * pp[s * (HD + 2) + HD + 1];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] += w * pp[s * (HD + 2) + lane * E + e];
    }
    const float inv = L > 0 ? 1.0f / l : 0.0f;
    const int64_t gi = (int64_t)r * a.ld_in + (int64_t)h * a.q_hs + lane * E;
    const int64_t oi = (int64_t)r * a.ld_out + (int64_t)h * HD + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float y = o[e] * inv * (1.0f / (1.0f + __expf(-at_load(a.gate, a.in_dt, gi + e))));
        if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = y;
        else store_act(a.out, a.out_dt, oi + e, y);
    }
}

size_t attn_bytes_per_row(int nh, int hd, int nsplit) {
    return (size_t)nh * hd * 4 + (size_t)nh * nsplit * (hd + 2) * 4;
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(attn_prep<HD>, dim3(a.rows), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(attn_split<HD>, dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(attn_combine<HD>, dim3(a.rows, a.nh), dim3(64), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t stream) {
    if (a.nkv < 1 || a.nh % a.nkv || a.nh / a.nkv > 4 || a.rot % 2 || a.rot > a.hd) return hipErrorInvalidValue;
    if (a.hd == 256) return launch_attn_hd<256>(a, stream);
    if (a.hd == 128) return launch_attn_hd<128>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace qwk
