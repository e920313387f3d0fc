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

// FP32 MFMA 16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
// D[4*(l/16) + r][l%16] in element r.
__device__ __forceinline__ f32x4 at_mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

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
// prep: one workgroup per row with one wave per work item (nh q heads, nkv k
// heads, nkv v heads; 64 x items threads); lane l holds dims [l*E, l*E + E).
template <int HD>
__global__ __launch_bounds__(1024) void attn_prep(AttnArgs a) {
    constexpr int E = HD / 64;
    const int rl = blockIdx.x, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    // a position outside the cache, or past the keys the launch was sized for
    const bool ok = P >= 0 && P < a.cap && P < a.nsplit * a.split;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (!ok && threadIdx.x == 0) *a.err = 1u;
    // the rotation of this position, shared by every q and k head
    __shared__ float rc[HD / 2], rs[HD / 2];
    if ((int)threadIdx.x < a.rot / 2) {
        const float freq = 1.0f / powf(a.theta, (float)(2 * threadIdx.x) / (float)a.rot);
        const float ang = (float)P * freq;
        rc[threadIdx.x] = cosf(ang);
        rs[threadIdx.x] = sinf(ang);
    }
    __syncthreads();
    const int items = a.nh + 2 * a.nkv;
    const int64_t row = (int64_t)r * a.ld_in;
    for (int it = wave; it < items; it += blockDim.x >> 6) {
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
                    const float c = rc[d / 2], s = rs[d / 2];
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
// The K and V tiles of 32 keys are staged in LDS once for the whole KV group:
// INT8 codes as they are (the scales multiply the score and the probability),
// FP32 values as they are; every thread issues its share of the next tile's
// loads before the current tile is computed.
template <int HD, bool I8>
struct AtTile {
    static constexpr int KROW = I8 ? HD + 4 : (HD + 4) * 4;   // K row stride, bytes (bank spread)
    static constexpr int VROW = I8 ? HD : HD * 4;             // V row stride, bytes
    static constexpr int CH = AT_KT * (I8 ? HD : HD * 4) / 16; // 16-byte chunks per K (or V) tile
    static constexpr int PER = 2 * CH / 256;                   // chunks per thread (K and V)
};

template <int HD, bool I8>
__global__ __launch_bounds__(256) void attn_split(AttnArgs a) {
    using Tl = AtTile<HD, I8>;
    constexpr int E = HD / 64, ESZ = I8 ? 1 : 4, CPR = HD * ESZ / 16;  // chunks per row
    const int s = blockIdx.x, g = blockIdx.y, rl = blockIdx.z, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    const int L = (P >= 0 && P < a.cap && P < a.nsplit * a.split) ? P + 1 : 0;  // causal: keys 0 .. P
    const int k0 = s * a.split, k1 = min(k0 + a.split, L);
    const int G = a.nh / a.nkv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = g * G + wave;
    if (k0 >= k1) {  // uniform over the workgroup
        if (L == 0 && a.nsplit == 1 && wave < G) {  // a flagged token without a combine step: zeros
            const int64_t oi = (int64_t)r * a.ld_out + (int64_t)h * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = 0.0f;
                else store_act(a.out, a.out_dt, oi + e, 0.0f);
            }
        }
        return;
    }

    __shared__ __attribute__((aligned(16))) float qs[4][HD];
    __shared__ __attribute__((aligned(16))) uint8_t Kt[AT_KT * Tl::KROW];
    __shared__ __attribute__((aligned(16))) uint8_t Vt[AT_KT * Tl::VROW];
    __shared__ float ksc[AT_KT], vsc[AT_KT];

    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.kc);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.vc);
    const int64_t slot0 = (int64_t)b * a.cap * a.nkv + g;  // slot of key j: slot0 + j * nkv
    u32x4 pre[Tl::PER];
    float psc = 0.0f;
    auto issue = [&](int kt) {  // the loads of the tile starting at key kt
        const int n = min(AT_KT, k1 - kt);
#pragma unroll
        for (int i = 0; i < Tl::PER; ++i) {
            const int c = threadIdx.x + 256 * i, isv = c >= Tl::CH, cc = c - isv * Tl::CH;
            const int j = cc / CPR, part = cc % CPR;
            const int64_t slot = slot0 + (int64_t)(kt + j) * a.nkv;
            if (j < n) pre[i] = *reinterpret_cast<const u32x4*>((isv ? vbase : kbase) + slot * (HD * ESZ) + part * 16);
            else pre[i] = u32x4{0u, 0u, 0u, 0u};
        }
        if (I8 && threadIdx.x < 2 * AT_KT) {
            const int j = threadIdx.x & (AT_KT - 1);
            psc = j < n ? (threadIdx.x < AT_KT ? a.ks : a.vs)[slot0 + (int64_t)(kt + j) * a.nkv] : 0.0f;
        }
    };
    issue(k0);
    for (int e = threadIdx.x; e < G * HD; e += 256) qs[e / HD][e % HD] = a.qn[((int64_t)rl * a.nh + g * G) * HD + e];
    const float scale = 1.0f / sqrtf((float)HD);
    float m = -INFINITY, l = 0.0f, o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
    const int kj = lane >> 1, half = lane & 1;  // score lane: key kj of the tile, half of the dims

    for (int kt = k0; kt < k1; kt += AT_KT) {
        const int n = min(AT_KT, k1 - kt);
        __syncthreads();  // the previous tile is consumed; qs is in place
#pragma unroll
        for (int i = 0; i < Tl::PER; ++i) {
            const int c = threadIdx.x + 256 * i, isv = c >= Tl::CH, cc = c - isv * Tl::CH;
            const int j = cc / CPR, part = cc % CPR;
            if (isv) {
                *reinterpret_cast<u32x4*>(&Vt[j * Tl::VROW + part * 16]) = pre[i];
            } else {
                uint32_t* d32 = reinterpret_cast<uint32_t*>(&Kt[j * Tl::KROW + part * 16]);
                d32[0] = pre[i][0]; d32[1] = pre[i][1]; d32[2] = pre[i][2]; d32[3] = pre[i][3];
            }
        }
        if (I8 && threadIdx.x < 2 * AT_KT) (threadIdx.x < AT_KT ? ksc : vsc)[threadIdx.x & (AT_KT - 1)] = psc;
        if (kt + AT_KT < k1) issue(kt + AT_KT);
        __syncthreads();
        if (wave < G) {
            float dot = 0.0f;
            if (kj < n) {
                const float* qr = &qs[wave][half * (HD / 2)];
                if (I8) {
                    const uint32_t* kr = reinterpret_cast<const uint32_t*>(&Kt[kj * Tl::KROW + half * (HD / 2)]);
#pragma unroll 8
                    for (int w = 0; w < HD / 8; ++w) {
                        const uint32_t c4 = kr[w];
                        const float4 qv = *reinterpret_cast<const float4*>(qr + 4 * w);
                        dot += qv.x * (float)(int8_t)(c4 & 0xff) + qv.y * (float)(int8_t)((c4 >> 8) & 0xff) +
                               qv.z * (float)(int8_t)((c4 >> 16) & 0xff) + qv.w * (float)(int8_t)(c4 >> 24);
                    }
                    dot *= ksc[kj];
                } else {
                    const float* kr = reinterpret_cast<const float*>(&Kt[kj * Tl::KROW]) + half * (HD / 2);
#pragma unroll 8
                    for (int d = 0; d < HD / 2; d += 4) {
                        const float4 kv = *reinterpret_cast<const float4*>(kr + d);
                        const float4 qv = *reinterpret_cast<const float4*>(qr + d);
                        dot += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
                    }
                }
            }
            dot += __shfl_xor(dot, 1);
            const float sc = kj < n ? dot * scale : -INFINITY;
            const float mt = wave_max(sc);
            const float mn = fmaxf(m, mt);
            const float corr = __expf(m - mn);  // m = -inf on the first tile: 0
            const float p = kj < n ? __expf(sc - mn) : 0.0f;
            l = l * corr + wave_sum(half == 0 ? p : 0.0f);
            const float pv = I8 ? p * vsc[kj < n ? kj : 0] : p;  // probability times the V row's scale
#pragma unroll
            for (int e = 0; e < E; ++e) o[e] *= corr;
            for (int j = 0; j < n; ++j) {
                const float pj = __shfl(pv, 2 * j);
                if (I8 && E == 4) {
                    const uint32_t c4 = reinterpret_cast<const uint32_t*>(&Vt[j * Tl::VROW])[lane];
#pragma unroll
                    for (int e = 0; e < E; ++e) o[e] += pj * (float)(int8_t)((c4 >> (8 * e)) & 0xff);
                } else if (I8) {
#pragma unroll
                    for (int e = 0; e < E; ++e) o[e] += pj * (float)(int8_t)Vt[j * Tl::VROW + lane * E + e];
                } else {
                    const float* vr = reinterpret_cast<const float*>(&Vt[j * Tl::VROW]) + lane * E;
#pragma unroll
                    for (int e = 0; e < E; ++e) o[e] += pj * vr[e];
                }
            }
            m = mn;
        }
    }
    if (wave >= G) return;
    if (a.nsplit == 1) {  // the only split: finish the row here
        const float inv = 1.0f / l;
        const int64_t gi = (int64_t)r * a.ld_in + (int64_t)h * a.q_hs + lane * E;
        const int64_t oi = (int64_t)r * a.ld_out + (int64_t)h * HD + lane * E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float y = o[e] * inv * (1.0f / (1.0f + __expf(-at_load(a.gate, a.in_dt, gi + e))));
            if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = y;
            else store_act(a.out, a.out_dt, oi + e, y);
        }
        return;
    }
    float* dst = a.part + (((int64_t)rl * a.nh + h) * a.nsplit + s) * (HD + 2);
#pragma unroll
    for (int e = 0; e < E; ++e) dst[lane * E + e] = o[e];
    if (lane == 0) {
        dst[HD] = m;
        dst[HD + 1] = l;
    }
}

// ---------------------------------------------------------------------------
// combine: one workgroup of NW waves per (row, head) (NW = 1 for up to 16
// splits, else 4).  The split maxima are reduced over all threads; each wave
// then sums the partial outputs of every NW-th split, eight splits' loads in
// flight; the wave sums are merged in LDS.
// Merge of ns split partials (o, max, sum) of one (row, head) by one wave,
// in a fixed order; COH: device-coherent loads (partials written by other
// workgroups of the same launch).  Returns the unnormalized o and the sum.
template <bool COH>
__device__ __forceinline__ float part_ld(const float* p) {
    if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

template <int HD, bool COH>
__device__ __forceinline__ void merge_splits_wave(const float* pp, int ns, int lane, float (&o)[HD / 64], float& l) {
    constexpr int E = HD / 64;
    float M = -INFINITY;
    for (int s = lane; s < ns; s += 64) M = fmaxf(M, part_ld<COH>(pp + s * (HD + 2) + HD));
    M = wave_max(M);
    l = 0.0f;
    for (int s = lane; s < ns; s += 64)
        l += __expf(part_ld<COH>(pp + s * (HD + 2) + HD) - M) * part_ld<COH>(pp + s * (HD + 2) + HD + 1);
    l = wave_sum(l);
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
    int s = 0;
    for (; s + 7 < ns; s += 8) {  // splits s .. s+7
        float w[8], v[8][E];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            w[u] = part_ld<COH>(pp + (s + u) * (HD + 2) + HD);
#pragma unroll
            for (int e = 0; e < E; ++e) v[u][e] = part_ld<COH>(pp + (s + u) * (HD + 2) + lane * E + e);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float wu = __expf(w[u] - M);
#pragma unroll
            for (int e = 0; e < E; ++e) o[e] += wu * v[u][e];
        }
    }
    for (; s < ns; ++s) {
        const float wu = __expf(part_ld<COH>(pp + s * (HD + 2) + HD) - M);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] += wu * part_ld<COH>(pp + s * (HD + 2) + lane * E + e);
    }
}

// out = o / l * sigmoid(gate) for the E dims of this lane
template <int HD>
__device__ __forceinline__ void gate_store(const AttnArgs& a, int r, int h, int lane, const float (&o)[HD / 64], float inv) {
    constexpr int E = HD / 64;
    const int64_t gi = (int64_t)r * a.ld_in + (int64_t)h * a.q_hs + lane * E;
    const int64_t oi = (int64_t)r * a.ld_out + (int64_t)h * HD + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float y = o[e] * inv * (1.0f / (1.0f + __expf(-at_load(a.gate, a.in_dt, gi + e))));
        if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = y;
        else store_act(a.out, a.out_dt, oi + e, y);
    }
}

// DC > 1 (many splits): blockIdx.z takes HD/DC of the head's dims, so more
// workgroups share the split partials' reads (each recomputes M and l from
// the splits' two floats).
template <int HD, int NW, int DC = 1>
__global__ __launch_bounds__(64 * NW) void attn_combine(AttnArgs a) {
    static_assert(DC == 1 || NW > 1, "dim chunks with the multi-wave merge");
    constexpr int E = HD / 64 / DC;  // dims per lane
    const int d0 = (int)blockIdx.z * (HD / DC);
    const int rl = blockIdx.x, h = blockIdx.y, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    const int L = (P >= 0 && P < a.cap && P < a.nsplit * a.split) ? P + 1 : 0;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ns = (L + a.split - 1) / a.split;
    const float* pp = a.part + ((int64_t)rl * a.nh + h) * a.nsplit * (HD + 2);
    __shared__ float red[2][NW];
    __shared__ __attribute__((aligned(16))) float osum[NW][HD / DC];
    if constexpr (NW == 1) {
        float o[E], l;
        merge_splits_wave<HD, false>(pp, ns, lane, o, l);
        gate_store<HD>(a, r, h, lane, o, L > 0 ? 1.0f / l : 0.0f);
        return;
    }
    float M = -INFINITY;
    for (int s = threadIdx.x; s < ns; s += 64 * NW) M = fmaxf(M, pp[s * (HD + 2) + HD]);
    M = wave_max(M);
    if (NW > 1) {
        if (lane == 0) red[0][wave] = M;
        __syncthreads();
        M = red[0][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) M = fmaxf(M, red[0][w]);
    }
    float l = 0.0f;
    for (int s = threadIdx.x; s < ns; s += 64 * NW) l += __expf(pp[s * (HD + 2) + HD] - M) * pp[s * (HD + 2) + HD + 1];
    l = wave_sum(l);
    if (NW > 1 && lane == 0) red[1][wave] = l;
    float o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.0f;
    int s = wave;
    for (; s + 7 * NW < ns; s += 8 * NW) {  // splits s, s+NW, ..., s+7NW
        float w[8], v[8][E];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            w[u] = pp[(s + NW * u) * (HD + 2) + HD];
#pragma unroll
            for (int e = 0; e < E; ++e) v[u][e] = pp[(s + NW * u) * (HD + 2) + d0 + lane * E + e];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float wu = __expf(w[u] - M);
#pragma unroll
            for (int e = 0; e < E; ++e) o[e] += wu * v[u][e];
        }
    }
    for (; s < ns; s += NW) {
        const float wu = __expf(pp[s * (HD + 2) + HD] - M);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] += wu * pp[s * (HD + 2) + d0 + lane * E + e];
    }
    if (NW > 1) {
#pragma unroll
        for (int e = 0; e < E; ++e) osum[wave][lane * E + e] = o[e];
        __syncthreads();
        if (wave != 0) return;
        l = red[1][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) l += red[1][w];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += osum[w][lane * E + e];
            o[e] = t;
        }
    }
    const float inv = L > 0 ? 1.0f / l : 0.0f;
    const int64_t gi = (int64_t)r * a.ld_in + (int64_t)h * a.q_hs + d0 + lane * E;
    const int64_t oi = (int64_t)r * a.ld_out + (int64_t)h * HD + d0 + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int d = lane * E + e;
        const float y = o[e] * inv * (1.0f / (1.0f + __expf(-at_load(a.gate, a.in_dt, gi + e))));
        if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = y;
        else store_act(a.out, a.out_dt, oi + e, y);
    }
}

// ---------------------------------------------------------------------------
// prefill: (16-token query block, KV head g, sequence b); wave w handles query
// head g*G + w for the 16 tokens of the block, all on FP32 MFMA (16x16x4):
//   S^T = K Q^T (32 keys x 16 queries per tile; Q in registers as the B
//   operand), causal mask, online softmax per query column, O^T += V^T P^T
//   (P^T is the score tile's own D layout: the B operand needs no shuffle).
// K and V tiles of 32 keys are staged in LDS once for the KV group (INT8
// codes with their scales folded into the scores and probabilities, or FP32).
template <int HD, bool I8>
__global__ __launch_bounds__(256) void attn_prefill(AttnArgs a) {
    using Tl = AtTile<HD, I8>;
    constexpr int ESZ = I8 ? 1 : 4, CPR = HD * ESZ / 16, KB = HD / 16, DT = HD / 16;
    const int qb = blockIdx.x, g = blockIdx.y, b = a.b0 + blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const int G = a.nh / a.nkv;
    const int h = g * G + min(wave, G - 1);
    const int tok0 = a.tb + qb * 16;
    const int P0 = a.pos[b];
    const int nq = min(16, a.tb + a.ntok - tok0);          // valid queries of the block
    const int plast = P0 + tok0 + nq - 1;                  // last query position
    const int pend = min(a.cap, a.nsplit * a.split);       // positions must stay below this
    const int L = P0 >= 0 ? min(plast, pend - 1) + 1 : 0;  // keys 0 .. last valid query position
    const int qpos = P0 + tok0 + li;                       // this lane's query position
    const bool qvalid = li < nq && P0 >= 0 && qpos < pend; // an invalid query outputs zeros

    __shared__ __attribute__((aligned(16))) uint8_t Kt[AT_KT * Tl::KROW];
    __shared__ __attribute__((aligned(16))) uint8_t Vt[AT_KT * Tl::VROW];
    __shared__ float ksc[AT_KT], vsc[AT_KT];

    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.kc);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.vc);
    const int64_t slot0 = (int64_t)b * a.cap * a.nkv + g;
    u32x4 pre[Tl::PER];
    float psc = 0.0f;
    auto issue = [&](int kt) {
        const int n = min(AT_KT, L - kt);
#pragma unroll
        for (int i = 0; i < Tl::PER; ++i) {
            const int c = threadIdx.x + 256 * i, isv = c >= Tl::CH, cc = c - isv * Tl::CH;
            const int j = cc / CPR, part = cc % CPR;
            const int64_t slot = slot0 + (int64_t)(kt + j) * a.nkv;
            if (j < n) pre[i] = *reinterpret_cast<const u32x4*>((isv ? vbase : kbase) + slot * (HD * ESZ) + part * 16);
            else pre[i] = u32x4{0u, 0u, 0u, 0u};
        }
        if (I8 && threadIdx.x < 2 * AT_KT) {
            const int j = threadIdx.x & (AT_KT - 1);
            psc = j < n ? (threadIdx.x < AT_KT ? a.ks : a.vs)[slot0 + (int64_t)(kt + j) * a.nkv] : 0.0f;
        }
    };
    if (L > 0) issue(0);

    // Q block of this wave's head in registers: lane (lg, li) holds Q[li][16kb + 4lg + q]
    f32x4 qr[KB];
    {
        const int64_t row = (int64_t)b * a.T + tok0 + li - a.row0;  // segment-local row
        const float* qp = a.qn + (row * a.nh + h) * HD + 4 * lg;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) qr[kb] = li < nq ? *reinterpret_cast<const f32x4*>(qp + 16 * kb) : f32x4{0, 0, 0, 0};
    }
    const float scale = 1.0f / sqrtf((float)HD);
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    for (int kt = 0; kt < L; kt += AT_KT) {
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int i = 0; i < Tl::PER; ++i) {
            const int c = threadIdx.x + 256 * i, isv = c >= Tl::CH, cc = c - isv * Tl::CH;
            const int j = cc / CPR, part = cc % CPR;
            if (isv) {
                *reinterpret_cast<u32x4*>(&Vt[j * Tl::VROW + part * 16]) = pre[i];
            } else {
                uint32_t* d32 = reinterpret_cast<uint32_t*>(&Kt[j * Tl::KROW + part * 16]);
                d32[0] = pre[i][0]; d32[1] = pre[i][1]; d32[2] = pre[i][2]; d32[3] = pre[i][3];
            }
        }
        if (I8 && threadIdx.x < 2 * AT_KT) (threadIdx.x < AT_KT ? ksc : vsc)[threadIdx.x & (AT_KT - 1)] = psc;
        if (kt + AT_KT < L) issue(kt + AT_KT);
        __syncthreads();
        if (wave >= G) continue;
        // S^T for keys kt + 16*sub + (4lg + r), queries li
        f32x4 sc[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            f32x4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
            const int key = 16 * sub + li;  // A operand row: key, k = dim
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                float k4[4];
                if (I8) {
                    const uint32_t c4 = *reinterpret_cast<const uint32_t*>(&Kt[key * Tl::KROW + 16 * kb + 4 * lg]);
#pragma unroll
                    for (int q = 0; q < 4; ++q) k4[q] = (float)(int8_t)((c4 >> (8 * q)) & 0xff);
                } else {
                    const f32x4 kv = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(&Kt[key * Tl::KROW]) + 16 * kb + 4 * lg);
#pragma unroll
                    for (int q = 0; q < 4; ++q) k4[q] = kv[q];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) sacc = at_mfma16(k4[q], qr[kb][q], sacc);
            }
            sc[sub] = sacc;
        }
        // scale, mask, running max per query column li
        float mt = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kl = 16 * sub + 4 * lg + r, kp = kt + kl;
                float v = sc[sub][r] * scale * (I8 ? ksc[kl] : 1.0f);
                v = (qvalid && kp <= qpos && kp < L) ? v : -INFINITY;
                sc[sub][r] = v;
                mt = fmaxf(mt, v);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float corr = mn == -INFINITY ? 1.0f : __expf(m - mn);
        float ps = 0.0f;
        f32x4 pb[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kl = 16 * sub + 4 * lg + r;
                const float p = mn == -INFINITY ? 0.0f : __expf(sc[sub][r] - mn);
                ps += p;
                pb[sub][r] = I8 ? p * vsc[kl] : p;  // B operand of P V: (key 4lg+r, query li)
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = acc[dt] * corr;
        // O^T[d][query] += V^T[d][key] P^T[key][query]
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int key = 16 * sub + 4 * lg + q, d = 16 * dt + li;
                    const float va = I8 ? (float)(int8_t)Vt[key * Tl::VROW + d]
                                        : reinterpret_cast<const float*>(&Vt[key * Tl::VROW])[d];
                    acc[dt] = at_mfma16(va, pb[sub][q], acc[dt]);
                }
    }
    if (wave >= G || li >= nq) return;
    // acc[dt] lane (lg, li) element r: O^T[16dt + 4lg + r][query li]
    const int64_t r = (int64_t)b * a.T + tok0 + li;
    const float inv = L > 0 && l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int d = 16 * dt + 4 * lg + rr;
            const float gt = at_load(a.gate, a.in_dt, r * a.ld_in + (int64_t)h * a.q_hs + d);
            const float y = acc[dt][rr] * inv * (1.0f / (1.0f + __expf(-gt)));
            const int64_t oi = r * a.ld_out + (int64_t)h * HD + d;
            if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi] = y;
            else store_act(a.out, a.out_dt, oi, y);
        }
}

// ---------------------------------------------------------------------------
// prefill over an INT8 cache on f16 MFMA (16x16x16): the cached codes are
// integers of at most 127 in magnitude, exact in f16, and their scales are
// applied in FP32 (to the scores, and to the probabilities before P V), so
// only q and p are rounded to f16 (relative 2^-11).  Same work decomposition
// as attn_prefill; each tile is converted to f16 once as it is staged (K by
// rows, V transposed, VhT[d][key], built from 4-key x 4-dim blocks), so the
// MFMA operands are single 64-bit LDS reads.
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// Four signed INT8 codes to f16 without conversions: each byte u = c + 128
// is placed under the f16 exponent of 1024 (bits 0x6400 | u = 1024 + u) by a
// byte permute, then one packed f16 subtraction of 1152 leaves c (exact).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x4 i8x4_to_h4(uint32_t c4) {
    const uint32_t u = c4 ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 x = __builtin_bit_cast(f16x2, lo) - off, y = __builtin_bit_cast(f16x2, hi) - off;
    return f16x4{x[0], x[1], y[0], y[1]};
}

// 4x4 byte transpose: byte q of o[e] = byte e of w[q] (four keys' codes of one
// dim from four keys' rows of four dims)
__device__ __forceinline__ void transpose4x4(const uint32_t w[4], uint32_t o[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
    const uint32_t t2 = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);
    const uint32_t t3 = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
    o[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_i8h(AttnArgs a) {
    constexpr int KB = HD / 16, DT = HD / 16;
    constexpr int KHP = HD + 8;           // f16 K row stride (elements)
    constexpr int VHP = AT_KT + 4;        // f16 V^T row stride (elements)
    constexpr int KCH = AT_KT * HD / 16;  // 16-code chunks of the K tile
    constexpr int KPER = KCH / 256;       // per thread
    constexpr int VBL = AT_KT * HD / 16;  // 4-key x 4-dim blocks of the V tile
    constexpr int VPER = VBL / 256;
    constexpr int KT4 = AT_KT / 4;        // lanes take consecutive 4-key groups: conflict-free V^T stores
    const int qb = blockIdx.x / a.nsplit, sp = blockIdx.x % a.nsplit, g = blockIdx.y, b = a.b0 + blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    const int G = a.nh / a.nkv;
    const int h = g * G + min(wave, G - 1);
    const int tok0 = a.tb + qb * 16;
    const int P0 = a.pos[b];
    const int nq = min(16, a.tb + a.ntok - tok0);
    const int plast = P0 + tok0 + nq - 1;
    const int pend = min(a.cap, a.nsplit * a.split);
    const int L = P0 >= 0 ? min(plast, pend - 1) + 1 : 0;
    const int qpos = P0 + tok0 + li;
    const bool qvalid = li < nq && P0 >= 0 && qpos < pend;
    // this workgroup's keys: [k0, k1) of the block's causal range
    const int k0 = sp * a.split, k1 = min(k0 + a.split, L);
    if (k0 >= k1 && !(k0 == 0 && a.nsplit == 1)) return;  // uniform; a lone split still writes zeros

    __shared__ __attribute__((aligned(16))) _Float16 Kh[AT_KT * KHP];
    __shared__ __attribute__((aligned(16))) _Float16 VhT[HD * VHP];
    __shared__ float ksc[AT_KT], vsc[AT_KT];

    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.kc);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.vc);
    const int64_t slot0 = (int64_t)b * a.cap * a.nkv + g;
    u32x4 kpre[KPER];
    uint32_t vpre[VPER][4];
    float psc = 0.0f;
    auto issue = [&](int kt) {
        const int n = min(AT_KT, k1 - kt);
#pragma unroll
        for (int i = 0; i < KPER; ++i) {  // K: 16 consecutive codes of one key
            const int c = threadIdx.x + 256 * i, j = c / (HD / 16), part = c % (HD / 16);
            // keys past the range read the range's last key: finite, masked out later
            kpre[i] = *reinterpret_cast<const u32x4*>(kbase + (slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv) * HD + part * 16);
        }
#pragma unroll
        for (int i = 0; i < VPER; ++i) {  // V: 4 dims of 4 consecutive keys
            const int blk = threadIdx.x + 256 * i, k4 = blk % (KT4), d4 = blk / (KT4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = 4 * k4 + q;
                vpre[i][q] = *reinterpret_cast<const uint32_t*>(vbase + (slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv) * HD + 4 * d4);
            }
        }
        if (threadIdx.x < 2 * AT_KT) {
            const int j = threadIdx.x & (AT_KT - 1);
            psc = (threadIdx.x < AT_KT ? a.ks : a.vs)[slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv];
        }
    };

    f16x4 qh[KB];
    {
        const int64_t row = (int64_t)b * a.T + tok0 + li - a.row0;
        const float* qp = a.qn + (row * a.nh + h) * HD + 4 * lg;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const f32x4 v = li < nq ? *reinterpret_cast<const f32x4*>(qp + 16 * kb) : f32x4{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q) qh[kb][q] = (_Float16)v[q];
        }
    }
    if (k0 < k1) issue(k0);  // after the q loads, so that waiting for q does not wait for the tile
    const float scale = 1.0f / sqrtf((float)HD);
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    for (int kt = k0; kt < k1; kt += AT_KT) {
        __syncthreads();
        // stage the tile as f16, converting every code once
#pragma unroll
        for (int i = 0; i < KPER; ++i) {
            const int c = threadIdx.x + 256 * i, j = c / (HD / 16), part = c % (HD / 16);
            f16x4 hv[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) hv[w] = i8x4_to_h4(kpre[i][w]);
            u32x4* dst = reinterpret_cast<u32x4*>(&Kh[j * KHP + part * 16]);
            dst[0] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
            dst[1] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hv[2], hv[3], 0, 1, 2, 3, 4, 5, 6, 7));
        }
#pragma unroll
        for (int i = 0; i < VPER; ++i) {
            const int blk = threadIdx.x + 256 * i, k4 = blk % (KT4), d4 = blk / (KT4);
            uint32_t tw[4];
            transpose4x4(vpre[i], tw);  // tw[e]: dim 4*d4 + e of keys 4*k4 .. 4*k4+3
#pragma unroll
            for (int e = 0; e < 4; ++e) *reinterpret_cast<f16x4*>(&VhT[(4 * d4 + e) * VHP + 4 * k4]) = i8x4_to_h4(tw[e]);
        }
        if (threadIdx.x < 2 * AT_KT) (threadIdx.x < AT_KT ? ksc : vsc)[threadIdx.x & (AT_KT - 1)] = psc;
        if (kt + AT_KT < k1) issue(kt + AT_KT);
        __syncthreads();
        if (wave >= G) continue;
        f32x4 sc[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            f32x4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
            const _Float16* kr = &Kh[(16 * sub + li) * KHP + 4 * lg];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(*reinterpret_cast<const f16x4*>(kr + 16 * kb), qh[kb], sacc, 0, 0, 0);
            sc[sub] = sacc;
        }
        float mt = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kl = 16 * sub + 4 * lg + r, kp = kt + kl;
                float v = sc[sub][r] * scale * ksc[kl];
                v = (qvalid && kp <= qpos && kp < k1) ? v : -INFINITY;
                sc[sub][r] = v;
                mt = fmaxf(mt, v);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float corr = mn == -INFINITY ? 1.0f : __expf(m - mn);
        float ps = 0.0f;
        f16x4 pb[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kl = 16 * sub + 4 * lg + r;
                const float p = mn == -INFINITY ? 0.0f : __expf(sc[sub][r] - mn);
                ps += p;
                pb[sub][r] = (_Float16)(p * vsc[kl]);
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = acc[dt] * corr;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    *reinterpret_cast<const f16x4*>(&VhT[(16 * dt + li) * VHP + 16 * sub + 4 * lg]), pb[sub], acc[dt],
                    0, 0, 0);
    }
    if (wave >= G || li >= nq) return;
    const int64_t r = (int64_t)b * a.T + tok0 + li;
    if (a.nsplit > 1) {  // a partial (o, max, sum) for the combine kernel
        if (!qvalid || qpos < k0) return;  // never read for this query
        float* dst = a.part + (((r - a.row0) * a.nh + h) * a.nsplit + sp) * (HD + 2);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) dst[16 * dt + 4 * lg + rr] = acc[dt][rr];
        if (lg == 0) {
            dst[HD] = m;
            dst[HD + 1] = l;
        }
        return;
    }
    const float inv = L > 0 && l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int d = 16 * dt + 4 * lg + rr;
            const float gt = at_load(a.gate, a.in_dt, r * a.ld_in + (int64_t)h * a.q_hs + d);
            const float y = acc[dt][rr] * inv * (1.0f / (1.0f + __expf(-gt)));
            const int64_t oi = r * a.ld_out + (int64_t)h * HD + d;
            if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi] = y;
            else store_act(a.out, a.out_dt, oi, y);
        }
}

// ---------------------------------------------------------------------------
// decode over an INT8 cache on f16 MFMA: (key split, KV head g, row).  The
// group's query heads are the MFMA columns (B = Q^T, 16 columns of which G
// are used); a 64-key tile is staged as f16 once (K rows, V transposed) and
// wave w takes its 16-key quarter: S^T = K Q^T, an online softmax of its own
// per column, O^T += V^T P^T.  The four waves' (max, sum, O) are merged in LDS
// at the end; a lone split writes the output, otherwise a partial.
constexpr int AD_KT = 64;  // keys per tile

// FUSED (one new token per sequence): the kernel also does the work of
// attn_prep and attn_combine, saving two launches per decode step:
//   * every workgroup normalizes and rotates its G query heads itself (one
//     wave each) from the projection output;
//   * the workgroup whose key range holds the new position P computes the
//     new token's K and V of its KV head (norm, RoPE, INT8 codes and scale,
//     as attn_prep), writes them to the cache for later steps, and puts the
//     same codes and scales into its LDS tile in place of the cache's (so
//     nothing in this launch reads the slot it writes);
//   * the splits of a (row, KV head) hand their partials over with
//     agent-scope stores and an arrival count; the last one to arrive merges
//     them (merge_splits_wave, as attn_combine) and writes the gated output.
// No workgroup waits for another, so the launch cannot stall.
template <int HD, bool FUSED, bool VCOAL>
__global__ __launch_bounds__(256) void attn_decode_i8h(AttnArgs a) {
    constexpr int KB = HD / 16, DT = HD / 16, E = HD / 64;
    constexpr int KHP = HD + 8, VHP = AD_KT + 4;
    constexpr int KPER = AD_KT * HD / 16 / 256;  // 16-code K chunks per thread
    // V tile loads, two patterns (VCOAL chosen per launch):
    //   VCOAL: 16 codes of each of 4 consecutive keys per thread, consecutive
    //     threads on consecutive 16-byte chunks of a key row (coalesced rows);
    //   else: 4 codes of each of 4 consecutive keys per thread, consecutive
    //     threads on consecutive key groups (conflict-free V^T stores).
    // Measured: the coalesced rows win once the launch fills the chip (B=32,
    // context 4096: 84 vs 97 us; B=1, context 32768: 42 vs 43 us) and lose
    // with few workgroups (B=1, context 4096, 64 workgroups: 33 vs 24 us).
    constexpr int VNG = AD_KT / 4 * (HD / 16);  // 4-key x 16-dim groups of the V tile
    constexpr int VPG = (VNG + 255) / 256;      // per thread
    constexpr int VPER = AD_KT * HD / 16 / 256;  // 4x4 V blocks per thread (scattered pattern)
    constexpr int KT4 = AD_KT / 4;
    const int s = blockIdx.x, g = blockIdx.y, rl = blockIdx.z, r = a.row0 + rl;
    const int b = r / a.T, t = r % a.T;
    const int P = a.pos[b] + t;
    const int L = (P >= 0 && P < a.cap && P < a.nsplit * a.split) ? P + 1 : 0;
    const int k0 = s * a.split, k1 = min(k0 + a.split, L);
    const int G = a.nh / a.nkv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
    if (k0 >= k1) {  // uniform over the workgroup
        if (FUSED && L == 0 && s == 0 && g == 0 && threadIdx.x == 0) *a.err = 1u;
        if (L == 0 && (a.nsplit == 1 || (FUSED && s == 0)) && wave < G) {
            const int64_t oi = (int64_t)r * a.ld_out + (int64_t)(g * G + wave) * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi + e] = 0.0f;
                else store_act(a.out, a.out_dt, oi + e, 0.0f);
            }
        }
        return;
    }

    __shared__ __attribute__((aligned(16))) _Float16 Kh[AD_KT * KHP];
    __shared__ __attribute__((aligned(16))) _Float16 VhT[HD * VHP];
    __shared__ float ksc[AD_KT], vsc[AD_KT];
    __shared__ float wm[4][16], wl[4][16];

    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.kc);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.vc);
    const int64_t slot0 = (int64_t)b * a.cap * a.nkv + g;
    u32x4 kpre[KPER];
    u32x4 vpre[VCOAL ? VPG : 1][4];
    uint32_t vpre4[VCOAL ? 1 : VPER][4];
    float psc = 0.0f;
    auto issue = [&](int kt) {
        const int n = min(AD_KT, k1 - kt);
#pragma unroll
        for (int i = 0; i < KPER; ++i) {
            const int c = threadIdx.x + 256 * i, j = c / (HD / 16), part = c % (HD / 16);
            // keys past the range read the range's last key: finite, masked out later
            kpre[i] = *reinterpret_cast<const u32x4*>(kbase + (slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv) * HD + part * 16);
        }
        if constexpr (VCOAL) {
            for (int i = 0; i < VPG; ++i) {  // V: 16 codes of each of 4 consecutive keys
                const int grp = threadIdx.x + 256 * i, c = grp % (HD / 16), k4 = grp / (HD / 16);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = 4 * k4 + q;
                    if (VNG % 256 == 0 || grp < VNG)
                        vpre[i][q] = *reinterpret_cast<const u32x4*>(vbase + (slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv) * HD + 16 * c);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < VPER; ++i) {  // V: 4 codes of each of 4 consecutive keys
                const int blk = threadIdx.x + 256 * i, k4 = blk % (KT4), d4 = blk / (KT4);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = 4 * k4 + q;
                    vpre4[i][q] = *reinterpret_cast<const uint32_t*>(vbase + (slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv) * HD + 4 * d4);
                }
            }
        }
        if (threadIdx.x < 2 * AD_KT) {
            const int j = threadIdx.x & (AD_KT - 1);
            psc = (threadIdx.x < AD_KT ? a.ks : a.vs)[slot0 + (int64_t)(kt + min(j, n - 1)) * a.nkv];
        }
    };
    // fused: q of the G heads (wave w: head g*G + w), and -- in the workgroup
    // that holds position P -- the new K and V of head g, as attn_prep
    const bool owner = FUSED && k1 == L;  // this split's range ends at P
    __shared__ __attribute__((aligned(16))) float qs[FUSED ? 4 : 1][FUSED ? HD : 1];
    __shared__ float rc[FUSED ? HD / 2 : 1], rs[FUSED ? HD / 2 : 1];
    __shared__ int8_t newkv[FUSED ? 2 : 1][FUSED ? HD : 1];
    __shared__ float newsc[2];
    if constexpr (FUSED) {
        // the first tile's loads go out before the q work: they do not depend
        // on it (a stale slot P is replaced in LDS below), and the q loads
        // then wait for the tile instead of the tile waiting for the q work
        issue(k0);
        if ((int)threadIdx.x < a.rot / 2) {
            const float freq = 1.0f / powf(a.theta, (float)(2 * threadIdx.x) / (float)a.rot);
            const float ang = (float)P * freq;
            rc[threadIdx.x] = cosf(ang);
            rs[threadIdx.x] = sinf(ang);
        }
        __syncthreads();
        const int64_t row = (int64_t)r * a.ld_in;
        // items: q head g*G + it for it < G; then (owner) it = G: k, G+1: v of head g
        for (int it = wave; it < G + (owner ? 2 : 0); it += 4) {
            const bool isq = it < G, isk = it == G;
            const void* src = isq ? a.q : (isk ? a.k : a.v);
            const int64_t base = row + (isq ? (int64_t)(g * G + it) * a.q_hs : (int64_t)g * HD) + lane * E;
            float x[E];
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = at_load(src, a.in_dt, base + e);
            if (it <= G) {  // q or k: RMSNorm (1 + w), then RoPE on d < rot
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
                        const float c = rc[d / 2], sn = rs[d / 2];
                        const float x0 = x[e], x1 = x[e + 1];
                        x[e] = x0 * c - x1 * sn;
                        x[e + 1] = x0 * sn + x1 * c;
                    }
                }
            }
            if (isq) {
#pragma unroll
                for (int e = 0; e < E; ++e) qs[it][lane * E + e] = x[e];
                continue;
            }
            // the new token's INT8 codes and scale (kv 0: K, 1: V)
            const int kv = isk ? 0 : 1;
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) m = fmaxf(m, fabsf(x[e]));
            m = wave_max(m);
            float sc = m / 127.0f;
            sc = sc > 1e-8f ? sc : 1.0f;
            const int64_t slot = ((int64_t)b * a.cap + P) * a.nkv + g;
            int8_t* cdst = reinterpret_cast<int8_t*>(isk ? a.kc : a.vc) + slot * HD + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int8_t c = (int8_t)fmaxf(-127.0f, fminf(127.0f, roundf(x[e] / sc)));
                cdst[e] = c;
                newkv[kv][lane * E + e] = c;
            }
            if (lane == 0) {
                (isk ? a.ks : a.vs)[slot] = sc;
                newsc[kv] = sc;
            }
        }
        __syncthreads();
    }
    // B operand: column li = query head g*G + li of this row (zero for li >= G)
    f16x4 qh[KB];
    {
        const float* qp = FUSED ? &qs[min(li, G - 1)][4 * lg]
                                : a.qn + ((int64_t)rl * a.nh + g * G + min(li, G - 1)) * HD + 4 * lg;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const f32x4 v = li < G ? *reinterpret_cast<const f32x4*>(qp + 16 * kb) : f32x4{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q) qh[kb][q] = (_Float16)v[q];
        }
    }
    if constexpr (!FUSED) issue(k0);  // after the q loads, so that waiting for q does not wait for the tile
    const float scale = 1.0f / sqrtf((float)HD);
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    for (int kt = k0; kt < k1; kt += AD_KT) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < KPER; ++i) {
            const int c = threadIdx.x + 256 * i, j = c / (HD / 16), part = c % (HD / 16);
            f16x4 hv[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) hv[w] = i8x4_to_h4(kpre[i][w]);
            u32x4* dst = reinterpret_cast<u32x4*>(&Kh[j * KHP + part * 16]);
            dst[0] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
            dst[1] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hv[2], hv[3], 0, 1, 2, 3, 4, 5, 6, 7));
        }
        if constexpr (VCOAL) {
            for (int i = 0; i < VPG; ++i) {
                const int grp = threadIdx.x + 256 * i, c = grp % (HD / 16), k4 = grp / (HD / 16);
                if (VNG % 256 == 0 || grp < VNG) {
#pragma unroll
                    for (int blk = 0; blk < 4; ++blk) {
                        const uint32_t w4[4] = {vpre[i][0][blk], vpre[i][1][blk], vpre[i][2][blk], vpre[i][3][blk]};
                        uint32_t tw[4];
                        transpose4x4(w4, tw);  // tw[e]: dim 16*c + 4*blk + e of keys 4*k4 .. 4*k4+3
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            *reinterpret_cast<f16x4*>(&VhT[(16 * c + 4 * blk + e) * VHP + 4 * k4]) = i8x4_to_h4(tw[e]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < VPER; ++i) {
                const int blk = threadIdx.x + 256 * i, k4 = blk % (KT4), d4 = blk / (KT4);
                uint32_t tw[4];
                transpose4x4(vpre4[i], tw);  // tw[e]: dim 4*d4 + e of keys 4*k4 .. 4*k4+3
#pragma unroll
                for (int e = 0; e < 4; ++e) *reinterpret_cast<f16x4*>(&VhT[(4 * d4 + e) * VHP + 4 * k4]) = i8x4_to_h4(tw[e]);
            }
        }
        if (threadIdx.x < 2 * AD_KT) (threadIdx.x < AD_KT ? ksc : vsc)[threadIdx.x & (AD_KT - 1)] = psc;
        if (kt + AD_KT < k1) issue(kt + AD_KT);
        __syncthreads();
        if (owner && P < kt + AD_KT) {  // the tile of position P: its K/V from this launch, not the cache
            const int jp = P - kt;
            for (int d = threadIdx.x; d < HD; d += 256) {
                Kh[jp * KHP + d] = (_Float16)newkv[0][d];
                VhT[d * VHP + jp] = (_Float16)newkv[1][d];
            }
            if (threadIdx.x < 2) (threadIdx.x == 0 ? ksc : vsc)[jp] = newsc[threadIdx.x];
            __syncthreads();
        }
        const int kw = 16 * wave;  // this wave's quarter of the tile
        if (kt + kw >= k1) continue;
        f32x4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
        const _Float16* kr = &Kh[(kw + li) * KHP + 4 * lg];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(*reinterpret_cast<const f16x4*>(kr + 16 * kb), qh[kb], sacc, 0, 0, 0);
        float mt = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int kl = kw + 4 * lg + q;
            const float v = kt + kl < k1 ? sacc[q] * scale * ksc[kl] : -INFINITY;
            sacc[q] = v;
            mt = fmaxf(mt, v);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);  // finite: the quarter has at least one key
        const float corr = __expf(m - mn);
        float ps = 0.0f;
        f16x4 pb;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float p = __expf(sacc[q] - mn);
            ps += p;
            pb[q] = (_Float16)(p * vsc[kw + 4 * lg + q]);
        }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            acc[dt] = acc[dt] * corr;
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                *reinterpret_cast<const f16x4*>(&VhT[(16 * dt + li) * VHP + kw + 4 * lg]), pb, acc[dt], 0, 0, 0);
        }
    }
    // merge the four waves: column li of each wave's (m, l, O^T)
    __syncthreads();  // the tiles are no longer read; reuse VhT for the wave outputs
    float* ow = reinterpret_cast<float*>(VhT);  // [4 waves][G cols][HD]
    if (lg == 0) {
        wm[wave][li] = m;
        wl[wave][li] = l;
    }
    if (li < G) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(&ow[(wave * 4 + li) * HD + 16 * dt + 4 * lg]) = acc[dt];
    }
    __syncthreads();
    // wave w < G finishes query head g*G + w: merge the four waves' columns
    auto wave_merge = [&](float (&o)[E], float& M, float& lt) {
        const int col = wave;
        M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][col]);
        float wsc[4];
        lt = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            wsc[w] = wm[w][col] == -INFINITY ? 0.0f : __expf(wm[w][col] - M);
            lt += wsc[w] * wl[w][col];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = lane * E + e;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) v += wsc[w] * ow[(w * 4 + col) * HD + d];
            o[e] = v;
        }
    };
    const int h = g * G + wave;
    if constexpr (!FUSED) {
        if (wave >= G) return;
        float o[E], M, lt;
        wave_merge(o, M, lt);
        if (a.nsplit == 1) {
            gate_store<HD>(a, r, h, lane, o, 1.0f / lt);
            return;
        }
        float* dst = a.part + (((int64_t)rl * a.nh + h) * a.nsplit + s) * (HD + 2);
#pragma unroll
        for (int e = 0; e < E; ++e) dst[lane * E + e] = o[e];
        if (lane == 0) {
            dst[HD] = M;
            dst[HD + 1] = lt;
        }
    } else {
        const int ns = (L + a.split - 1) / a.split;  // splits holding keys of this row
        __shared__ unsigned last_s;
        if (wave < G) {
            float o[E], M, lt;
            wave_merge(o, M, lt);
            if (ns == 1) {
                gate_store<HD>(a, r, h, lane, o, 1.0f / lt);
            } else {
                // hand-off: agent-scope stores of the partial
                float* dst = a.part + (((int64_t)rl * a.nh + h) * a.nsplit + s) * (HD + 2);
#pragma unroll
                for (int e = 0; e < E; ++e)
                    __hip_atomic_store(dst + lane * E + e, o[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (lane == 0) {
                    __hip_atomic_store(dst + HD, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(dst + HD + 1, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (ns > 1) {  // uniform over the workgroup
            // every wave waits for its stores' completion, then one arrival
            // count per workgroup; the last split of (row, g) merges them all
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x == 0) {
                unsigned* cnt = a.cnt + (int64_t)rl * a.nkv + g;
                const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_s = old == (unsigned)(ns - 1) ? 1u : 0u;
                if (old == (unsigned)(ns - 1)) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (last_s && wave < G) {
                const float* pp = a.part + ((int64_t)rl * a.nh + h) * a.nsplit * (HD + 2);
                float om[E], l;
                merge_splits_wave<HD, true>(pp, ns, lane, om, l);
                gate_store<HD>(a, r, h, lane, om, 1.0f / l);
            }
        }
    }
}

size_t attn_bytes_per_row(int nh, int hd, int nsplit) {
    return (size_t)nh * hd * 4 + (size_t)nh * nsplit * (hd + 2) * 4;
}

template <int HD>
static void launch_combine(const AttnArgs& a, hipStream_t stream) {
    if (a.nsplit <= 1) return;
    if (a.nsplit <= 16) hipLaunchKernelGGL((attn_combine<HD, 1>), dim3(a.rows, a.nh), dim3(64), 0, stream, a);
    else hipLaunchKernelGGL((attn_combine<HD, 4, HD / 64>), dim3(a.rows, a.nh, HD / 64), dim3(256), 0, stream, a);
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs& a, hipStream_t stream) {
    if (a.prefill) {
        hipLaunchKernelGGL(attn_prep<HD>, dim3(a.rows), dim3(64 * std::min(16, a.nh + 2 * a.nkv)), 0, stream, a);
        // INT8: query blocks x key splits (f16 MFMA), merged by attn_combine;
        // FP32: one workgroup per query block over all its keys (FP32 MFMA)
        if (a.kv_dt == DT_I8) {
            hipLaunchKernelGGL(attn_prefill_i8h<HD>, dim3((a.ntok + 15) / 16 * a.nsplit, a.nkv, a.nb), dim3(256), 0,
                               stream, a);
            launch_combine<HD>(a, stream);
        } else {
            hipLaunchKernelGGL((attn_prefill<HD, false>), dim3((a.ntok + 15) / 16, a.nkv, a.nb), dim3(256), 0, stream, a);
        }
        return hipGetLastError();
    }
    if (a.kv_dt == DT_I8 && a.T == 1 && a.cnt) {  // one launch: prep and combine inside
        if (a.vcoal) hipLaunchKernelGGL((attn_decode_i8h<HD, true, true>), dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((attn_decode_i8h<HD, true, false>), dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(attn_prep<HD>, dim3(a.rows), dim3(64 * std::min(16, a.nh + 2 * a.nkv)), 0, stream, a);
    if (a.kv_dt == DT_I8 && a.vcoal) hipLaunchKernelGGL((attn_decode_i8h<HD, false, true>), dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
    else if (a.kv_dt == DT_I8) hipLaunchKernelGGL((attn_decode_i8h<HD, false, false>), dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((attn_split<HD, false>), dim3(a.nsplit, a.nkv, a.rows), dim3(256), 0, stream, a);
    launch_combine<HD>(a, stream);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t stream) {
    if (a.nkv < 1 || a.nh % a.nkv || a.nh / a.nkv > 4 || a.rot % 2 || a.rot > a.hd) return hipErrorInvalidValue;
    if (a.hd == 256) return launch_attn_hd<256>(a, stream);
    if (a.hd == 128) return launch_attn_hd<128>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace qwk
