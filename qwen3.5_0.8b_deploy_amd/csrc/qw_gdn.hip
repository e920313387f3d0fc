// qw_gdn.hip -- Gated-DeltaNet decode step for gfx950: everything between the
// input projections (QKV, Z, a, b) and the out projection of a linear-
// attention layer, for T consecutive tokens of each of B sequences (T = 1 is
// the decode step; T > 1 is the serial prefill of the reference's
// forward_batch, linear_attention_cuda.cu:529-680, whose contract is
// equality with T single-token steps, verify_linear_attn_batch.cu:68-112).
//
// Math (reference CPU operator, src/backend/cpu/core/attention/
// language_linear_attn.cpp:143-256; CUDA chain conv1d_update_fused /
// l2norm_qk_fused / gated_delta / norm_gate_fused, linear_attention_cuda.cu:
// 47-172):
//   conv:  c[d] = silu(w[d][K-1]*x[d] + sum_j<K-1 w[d][j]*st[d][j]), then
//          st[d][j] = st[d][j-1] (j > 0), st[d][0] = x[d]   (st[d][0] newest)
//   q, k:  per head L2-normalized (eps 1e-6 under the root), q * 1/sqrt(kd)
//   gates: beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)
//   state: S *= exp(g); kv = S^T k; delta = (v - kv) * beta; S += k delta^T;
//          o = S^T q                                  (S: kd x vd, FP32)
//   out:   o * rsqrt(mean(o^2) + 1e-6) * norm_w * silu(z)   per head
//
// Work decomposition.  One workgroup of 256 threads per (sequence, head).
// The head's 2*kd + vd conv channels are spread over the threads (two at
// most per thread), each keeping its conv taps and state in registers; q, k,
// v land in LDS per token.  The state S[kd][vd] of the head (64 KB) is read
// once before the first token and written once after the last: thread t owns
// column t % vd for rows [64*(t/vd), +64), so every load and store of a row
// is one coalesced 512-byte access, the column sums kv and o need one two-way
// combine in LDS, and the update happens in registers between the two.
// Bound: at T = 1 HBM (state read + write, ~2 x 64 KB per head); at T > 1
// the per-token barrier chain (the recurrence is serial in T).
#include "qw_stream.hpp"

namespace qwk {

constexpr int GDN_T = 256;

__device__ __forceinline__ float gdn_load(const void* p, int dt, int64_t i) {
    return dt == DT_F32 ? reinterpret_cast<const float*>(p)[i] : load_act(p, dt, i);
}

template <int KD, int VD>
__global__ __launch_bounds__(GDN_T) void gdn_kernel(GdnArgs a) {
    static_assert(GDN_T % VD == 0 && KD % (GDN_T / VD) == 0, "state split");
    static_assert(2 * KD + VD <= 2 * GDN_T, "two conv channels per thread at most");
    constexpr int RH = GDN_T / VD;   // row groups
    constexpr int RPT = KD / RH;     // state rows per thread
    constexpr int SLMAX = 7;         // conv taps kept in registers (K <= 8)
    const int h = blockIdx.x, b = blockIdx.y;
    const int t = threadIdx.x;
    const int nh = a.nh;
    const int K = a.K, SL = a.K - 1;
    const int conv_dim = 2 * nh * KD + nh * VD;
    const int wave = t >> 6, lane = t & 63;

    __shared__ float qs[KD], ks[KD], vs[VD];
    __shared__ float red[RH][VD];
    __shared__ float scal[4];  // |q|, |k|, beta, exp(g)
    __shared__ float wsum[GDN_T / 64];

    // ---- per-thread conv channels (up to two) and their state, in registers ----
    int cd[2];
    float* cdst[2];
    float cw[2][SLMAX + 1], cst[2][SLMAX];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int c = t + u * GDN_T;
        cd[u] = -1;
        cdst[u] = nullptr;
        if (c < 2 * KD + VD) {
            if (c < KD) { cd[u] = h * KD + c; cdst[u] = &qs[c]; }
            else if (c < 2 * KD) { cd[u] = nh * KD + h * KD + (c - KD); cdst[u] = &ks[c - KD]; }
            else { cd[u] = 2 * nh * KD + h * VD + (c - 2 * KD); cdst[u] = &vs[c - 2 * KD]; }
        }
#pragma unroll
        for (int j = 0; j <= SLMAX; ++j) cw[u][j] = (cd[u] >= 0 && j < K) ? a.conv_w[(int64_t)cd[u] * K + j] : 0.0f;
#pragma unroll
        for (int j = 0; j < SLMAX; ++j)
            cst[u][j] = (cd[u] >= 0 && j < SL) ? a.conv_state[((int64_t)b * conv_dim + cd[u]) * SL + j] : 0.0f;
    }
    // ---- the head's state rows of this thread, resident for all tokens ----
    float* S = a.rec_state + ((int64_t)b * nh + h) * KD * VD;
    const int col = t % VD, r0 = (t / VD) * RPT;
    float s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = S[(r0 + i) * VD + col];
    const float q_scale = 1.0f / sqrtf((float)KD);
    const float expA = __expf(a.A_log[h]);

    for (int tok = 0; tok < a.T; ++tok) {
        const int64_t in_row = ((int64_t)b * a.T + tok) * a.ld_in;
        // ---- conv1d + SiLU, state shift (st[0] newest) ----
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (cd[u] < 0) continue;
            const float xv = gdn_load(a.mixed, a.in_dt, in_row + cd[u]);
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j <= SLMAX; ++j)
                if (j == K - 1) sum = cw[u][j] * xv;
#pragma unroll
            for (int j = 0; j < SLMAX; ++j)
                if (j < SL) sum += cw[u][j] * cst[u][j];
#pragma unroll
            for (int j = SLMAX - 1; j > 0; --j) cst[u][j] = cst[u][j - 1];
            cst[u][0] = xv;
            *cdst[u] = silu_f(sum);
        }
        __syncthreads();

        // ---- L2 norms of q and k (waves 0 and 1), gates (thread 128) ----
        if (wave < 2) {
            const float* v = wave == 0 ? qs : ks;
            float ss = 0.0f;
            for (int d = lane; d < KD; d += 64) ss += v[d] * v[d];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            if (lane == 0) scal[wave] = sqrtf(ss + 1e-6f);
        } else if (t == 128) {
            const float av = gdn_load(a.a, a.in_dt, in_row + h) + a.dt_bias[h];
            const float bv = gdn_load(a.b, a.in_dt, in_row + h);
            const float sp = av > 20.0f ? av : logf(1.0f + __expf(av));
            scal[2] = 1.0f / (1.0f + __expf(-bv));
            scal[3] = __expf(-expA * sp);
        }
        __syncthreads();
        for (int d = t; d < KD; d += GDN_T) {
            qs[d] = qs[d] / scal[0] * q_scale;
            ks[d] = ks[d] / scal[1];
        }
        __syncthreads();

        // ---- delta rule on this thread's column slice ----
        const float beta = scal[2], gt = scal[3];
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            s[i] *= gt;
            kv += s[i] * ks[r0 + i];
        }
        red[t / VD][col] = kv;
        __syncthreads();
        float kvs = 0.0f;
#pragma unroll
        for (int g = 0; g < RH; ++g) kvs += red[g][col];
        const float delta = (vs[col] - kvs) * beta;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            s[i] += ks[r0 + i] * delta;
            o += s[i] * qs[r0 + i];
        }
        __syncthreads();  // every thread has read red[] for kv
        red[t / VD][col] = o;
        __syncthreads();

        // ---- per-head RMSNorm x norm_w x SiLU(z): threads 0 .. VD-1 own a
        // column; every wave takes part in the reduction and its barrier ----
        float os = 0.0f;
        if (t < VD) {
#pragma unroll
            for (int g = 0; g < RH; ++g) os += red[g][t];
        }
        float ss = os * os;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0) wsum[wave] = ss;
        __syncthreads();
        if (t < VD) {
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < GDN_T / 64; ++w) tot += wsum[w];
            const float inv = 1.0f / sqrtf(tot / (float)VD + 1e-6f);
            const float zv = gdn_load(a.z, a.in_dt, in_row + h * VD + t);
            const float y = os * inv * a.norm_w[t] * silu_f(zv);
            const int64_t oi = ((int64_t)b * a.T + tok) * a.ld_out + h * VD + t;
            if (a.out_dt == DT_F32) reinterpret_cast<float*>(a.out)[oi] = y;
            else store_act(a.out, a.out_dt, oi, y);
        }
        // the next token rewrites qs/ks/vs, red and wsum only after this barrier
        __syncthreads();
    }

    // ---- write back the state: recurrent once, conv taps once ----
#pragma unroll
    for (int i = 0; i < RPT; ++i) S[(r0 + i) * VD + col] = s[i];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        if (cd[u] < 0) continue;
#pragma unroll
        for (int j = 0; j < SLMAX; ++j)
            if (j < SL) a.conv_state[((int64_t)b * conv_dim + cd[u]) * SL + j] = cst[u][j];
    }
}

hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream) {
    if (a.kd != 128 || a.vd != 128 || a.K < 1 || a.K > 8 || a.T < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gdn_kernel<128, 128>), dim3(a.nh, a.B), dim3(GDN_T), 0, stream, a);
    return hipGetLastError();
}

}  // namespace qwk
