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

// ===========================================================================
// Chunked form for long token runs.  The serial recurrence above costs one
// barrier chain per token; here the tokens of a sequence are cut into chunks
// of C = 64 and the delta rule is rewritten per chunk (the WY form of the
// delta rule, Yang et al. 2024, "Parallelizing Linear Transformers with the
// Delta Rule over Sequence Length", with the per-token decay of Gated
// DeltaNet).  For a chunk with start state S0, per-token decays gamma_i,
// G_i = sum_{m<=i} log gamma_m (so Gamma_i = exp(G_i)), the serial steps
//   S_i = gamma_i S_{i-1} + k_i u_i^T,  u_i = beta_i (v_i - gamma_i S_{i-1}^T k_i),
//   o_i = S_i^T q_i
// unroll to
//   (I + A) U = diag(beta) V - diag(beta Gamma) K S0,
//       A_ij = beta_i exp(G_i - G_j) k_i.k_j  (j < i, else 0)
//   U = Ut - W S0,  Ut = (I+A)^-1 diag(beta) V,  W = (I+A)^-1 diag(beta Gamma) K
//   O = diag(Gamma) Q S0 + Aq U,  Aq_ij = exp(G_i - G_j) q_i.k_j  (j <= i)
//   S_C = Gamma_C S0 + K^T diag(exp(G_C - G_i)) U.
// Every decay ratio is exp of a non-positive number, so nothing overflows.
// Three launches per segment of tokens:
//   gdn_chunk_prep   (chunk, head, sequence): conv + SiLU, L2 norms, gates,
//                    the two Gram matrices, the unit-triangular solve for Ut
//                    and W (one column of [W | Ut] per thread, in registers),
//                    and the decayed Q and K, written to a chunk record;
//   gdn_chunk_state  (16-column slice of the state, head, sequence): the only
//                    serial pass, S_{c+1} = Gamma_C S_c + Kd^T (Ut - W S_c);
//                    it records each chunk's start state S_c and U = Ut - W S_c,
//                    with the next chunk's W and Kd prefetched into registers
//                    while the current one is computed;
//   gdn_chunk_out    (chunk, head, sequence), in parallel over the chunks:
//                    O = Qd S_c + Aq U, then RMSNorm x norm_w x SiLU(z).
// The state update is column-separable (column j of S only needs column j of
// V), which is what lets the state pass split the state over 8 workgroups.
// Every product runs on FP32 MFMA (exact FP32 products, FP32 accumulation).
constexpr int GC_C = 64;     // tokens per chunk
constexpr int GC_D = 128;    // key_dim = value_dim
constexpr int GC_P = GC_D + 4;  // LDS row stride (floats) of the [C][D] tiles
constexpr int GC_VS = 16;    // state columns per state-pass workgroup
// chunk record (floats): W[C][D] | Ut[C][D] (U after the state pass) | Qd[C][D] | Kd[C][D] |
// Aq[C][C] | Gamma_C, padding | S_c[D][D] (start state, written by the state pass)
constexpr int GR_W = 0, GR_U = GC_C * GC_D, GR_Q = 2 * GC_C * GC_D, GR_K = 3 * GC_C * GC_D,
              GR_AQ = 4 * GC_C * GC_D, GR_G = GR_AQ + GC_C * GC_C, GR_S = GR_G + 64, GR_SIZE = GR_S + GC_D * GC_D;

// FP32 MFMA 16x16x4: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
// D[4*(l/16) + r][l%16] in element r.  The k index of a product only has to be
// the same permutation on both sides, so a 16-deep k block is fed as four
// steps q with k = 4*(l/16) + q: a float4 along k per lane and operand, and a
// D tile is directly the B operand of a following product.
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gdn_x(const GdnArgs& a, int b, int conv_dim, int d, int tau) {
    // conv input of channel d at token tau of sequence b; tau < 0 reads the conv state
    // (state[0] is token -1), tau >= T is padding
    if (tau >= a.T) return 0.0f;
    if (tau >= 0) return gdn_load(a.mixed, a.in_dt, ((int64_t)b * a.T + tau) * a.ld_in + d);
    return a.conv_state[((int64_t)b * conv_dim + d) * (a.K - 1) + (-tau - 1)];
}

__global__ __launch_bounds__(256) void gdn_chunk_prep(GdnArgs a, int t0, int nchunk, float* rec) {
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nh = a.nh, K = a.K;
    const int conv_dim = 3 * nh * GC_D;
    const int tc = t0 + c * GC_C;  // first token of the chunk

    __shared__ __attribute__((aligned(16))) float qkv_s[3 * GC_C * GC_P];  // q | k | v tiles [C][P]
    float* const qs = qkv_s;
    float* const ks = qkv_s + GC_C * GC_P;
    float* const vs = qkv_s + 2 * GC_C * GC_P;
    __shared__ __attribute__((aligned(16))) float As[GC_C * GC_C];
    __shared__ float hx[7 * 3 * GC_D];  // the K-1 inputs before the chunk: hx[j][channel] = x_{-1-j}
    __shared__ double Gs[GC_C];  // decay prefix sums in FP64: their differences stay exact to ~1e-16
    __shared__ float bs[GC_C];

    // ---- conv1d + SiLU.  Raw inputs of the chunk go to LDS first (coalesced
    // rows); then one thread per channel convolves in place from the last
    // token backwards, so the inputs it still needs are not yet overwritten;
    // the K-1 inputs before the chunk come from the rows or the conv state ----
    {
        // 4 consecutive channels per item, all 24 loads of a thread in flight
        // together (vector loads when the rows allow; element loads otherwise)
        const int esz = a.in_dt == DT_F32 ? 4 : 2;
        const bool vec = ((uintptr_t)a.mixed % (4 * esz)) == 0 && (a.ld_in % 4) == 0;
        f32x4 xv[GC_C * 3 * GC_D / 4 / 256];
        if (vec) {  // branch-free: rows past T are read clamped and zeroed
#pragma unroll
            for (int v = 0; v < GC_C * 3 * GC_D / 4 / 256; ++v) {
                const int e = t + 256 * v, i = e / (3 * GC_D / 4), cl = (e % (3 * GC_D / 4)) * 4;
                const int d = (cl / GC_D) * nh * GC_D + h * GC_D + cl % GC_D;
                const int tau = tc + i;
                const int64_t o = ((int64_t)b * a.T + min(tau, a.T - 1)) * a.ld_in + d;
                const f32x4 x = a.in_dt == DT_F32 ? *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.mixed) + o)
                                                  : load_act4(a.mixed, a.in_dt, o);
                xv[v] = tau < a.T ? x : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        } else {
#pragma unroll
            for (int v = 0; v < GC_C * 3 * GC_D / 4 / 256; ++v) {
                const int e = t + 256 * v, i = e / (3 * GC_D / 4), cl = (e % (3 * GC_D / 4)) * 4;
                const int d = (cl / GC_D) * nh * GC_D + h * GC_D + cl % GC_D;
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[v][q] = gdn_x(a, b, conv_dim, d + q, tc + i);
            }
        }
#pragma unroll
        for (int v = 0; v < GC_C * 3 * GC_D / 4 / 256; ++v) {
            const int e = t + 256 * v, i = e / (3 * GC_D / 4), cl = (e % (3 * GC_D / 4)) * 4;
            const int g3 = cl / GC_D, ch = cl % GC_D;
            *reinterpret_cast<f32x4*>(&qkv_s[g3 * GC_C * GC_P + i * GC_P + ch]) = xv[v];
        }
    }
    for (int e = t; e < (K - 1) * 3 * GC_D; e += 256) {
        const int j = e / (3 * GC_D), cl = e % (3 * GC_D), g3 = cl / GC_D, ch = cl % GC_D;
        hx[e] = gdn_x(a, b, conv_dim, g3 * nh * GC_D + h * GC_D + ch, tc - 1 - j);
        (void)j;
    }
    __syncthreads();
    {
        // thread = (channel, 32-token half): 384 x 2 = 3 x 256 work items; the
        // K-1 inputs before a block are read into registers before any output
        // is written (barrier), then each thread convolves its 32 tokens in place
        float hist[3][7], wv[3][8];
        int colo[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int item = t + 256 * u, cl = item % (3 * GC_D), i0 = (item / (3 * GC_D)) * (GC_C / 2);
            const int g3 = cl / GC_D, ch = cl % GC_D;
            const int d = g3 * nh * GC_D + h * GC_D + ch;
            colo[u] = g3 * GC_C * GC_P + i0 * GC_P + ch;  // offset of token i0 in qs|ks|vs
#pragma unroll
            for (int j = 0; j < 8; ++j) wv[u][j] = j < K ? a.conv_w[(int64_t)d * K + j] : 0.0f;
#pragma unroll
            for (int j = 0; j < 7; ++j) {
                const int src = i0 - 1 - j;
                hist[u][j] = j < K - 1 ? (src >= 0 ? qs[colo[u] - (1 + j) * GC_P] : hx[(-src - 1) * 3 * GC_D + cl]) : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int item = t + 256 * u, i0 = (item / (3 * GC_D)) * (GC_C / 2);
            const float wl = a.conv_w[(int64_t)((item % (3 * GC_D)) / GC_D * nh * GC_D + h * GC_D + item % GC_D) * K + K - 1];
#pragma unroll 8
            for (int i = 0; i < GC_C / 2; ++i) {
                const float x = qs[colo[u] + i * GC_P];
                float sum = wl * x;
#pragma unroll
                for (int j = 0; j < 7; ++j)
                    if (j < K - 1) sum += wv[u][j] * hist[u][j];
#pragma unroll
                for (int j = 6; j > 0; --j) hist[u][j] = hist[u][j - 1];
                hist[u][0] = x;
                qs[colo[u] + i * GC_P] = tc + i0 + i < a.T ? silu_f(sum) : 0.0f;
            }
        }
    }
    // ---- gates and the decay prefix sum (wave 0, one token per lane) ----
    if (wave == 0) {
        const int tau = tc + lane;
        double g = 0.0;
        float beta = 0.0f;
        if (tau < a.T) {
            const int64_t row = ((int64_t)b * a.T + tau) * a.ld_in;
            const float av = gdn_load(a.a, a.in_dt, row + h) + a.dt_bias[h];
            const float bv = gdn_load(a.b, a.in_dt, row + h);
            const float sp = av > 20.0f ? av : logf(1.0f + __expf(av));
            beta = 1.0f / (1.0f + __expf(-bv));
            g = (double)(-__expf(a.A_log[h]) * sp);
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(g, off);
            if (lane >= off) g += o;
        }
        Gs[lane] = g;
        bs[lane] = beta;
    }
    __syncthreads();
    // ---- per-token L2 norms of q (times 1/sqrt(D)) and k: a lane pair per
    // (token, vector), each lane summing 64 squares ----
    {
        const int item = t >> 1, half = t & 1;          // 128 items: token item/2, q or k
        float* v = (item & 1 ? ks : qs) + (item >> 1) * GC_P + half * 64;
        float ss = 0.0f;
#pragma unroll
        for (int d = 0; d < 64; d += 4) {
            const float4 x = *reinterpret_cast<const float4*>(&v[d]);
            ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        }
        ss += __shfl_xor(ss, 1);
        const float sc = 1.0f / sqrtf(ss + 1e-6f) * (item & 1 ? 1.0f : 1.0f / sqrtf((float)GC_D));
        __syncthreads();  // every lane has read its row
#pragma unroll
        for (int d = 0; d < 64; d += 4) {
            float4 x = *reinterpret_cast<const float4*>(&v[d]);
            x.x *= sc; x.y *= sc; x.z *= sc; x.w *= sc;
            *reinterpret_cast<float4*>(&v[d]) = x;
        }
    }
    __syncthreads();
    // ---- Gram tiles on MFMA: the 10 lower 16x16 tiles (ti >= tj) of K K^T and
    // Q K^T; A = beta_i exp(G_i - G_j) k_i.k_j (j < i) into LDS transposed
    // (As[j][i]); Aq = exp(G_i - G_j) q_i.k_j (j <= i) to the record ----
    float* R = rec + ((int64_t)(b * nh + h) * nchunk + c) * GR_SIZE;
    const int li = lane & 15, lg = lane >> 4;
    for (int job = wave; job < 10; job += 4) {
        const int ti = job < 1 ? 0 : job < 3 ? 1 : job < 6 ? 2 : 3;
        const int tj = job - ti * (ti + 1) / 2;
        f32x4 kk = {0.0f, 0.0f, 0.0f, 0.0f}, qk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
        for (int kb = 0; kb < GC_D; kb += 16) {
            const f32x4 ka = *reinterpret_cast<const f32x4*>(&ks[(16 * ti + li) * GC_P + kb + 4 * lg]);
            const f32x4 qa = *reinterpret_cast<const f32x4*>(&qs[(16 * ti + li) * GC_P + kb + 4 * lg]);
            const f32x4 kb4 = *reinterpret_cast<const f32x4*>(&ks[(16 * tj + li) * GC_P + kb + 4 * lg]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                kk = mfma16(ka[q], kb4[q], kk);
                qk = mfma16(qa[q], kb4[q], qk);
            }
        }
        const int j = 16 * tj + li;
        f32x4 av;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * ti + 4 * lg + r;
            const float dec = j <= i ? __expf((float)(Gs[i] - Gs[j])) : 0.0f;
            av[r] = j < i ? bs[i] * dec * kk[r] : 0.0f;
            R[GR_AQ + i * GC_C + j] = j <= i ? dec * qk[r] : 0.0f;
        }
        *reinterpret_cast<f32x4*>(&As[j * GC_C + 16 * ti + 4 * lg]) = av;
    }
    // upper tiles of Aq are zero
    for (int e = t; e < 6 * 256; e += 256) {
        const int tile = e >> 8, w = e & 255;
        const int ti = tile < 3 ? 0 : tile < 5 ? 1 : 2;
        const int tj = ti + 1 + (tile - (ti == 0 ? 0 : ti == 1 ? 3 : 5));
        R[GR_AQ + (16 * ti + (w >> 4)) * GC_C + 16 * tj + (w & 15)] = 0.0f;
    }
    __syncthreads();
    // ---- (I + A) X = [diag(beta Gamma) K | diag(beta) V] by 16-row blocks:
    // the four diagonal blocks are inverted by substitution (wave 0, one lane
    // per column of a block), then each wave runs the block substitution
    //   X_b = T_bb (R_b - sum_{c<b} A_bc X_c)
    // on MFMA for its 64 of the 256 right-hand-side columns, X in registers ----
    __shared__ __attribute__((aligned(16))) float Tl[4 * 256];  // T_bb[m][j]
    if (wave == 0) {
        const int bb = lg, jc = li;
        float x[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            float v = m == jc ? 1.0f : 0.0f;
#pragma unroll
            for (int n = 0; n < m; ++n) v -= As[(16 * bb + n) * GC_C + 16 * bb + m] * x[n];
            x[m] = v;
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) Tl[bb * 256 + m * 16 + jc] = x[m];
    }
    __syncthreads();
    {
        const bool isw = wave < 2;
        const float* src = isw ? ks : vs;
        const int cbase = (wave & 1) * 64;  // column base within K (waves 0, 1) or V (waves 2, 3)
        f32x4 X[4][4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * rb + 4 * lg + r;
                const float sc = bs[i] * (isw ? __expf((float)Gs[i]) : 1.0f);
#pragma unroll
                for (int ct = 0; ct < 4; ++ct) X[rb][ct][r] = sc * src[i * GC_P + cbase + 16 * ct + li];
            }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int cb = 0; cb < rb; ++cb) {
                float na[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) na[q] = -As[(16 * cb + 4 * lg + q) * GC_C + 16 * rb + li];
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
#pragma unroll
                    for (int q = 0; q < 4; ++q) X[rb][ct] = mfma16(na[q], X[cb][ct][q], X[rb][ct]);
            }
            const f32x4 ta = *reinterpret_cast<const f32x4*>(&Tl[rb * 256 + li * 16 + 4 * lg]);
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                f32x4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int q = 0; q < 4; ++q) y = mfma16(ta[q], X[rb][ct][q], y);
                X[rb][ct] = y;
            }
        }
        float* dstp = R + (isw ? GR_W : GR_U) + cbase;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
#pragma unroll
                for (int r = 0; r < 4; ++r) dstp[(16 * rb + 4 * lg + r) * GC_D + 16 * ct + li] = X[rb][ct][r];
    }
    // ---- decayed q and k for the scan ----
    const double GC = Gs[GC_C - 1];
    for (int e = t; e < GC_C * GC_D / 4; e += 256) {
        const int i = e / (GC_D / 4), d = (e % (GC_D / 4)) * 4;
        const float gq = __expf((float)Gs[i]), gk = __expf((float)(GC - Gs[i]));
        float4 qv = *reinterpret_cast<const float4*>(&qs[i * GC_P + d]);
        float4 kv = *reinterpret_cast<const float4*>(&ks[i * GC_P + d]);
        qv.x *= gq; qv.y *= gq; qv.z *= gq; qv.w *= gq;
        kv.x *= gk; kv.y *= gk; kv.z *= gk; kv.w *= gk;
        *reinterpret_cast<float4*>(&R[GR_Q + i * GC_D + d]) = qv;
        *reinterpret_cast<float4*>(&R[GR_K + i * GC_D + d]) = kv;
    }
    if (t == 0) R[GR_G] = __expf((float)GC);
}

// The serial pass over the chunks of one segment for a 16-column slice of
// one head's state, on MFMA.  Per chunk: record S_c, U = Ut - W S_c (wave w:
// rows 16w..16w+15, written over Ut), S_{c+1} = Gamma_C S_c + Kd^T U (wave w:
// state rows 32w..32w+31).  The state slice lives in LDS transposed
// (St[j][d]); the next chunk's W, Kd, Ut tile and Gamma_C are prefetched into
// registers while the current one is computed.  On the last segment the
// workgroup also moves the conv state of 48 of the head's 384 channels (the
// prep kernel of this segment has finished reading it).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gdn_chunk_state(GdnArgs a, int nchunk, float* rec, int last_segment) {
    const int sl = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, li = lane & 15, lg = lane >> 4;
    const int nh = a.nh;
    const int c0 = sl * GC_VS;  // first state column of the slice
    constexpr int NV = GC_C * GC_D / 4 / 256;  // float4 of W (and of Kd) per thread: 8
    constexpr int UP = GC_C + 4;               // row stride of the transposed U tile

    __shared__ __attribute__((aligned(16))) float Wl[GC_C * GC_P], Kl[GC_C * GC_P];
    __shared__ __attribute__((aligned(16))) float St[GC_VS * GC_P], Ut[GC_VS * UP];

    float* Sg = a.rec_state + ((int64_t)b * nh + h) * GC_D * GC_D;
    for (int e = t; e < GC_D * GC_VS; e += 256) {
        const int d = e / GC_VS, j = e % GC_VS;
        St[j * GC_P + d] = Sg[d * GC_D + c0 + j];
    }

    float* R0 = rec + (int64_t)(b * nh + h) * nchunk * GR_SIZE;
    f32x4 wn[NV], kn[NV], un;
    float gCn;
    auto prefetch = [&](const float* Rc) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int e = (t + 256 * v) * 4;
            wn[v] = *reinterpret_cast<const f32x4*>(&Rc[GR_W + e]);
            kn[v] = *reinterpret_cast<const f32x4*>(&Rc[GR_K + e]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) un[r] = Rc[GR_U + (16 * wave + 4 * lg + r) * GC_D + c0 + li];
        gCn = Rc[GR_G];
    };
    prefetch(R0);
    for (int c = 0; c < nchunk; ++c) {
        float* R = R0 + (int64_t)c * GR_SIZE;
        __syncthreads();  // the previous chunk is done with Wl, Kl, Ut; St holds S_c
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int e = (t + 256 * v) * 4, i = e / GC_D, d = e % GC_D;
            *reinterpret_cast<f32x4*>(&Wl[i * GC_P + d]) = wn[v];
            *reinterpret_cast<f32x4*>(&Kl[i * GC_P + d]) = kn[v];
        }
        f32x4 u = un;
        const float gC = gCn;
        if (c + 1 < nchunk) prefetch(R + GR_SIZE);  // consumed after this chunk's compute
        // record the start state of this chunk
        for (int e = t; e < GC_D * GC_VS; e += 256) {
            const int d = e / GC_VS, j = e % GC_VS;
            R[GR_S + d * GC_D + c0 + j] = St[j * GC_P + d];
        }
        __syncthreads();
        // U = Ut - W S_c   (wave w: rows 16w .. 16w+15)
#pragma unroll 4
        for (int kb = 0; kb < GC_D; kb += 16) {
            const f32x4 wa = *reinterpret_cast<const f32x4*>(&Wl[(16 * wave + li) * GC_P + kb + 4 * lg]);
            const f32x4 sb = *reinterpret_cast<const f32x4*>(&St[li * GC_P + kb + 4 * lg]);
#pragma unroll
            for (int q = 0; q < 4; ++q) u = mfma16(-wa[q], sb[q], u);
        }
        *reinterpret_cast<f32x4*>(&Ut[li * UP + 16 * wave + 4 * lg]) = u;
#pragma unroll
        for (int r = 0; r < 4; ++r) R[GR_U + (16 * wave + 4 * lg + r) * GC_D + c0 + li] = u[r];
        __syncthreads();
        // S_{c+1} = Gamma_C S_c + Kd^T U   (wave w: state rows 32w .. 32w+31)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const int d0 = 32 * wave + 16 * dt;
            f32x4 acc = *reinterpret_cast<const f32x4*>(&St[li * GC_P + d0 + 4 * lg]);
            acc = acc * gC;
#pragma unroll
            for (int ib = 0; ib < GC_C; ib += 16) {
                const f32x4 ub = *reinterpret_cast<const f32x4*>(&Ut[li * UP + ib + 4 * lg]);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc = mfma16(Kl[(ib + 4 * lg + q) * GC_P + d0 + li], ub[q], acc);
            }
            *reinterpret_cast<f32x4*>(&St[li * GC_P + d0 + 4 * lg]) = acc;
        }
    }
    __syncthreads();
    for (int e = t; e < GC_D * GC_VS; e += 256) {
        const int d = e / GC_VS, j = e % GC_VS;
        Sg[d * GC_D + c0 + j] = St[j * GC_P + d];
    }

    constexpr int CPS = 3 * GC_D / (GC_D / GC_VS);  // conv channels per slice: 48
    if (last_segment && a.K > 1 && t < CPS) {
        const int conv_dim = 3 * nh * GC_D;
        const int cl = sl * CPS + t;  // 0 .. 383 within the head
        const int d = (cl / GC_D) * nh * GC_D + h * GC_D + cl % GC_D;
        float nv[7];
#pragma unroll
        for (int j = 0; j < 7; ++j) nv[j] = j < a.K - 1 ? gdn_x(a, b, conv_dim, d, a.T - 1 - j) : 0.0f;
#pragma unroll
        for (int j = 0; j < 7; ++j)
            if (j < a.K - 1) a.conv_state[((int64_t)b * conv_dim + d) * (a.K - 1) + j] = nv[j];
    }
}

// Outputs of one chunk of one head on MFMA: O = Qd S_c + Aq U (wave w: output
// columns 32w .. 32w+31, all 64 rows), then per token RMSNorm x norm_w x
// SiLU(z), the row sums combined across the waves in LDS.
__global__ __launch_bounds__(256) void gdn_chunk_out(GdnArgs a, int t0, int nchunk, const float* rec) {
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, li = lane & 15, lg = lane >> 4;
    const int nh = a.nh;
    constexpr int AP = GC_C + 4;  // row stride of Aq and of the transposed U
    __shared__ __attribute__((aligned(16))) float Ql[GC_C * GC_P], STl[GC_D * GC_P], Al[GC_C * AP], UTl[GC_D * AP];
    __shared__ float red[4][GC_C];
    const float* R = rec + ((int64_t)(b * nh + h) * nchunk + c) * GR_SIZE;
    for (int e = t; e < GC_C * GC_D / 4; e += 256) {
        const int i = e / (GC_D / 4), d = (e % (GC_D / 4)) * 4;
        *reinterpret_cast<f32x4*>(&Ql[i * GC_P + d]) = *reinterpret_cast<const f32x4*>(&R[GR_Q + i * GC_D + d]);
        const f32x4 uv = *reinterpret_cast<const f32x4*>(&R[GR_U + i * GC_D + d]);
#pragma unroll
        for (int q = 0; q < 4; ++q) UTl[(d + q) * AP + i] = uv[q];
    }
    for (int e = t; e < GC_C * GC_C / 4; e += 256) {
        const int i = e / (GC_C / 4), j = (e % (GC_C / 4)) * 4;
        *reinterpret_cast<f32x4*>(&Al[i * AP + j]) = *reinterpret_cast<const f32x4*>(&R[GR_AQ + i * GC_C + j]);
    }
    for (int e = t; e < GC_D * GC_D / 4; e += 256) {
        const int k = e / (GC_D / 4), j = (e % (GC_D / 4)) * 4;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(&R[GR_S + k * GC_D + j]);
#pragma unroll
        for (int q = 0; q < 4; ++q) STl[(j + q) * GC_P + k] = sv[q];
    }
    __syncthreads();
    f32x4 o[4][2];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) o[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int cb = 32 * wave;
#pragma unroll 2
    for (int kb = 0; kb < GC_D; kb += 16) {
        f32x4 qa[4], sb[2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) qa[rt] = *reinterpret_cast<const f32x4*>(&Ql[(16 * rt + li) * GC_P + kb + 4 * lg]);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) sb[ct] = *reinterpret_cast<const f32x4*>(&STl[(cb + 16 * ct + li) * GC_P + kb + 4 * lg]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) o[rt][ct] = mfma16(qa[rt][q], sb[ct][q], o[rt][ct]);
    }
#pragma unroll
    for (int kb = 0; kb < GC_C; kb += 16) {
        f32x4 qa[4], sb[2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) qa[rt] = *reinterpret_cast<const f32x4*>(&Al[(16 * rt + li) * AP + kb + 4 * lg]);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) sb[ct] = *reinterpret_cast<const f32x4*>(&UTl[(cb + 16 * ct + li) * AP + kb + 4 * lg]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) o[rt][ct] = mfma16(qa[rt][q], sb[ct][q], o[rt][ct]);
    }
    // ---- RMSNorm x norm_w x SiLU(z) per token row: partial sums per wave ----
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float ss = o[rt][0][r] * o[rt][0][r] + o[rt][1][r] * o[rt][1][r];
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            if (li == 0) red[wave][16 * rt + 4 * lg + r] = ss;
        }
    __syncthreads();
    const float nw0 = a.norm_w[cb + li], nw1 = a.norm_w[cb + 16 + li];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * rt + 4 * lg + r;
            const int tau = t0 + c * GC_C + i;
            if (tau >= a.T) continue;
            const float tot = red[0][i] + red[1][i] + red[2][i] + red[3][i];
            const float inv = 1.0f / sqrtf(tot / (float)GC_D + 1e-6f);
            const int64_t row = (int64_t)b * a.T + tau;
            const int64_t zi = row * a.ld_in + h * GC_D + cb + li;
            const int64_t oi = row * a.ld_out + h * GC_D + cb + li;
            const float y0 = o[rt][0][r] * inv * nw0 * silu_f(gdn_load(a.z, a.in_dt, zi));
            const float y1 = o[rt][1][r] * inv * nw1 * silu_f(gdn_load(a.z, a.in_dt, zi + 16));
            if (a.out_dt == DT_F32) {
                reinterpret_cast<float*>(a.out)[oi] = y0;
                reinterpret_cast<float*>(a.out)[oi + 16] = y1;
            } else {
                store_act(a.out, a.out_dt, oi, y0);
                store_act(a.out, a.out_dt, oi + 16, y1);
            }
        }
}

size_t gdn_chunked_bytes_per_token(int nh) { return (size_t)nh * GR_SIZE * 4 / GC_C; }

hipError_t launch_gdn_chunked(const GdnArgs& a, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (a.kd != GC_D || a.vd != GC_D || a.K < 1 || a.K > 8 || a.T < 1) return hipErrorInvalidValue;
    // tokens per segment: whole chunks whose records fit the workspace
    const size_t per_tok = (size_t)a.B * gdn_chunked_bytes_per_token(a.nh);
    int64_t seg = (int64_t)(ws_bytes / per_tok) / GC_C * GC_C;
    if (seg < GC_C) return hipErrorInvalidValue;
    seg = std::min<int64_t>(seg, ((int64_t)a.T + GC_C - 1) / GC_C * GC_C);
    float* rec = reinterpret_cast<float*>(ws);
    for (int t0 = 0; t0 < a.T; t0 += (int)seg) {
        const int len = (int)std::min<int64_t>(seg, a.T - t0);
        const int nchunk = (len + GC_C - 1) / GC_C;
        const bool last = t0 + len >= a.T;
        hipLaunchKernelGGL(gdn_chunk_prep, dim3(nchunk, a.nh, a.B), dim3(256), 0, stream, a, t0, nchunk, rec);
        hipLaunchKernelGGL(gdn_chunk_state, dim3(GC_D / GC_VS, a.nh, a.B), dim3(256), 0, stream, a, nchunk, rec,
                           last ? 1 : 0);
        hipLaunchKernelGGL(gdn_chunk_out, dim3(nchunk, a.nh, a.B), dim3(256), 0, stream, a, t0, nchunk,
                           (const float*)rec);
    }
    return hipGetLastError();
}

}  // namespace qwk
