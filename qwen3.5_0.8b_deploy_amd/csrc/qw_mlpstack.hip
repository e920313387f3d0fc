// qw_mlpstack.hip -- L consecutive decoder MLP blocks in one persistent launch
// (decode, M <= 2 tokens, Qwen3.5-0.8B shape H = 1024, I = 3584):
//     for l < L:  x = x + down_l( silu(gate_l . n_l(x)) * (up_l . n_l(x)) ),
//                 n_l(x) = RMSNorm(x) * (1 + gamma_l),  x rounded to its dtype
// -- the same result as L calls of qw_mlp_fused(y = residual = x).
//
// Why.  One MLP block streams 22 MB of BF16 weights, about 3.5 us at the
// HBM rate, but a launch per block pays its start/end (~3 us) and its two
// data hand-offs serially, and no weight of block l+1 moves while block l
// waits for its hand-offs.  Here the weights of every block are requested
// as soon as the registers that hold them are free, a full block ahead of
// their use, so HBM streams continuously while the hand-offs run.
//
// Work split (grid = 256 workgroups of 16 waves, one per CU, all resident):
//   * gate/up role, waves 0..7 of workgroup p < I/16: the gate/up tile pair p
//     (intermediate rows [16p, 16p+16)), the K = H reduction cut in eight
//     128-wide slices, one per wave;
//   * down role, waves 8..15 of every workgroup w: down tile w/4 (output rows
//     [16(w/4), +16)) over the K quarter w%4 (896 intermediate rows), cut in
//     eight by wave.
// The two roles never wait for each other inside a workgroup (no workgroup
// barrier): each role's eight waves reduce their partial tiles through LDS,
// and the last of the eight to arrive (an LDS counter) runs the epilogue.
//
// Hand-offs carry their own validity: every word written for another
// workgroup is a 64-bit agent-scope store of (tag << 32 | payload), tag =
// epoch * 64 + layer + 1, and a consumer polls the words it needs until
// every tag is the expected one -- no counters, no fences, no memset (a
// 64-bit store is seen whole or not at all).  `epoch` is a device word read
// by every wave at the start and advanced by workgroup 0 at the very end, so
// words of earlier launches never match.  Payloads:
//   * h (gate/up -> down): two 16-bit h values (the down MFMA input type),
//     h_buf[layer & 1][m][I/2];
//   * down partials (down -> gate/up of the next block, and the final x):
//     one FP32 value, p_buf[layer & 1][quarter][m][H].  The consumer forms
//     x_{l+1} = round(x_l + ((P0 + P1) + P2) + P3) itself, in a fixed order,
//     so every workgroup holds bit-identical copies.
// Buffers alternate by layer parity: a slot of layer l+2 is written only
// after every reader of layer l has passed (each layer's hand-offs depend on
// all of the previous one's).
//
// Polls read one word per lane (a few hundred bytes per wave) until those are
// valid, then the full set once, so waiting costs little memory traffic.
// Every wait is bounded (0.2 s of the 100 MHz real-time counter): on expiry
// it raises the error flag (qw_device_error) and the launch's abort word, and
// every wave stops waiting, so the grid always drains.  Workgroups must all be resident: the launcher takes one
// workgroup per CU and refuses devices with fewer than 256 CUs.
//
// Reference: the post-norm + MLP + residual chain of CudaLayer::forward
// (cuda_engine.cu:119-124) over consecutive layers, i.e. CudaMLP::forward_add_
// residual (mlp_cuda.cu:295-337, the residual added) with RMSNorm
// (language_common.cpp:21-36) per block.
#include "qw_stream.hpp"

namespace qwk {

constexpr int MS_NW = 16;          // waves per workgroup: 8 gate/up + 8 down
constexpr int MS_RW = 8;           // waves per role
constexpr int MS_MAXM = 4;         // tokens
constexpr int MS_H = 1024, MS_I = 3584;
constexpr int MS_Q = 4;            // K quarters of a down tile
constexpr int MS_GRID = (MS_H / 16) * MS_Q;  // 256 down pieces = 256 workgroups
constexpr int MS_SPAN = 128;       // K values per wave slice (both roles, both formats)
constexpr int MS_LROW = MS_SPAN + 8;  // LDS row of a wave's B slice (16-byte pad)

size_t mlp_stack_ws_bytes() { return (size_t)2 * MS_MAXM * (MS_I / 2) * 8 + (size_t)2 * MS_Q * MS_MAXM * MS_H * 8; }
int mlp_stack_max_m() { return 2; }  // register budget: two tokens per lane slice
int mlp_stack_grid() { return MS_GRID; }

struct MsLds {
    uint16_t bs[MS_NW][MS_MAXM][MS_LROW];  // per-wave B slices (MFMA input type bits; 16-byte rows)
    f32x4 red_gu[MS_RW][2][64];  // gate/up role partial tiles
    f32x4 red_dn[MS_RW][64];     // down role partial tiles
    float red_ss[MS_RW][MS_MAXM];
    unsigned cnt_gu, cnt_dn;
};

__device__ __forceinline__ uint32_t ms_tag(uint32_t epoch, int layer) { return (epoch << 6) | (uint32_t)(layer + 1); }

__device__ __forceinline__ uint64_t ms_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ms_store(uint64_t* p, uint32_t tag, uint32_t payload) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// What a wait needs to give up: the device error flag, this launch's abort
// word (set to epoch + 1 by the first wave whose wait expires, so the others
// stop at once; later launches compare with their own epoch) and the epoch.
struct MsAbort {
    unsigned* err;
    unsigned* abort;
    uint32_t epoch;
};

// Pause between polls; false once the wait that started at t0 has run 0.2 s
// of the 100 MHz real-time counter (then the error flag and the abort word
// are raised) or as soon as another wave of this launch has aborted.
__device__ __forceinline__ bool ms_pause(const MsAbort& ab, uint64_t t0, bool& dead) {
    const unsigned v = __hip_atomic_load(ab.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool expired = __builtin_amdgcn_s_memrealtime() - t0 > 20000000ull;
    if (v == ab.epoch + 1u || expired) {
        if (expired) {
            __hip_atomic_store(ab.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ab.abort, ab.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        dead = true;
        return false;
    }
    __builtin_amdgcn_s_sleep(2);
    return true;
}

// Bounded wait until every lane's probe word carries `tag` (probe = nullptr:
// nothing to wait for in that lane).
__device__ __forceinline__ void ms_wait(const uint64_t* probe, uint32_t tag, const MsAbort& ab, uint64_t t0,
                                        bool& dead) {
    while (!dead) {
        const bool ok = probe == nullptr || (uint32_t)(ms_load(probe) >> 32) == tag;
        if (__all(ok)) return;
        if (!ms_pause(ab, t0, dead)) return;
    }
}

// x rounded to the activation dtype
template <int XDT>
__device__ __forceinline__ float round_act(float v) {
    if constexpr (XDT == DT_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    else return f16_bits_to_f32(f32_to_f16_bits(v));
}

__device__ __forceinline__ void lds_fence_wave() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// B operand of k-step u of a wave's slice: lane (j, g) reads token j's
// elements [u*4*KE + g*KE, +KE) of the slice (zeros for j >= M).
template <int WF>
__device__ __forceinline__ BOps<WF, (WF == WF_BF16 ? DT_BF16 : DT_F16)> ms_bops(const uint16_t (*bs)[MS_LROW], int u,
                                                                                 int lane, int M) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int XDT = WF == WF_BF16 ? DT_BF16 : DT_F16;
    const int j = lane & 15, g = lane >> 4;
    BOps<WF, XDT> b;
    const uint16_t* p = &bs[j < M ? j : 0][u * 4 * KE + g * KE];
    if constexpr (WF == WF_BF16) {
        u32x4 v = *reinterpret_cast<const u32x4*>(p);
        if (j >= M) v = u32x4{0u, 0u, 0u, 0u};
        b.hi = __builtin_bit_cast(bf16x8, v);
    } else {
        u32x4 v0 = reinterpret_cast<const u32x4*>(p)[0], v1 = reinterpret_cast<const u32x4*>(p)[1];
        if (j >= M) v0 = v1 = u32x4{0u, 0u, 0u, 0u};
        b.hi0 = __builtin_bit_cast(f16x8, v0);
        b.hi1 = __builtin_bit_cast(f16x8, v1);
    }
    return b;
}

// WF: weight format (BF16 or INT8); XDT: activation / output dtype (BF16, or
// F16 for INT8 weights); GAM: per-layer gamma pointers given (else the norm
// weight is folded into the gate/up weights); MT: tokens the registers are
// sized for (M <= MT).
template <int WF, int XDT, bool GAM, int MT>
__global__ __launch_bounds__(MS_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void mlp_stack_kernel(MlpStackArgs a) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int OPDT = WF == WF_BF16 ? DT_BF16 : DT_F16;  // MFMA input type of x and h
    constexpr int KS_GU = MS_H / (4 * KE);                 // k-steps of a gate/up tile (32 / 16)
    constexpr int KS_DN = MS_I / (4 * KE);                 // k-steps of a down tile (112 / 56)
    constexpr int U_GU = KS_GU / MS_RW;                    // per gate/up wave (4 / 2)
    constexpr int U_DN = (KS_DN / MS_Q + MS_RW - 1) / MS_RW;  // per down wave, at most (4 / 2)
    extern __shared__ __attribute__((aligned(16))) uint8_t ms_raw[];
    MsLds& S = *reinterpret_cast<MsLds*>(ms_raw);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int wg = blockIdx.x;
    const int M = a.M;
    // every wave holds the epoch before the barrier, so workgroup 0 can only
    // advance it (at the very end, after all hand-offs) once all have read it
    const uint32_t epoch = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0) {
        S.cnt_gu = 0u;
        S.cnt_dn = 0u;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();  // the only workgroup barrier: counters set before either role uses them
    bool dead = false;
    const MsAbort ab{a.err, a.epoch + 1, epoch};
    uint64_t* const hbuf = a.hbuf;
    uint64_t* const pbuf = a.pbuf;

    if (wave < MS_RW) {
        // ===================== gate/up role =====================
        const int p = wg;
        if (p >= MS_I / 16) return;
        const int w = wave;
        const int k0 = w * MS_SPAN;            // this wave's K slice [k0, k0 + 128)
        const uint32_t tile_bytes = (uint32_t)KS_GU * 1024u;
        // this lane's slice elements: e = lane + 64 i (i < 2M): token e >> 7, k0 + (e & 127)
        float xv[2 * MT];
        u32x4 A[U_GU][2];
        float gm[2] = {0.f, 0.f};
        u32x4 sc[2];
        auto issue = [&](int l) {
            const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.gu[l], (uint32_t)(MS_I / 16) * 2u * tile_bytes);
#pragma unroll
            for (int u = 0; u < U_GU; ++u)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    A[u][rt] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   wr, lane * 16, (uint32_t)(p * 2 + rt) * tile_bytes + (uint32_t)(w * U_GU + u) * 1024u,
                                   AUX_NT));
            if constexpr (GAM) {
                gm[0] = a.gamma[l][k0 + lane];
                gm[1] = a.gamma[l][k0 + 64 + lane];
            }
            if constexpr (WF == WF_I8) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    sc[rt] = *reinterpret_cast<const u32x4*>(a.gu_scales[l] + (p * 2 + rt) * 16 + g * 4);
            }
        };
        // the layer input: x as given
#pragma unroll
        for (int i = 0; i < 2 * MT; ++i)
            xv[i] = (i >> 1) < M ? load_act(a.x, XDT, (int64_t)(i >> 1) * MS_H + k0 + (lane + 64 * (i & 1))) : 0.0f;
        issue(0);
        for (int l = 0; l <= a.L; ++l) {
            if (l > 0) {
                // x_l = round(x_{l-1} + ((P0 + P1) + P2) + P3) from the partials of block l-1
                const uint32_t tg = ms_tag(epoch, l - 1);
                const uint64_t* P = pbuf + (size_t)((l - 1) & 1) * MS_Q * MS_MAXM * MS_H;
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                ms_wait(P + k0 + lane, tg, ab, t0, dead);  // quarter 0, token 0 of this lane's first element
                for (;;) {
                    // tokens two at a time: 16 words in flight per lane
                    bool ok = true;
                    float nx[2 * MT];
#pragma unroll
                    for (int m0 = 0; m0 < MT; m0 += 2) {
                        uint64_t v[2][2][MS_Q];
#pragma unroll
                        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                            for (int h = 0; h < 2; ++h)
#pragma unroll
                                for (int q = 0; q < MS_Q; ++q)
                                    v[mm][h][q] = (m0 + mm < MT && m0 + mm < M)
                                                      ? ms_load(P + ((size_t)q * MS_MAXM + m0 + mm) * MS_H + k0 + lane + 64 * h)
                                                      : ((uint64_t)tg << 32);
#pragma unroll
                        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                const int i = 2 * (m0 + mm) + h;
                                if (i >= 2 * MT) continue;
                                float sum = 0.0f;
#pragma unroll
                                for (int q = 0; q < MS_Q; ++q) {
                                    ok = ok && (uint32_t)(v[mm][h][q] >> 32) == tg;
                                    sum += __uint_as_float((uint32_t)v[mm][h][q]);
                                }
                                nx[i] = m0 + mm < M ? round_act<XDT>(xv[i] + sum) : xv[i];
                            }
                    }
                    if (__all(ok) || dead) {
#pragma unroll
                        for (int i = 0; i < 2 * MT; ++i) xv[i] = nx[i];
                        break;
                    }
                    if (!ms_pause(ab, t0, dead)) break;
                }
            }
            if (l == a.L) {
                // after the last block: workgroup 0 writes the result
                if (wg == 0) {
#pragma unroll
                    for (int i = 0; i < 2 * MT; ++i)
                        if ((i >> 1) < M)
                            store_act(a.y, XDT, (int64_t)(i >> 1) * MS_H + k0 + lane + 64 * (i & 1), xv[i]);
                    if (w == 0) {
                        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                        if (lane == 0)
                            __hip_atomic_store(a.epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                break;
            }
            // B slice: round(x * (1 + gamma)) in the MFMA type; sums of squares per token
            float ss[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float a0 = xv[2 * m], a1 = xv[2 * m + 1];
                ss[m] = a0 * a0 + a1 * a1;
                if (m < M) {
                    const float b0 = GAM ? a0 * (1.0f + gm[0]) : a0;
                    const float b1 = GAM ? a1 * (1.0f + gm[1]) : a1;
                    S.bs[wave][m][lane] = (uint16_t)op_bits<WF>(b0);
                    S.bs[wave][m][lane + 64] = (uint16_t)op_bits<WF>(b1);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) ss[m] += __shfl_xor(ss[m], off);
            lds_fence_wave();
            f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U_GU; ++u) {
                const auto b = ms_bops<WF>(S.bs[wave], u, lane, M);
                accg = unit_mfma<WF, OPDT>(A[u][0], b, accg);
                accu = unit_mfma<WF, OPDT>(A[u][1], b, accu);
            }
            u32x4 sc_cur[2] = {sc[0], sc[1]};
            if (l + 1 < a.L) issue(l + 1);  // the next block's weights stream during the hand-offs
            // reduce the eight slices: the last wave to arrive runs the epilogue
            S.red_gu[w][0][lane] = accg;
            S.red_gu[w][1][lane] = accu;
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == m) S.red_ss[w][m] = ss[m];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&S.cnt_gu, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __shfl(old, 0);
            if (old != MS_RW - 1) continue;
            if (lane == 0) __hip_atomic_store(&S.cnt_gu, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            f32x4 gs = S.red_gu[0][0][lane], us = S.red_gu[0][1][lane];
#pragma unroll
            for (int v = 1; v < MS_RW; ++v) {
                gs += S.red_gu[v][0][lane];
                us += S.red_gu[v][1][lane];
            }
            float sst = 0.0f;
            const int jj = j < M ? j : 0;
#pragma unroll
            for (int v = 0; v < MS_RW; ++v) sst += S.red_ss[v][jj];
            const float inv = 1.0f / sqrtf(sst / (float)MS_H + a.eps);
            if constexpr (WF == WF_I8) {
                gs *= as_f32x4(sc_cur[0]);
                us *= as_f32x4(sc_cur[1]);
            }
            uint32_t hb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) hb[i] = op_bits<WF>(silu_f(gs[i] * inv) * (us[i] * inv));
            if (j < M) {
                const uint32_t tg = ms_tag(epoch, l);
                uint64_t* hw = hbuf + ((size_t)(l & 1) * MS_MAXM + j) * (MS_I / 2) + (p * 16 + g * 4) / 2;
                ms_store(hw, tg, hb[0] | (hb[1] << 16));
                ms_store(hw + 1, tg, hb[2] | (hb[3] << 16));
            }
        }
    } else {
        // ===================== down role =====================
        const int d = wave - MS_RW;
        const int t = wg / MS_Q, q = wg % MS_Q;
        const int kq0 = q * (KS_DN / MS_Q);
        int kb, kend;
        wave_range<MS_RW>(kq0, kq0 + KS_DN / MS_Q, d, kb, kend);
        const int n = kend - kb;
        const int kspan = n * 4 * KE;             // K values of this wave (<= 128)
        const int hk0 = kb * 4 * KE;              // first intermediate row
        const uint32_t tile_bytes = (uint32_t)KS_DN * 1024u;
        u32x4 A[U_DN];
        u32x4 sc = u32x4{0u, 0u, 0u, 0u};
        auto issue = [&](int l) {
            const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.dn[l], (uint32_t)(MS_H / 16) * tile_bytes);
#pragma unroll
            for (int u = 0; u < U_DN; ++u)
                A[u] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               wr, u < n ? lane * 16 : OOB, (uint32_t)t * tile_bytes + (uint32_t)(kb + u) * 1024u, AUX_NT));
            if constexpr (WF == WF_I8) sc = *reinterpret_cast<const u32x4*>(a.dn_scales[l] + t * 16 + g * 4);
        };
        issue(0);
        for (int l = 0; l < a.L; ++l) {
            const uint32_t tg = ms_tag(epoch, l);
            const uint64_t* hl = hbuf + (size_t)(l & 1) * MS_MAXM * (MS_I / 2);
            // words of token m: hl[m][hk0/2 + lane], lane < kspan/2
            const bool mine = lane < kspan / 2;
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            ms_wait(mine ? hl + hk0 / 2 + lane : nullptr, tg, ab, t0, dead);
            for (;;) {
                bool ok = true;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m < M && mine) {
                        const uint64_t v = ms_load(hl + (size_t)m * (MS_I / 2) + hk0 / 2 + lane);
                        ok = ok && (uint32_t)(v >> 32) == tg;
                        S.bs[wave][m][2 * lane] = (uint16_t)(v & 0xffffu);
                        S.bs[wave][m][2 * lane + 1] = (uint16_t)((v >> 16) & 0xffffu);
                    }
                }
                if (__all(ok) || dead) break;
                if (!ms_pause(ab, t0, dead)) break;
            }
            lds_fence_wave();
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U_DN; ++u) {
                if (u < n) {
                    const auto b = ms_bops<WF>(S.bs[wave], u, lane, M);
                    acc = unit_mfma<WF, OPDT>(A[u], b, acc);
                }
            }
            const u32x4 sc_cur = sc;
            if (l + 1 < a.L) issue(l + 1);
            S.red_dn[d][lane] = acc;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&S.cnt_dn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __shfl(old, 0);
            if (old != MS_RW - 1) continue;
            if (lane == 0) __hip_atomic_store(&S.cnt_dn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            f32x4 s = S.red_dn[0][lane];
#pragma unroll
            for (int v = 1; v < MS_RW; ++v) s += S.red_dn[v][lane];
            if constexpr (WF == WF_I8) s *= as_f32x4(sc_cur);
            if (j < M) {
                uint64_t* pw = pbuf + (((size_t)(l & 1) * MS_Q + q) * MS_MAXM + j) * MS_H + t * 16 + g * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i) ms_store(pw + i, tg, __float_as_uint(s[i]));
            }
        }
    }
}

template <typename Kern>
static hipError_t launch_ms(Kern k, const MlpStackArgs& a, hipStream_t st) {
    constexpr size_t lds = 96 * 1024;  // more than half the CU's LDS: one workgroup per CU
    static_assert(sizeof(MsLds) <= lds, "LDS layout");
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(k, dim3(MS_GRID), dim3(MS_NW * 64), lds, st, a);
    return hipGetLastError();
}

template <int WF, int XDT, bool GAM>
static hipError_t launch_ms2(const MlpStackArgs& a, hipStream_t st) {
    if (a.M == 1) return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 1>, a, st);
    return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 2>, a, st);
}

template <int WF, int XDT>
static hipError_t launch_ms1(const MlpStackArgs& a, hipStream_t st) {
    if (a.gamma[0]) return launch_ms2<WF, XDT, true>(a, st);
    return launch_ms2<WF, XDT, false>(a, st);
}

hipError_t launch_mlp_stack(const MlpStackArgs& a, int wf, int xdt, hipStream_t stream) {
    if (a.L < 1 || a.L > kMlpStackMaxLayers || a.M < 1 || a.M > mlp_stack_max_m()) return hipErrorInvalidValue;
    MlpStackArgs b = a;
    b.pbuf = a.hbuf + (size_t)2 * MS_MAXM * (MS_I / 2);  // the partials follow the h words
    if (wf == WF_BF16 && xdt == DT_BF16) return launch_ms1<WF_BF16, DT_BF16>(b, stream);
    if (wf == WF_I8 && xdt == DT_F16) return launch_ms1<WF_I8, DT_F16>(b, stream);
    return hipErrorInvalidValue;
}

}  // namespace qwk
