// qw_gemv.hip -- decode GEMV for gfx950 with register-direct activations
// (M <= 32 tokens; BF16 weights with BF16 activations, INT8 weights with F16
// or BF16 activations).
//
// Why a second small-M kernel.  The skinny kernel (qw_skinny.hip) stages the
// activations of its K range into LDS before any MFMA can run: a global load
// round trip, an LDS write pass and a workgroup barrier on the critical path
// of every launch.  At decode the whole launch lasts a few microseconds, so
// that prologue is a large share of it.  Here each lane loads its own MFMA B
// operand straight from global memory (L2-resident: x is a few KB shared by
// every workgroup), in the same instruction stream as the weights.  The
// waves of a workgroup never wait for each other until their partial tiles
// meet in LDS, and nothing precedes the first weight load but address math.
//
// B operand of k-step ks for lane l = r + 16g: token r, elements
// [ks*4*KE + g*KE, +KE) -- exactly the A layout of the packed weight unit
// (qw_device.hpp), so one MFMA per 16 B of weights (two for INT8).  Lanes of
// tokens >= M issue their loads out of range (zeros, no memory traffic).
// With the RMSNorm prologue the lane multiplies its values by (1 + gamma)
// and accumulates their squares; the per-token sums of squares ride along
// with the partial tiles through the reduction and any split-K hand-off, and
// 1/rms scales the final tile (RMSNorm is linear in x once rms is known).
//
// Work decomposition, split-K hand-off, epilogue and fused argmax follow the
// skinny kernel: an item is a 16-row tile (a gate/up pair for GLU weights)
// over one K split; the NW waves of a workgroup take contiguous pieces of the
// split; the loads of the next item are issued before the current item's
// reduction.  The cross-wave reduction sums the NW partials with all threads
// of the workgroup (independent LDS reads, fixed order).
//
// Reference operators replaced: cutlass_style_gemv_kernel / _bf16 /
// _fused_silu (cutlass_gemm_wrapper.cuh:41-200), int8_gemv_batch_kernel
// (mlp_cuda.cu:158-180), lm_head_gemv_kernel_optimized (lm_head_cuda.cu:38-99)
// + block_argmax_kernel (gpu_sampler_argmax.cu:14-43), and the thread-per-row
// decode projections of the attention operators (linear_attention_cuda.cu:
// 33-45,174-187; full_attention_cuda.cu:31-76,78-148,161-172).
#include "qw_stream.hpp"

namespace qwk {

// consecutive 16-row tiles per argmax item: two for INT8 (a 16 KB tile is
// too little work per cross-wave reduction), one for BF16 (measured)
template <int WF> struct ArgmaxTiles { static constexpr int v = WF == WF_I8 ? 2 : 1; };

template <int WF, int XDT, int CT, bool GLU, bool ARGMAX, int NW, bool NORM, bool GAM>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemv_kernel(SkinnyArgs ain) {
    // Token groups (tg_grid > 0): the grid is tg_grid workgroups per group of
    // tg_size tokens, all groups of a launch streaming the same weights
    // concurrently (workgroup w: group w / tg_grid); each workgroup sees its
    // group as a small-M problem of its own.
    const int tgi = ain.tg_grid ? (int)(blockIdx.x / (unsigned)ain.tg_grid) : 0;
    const int bid = (int)blockIdx.x - tgi * ain.tg_grid;
    const int gdim = ain.tg_grid ? ain.tg_grid : (int)gridDim.x;
    const int gofs = tgi * ain.n_groups;  // this group's split-K counters / partials
    SkinnyArgs a = ain;
    if (ain.tg_grid) {
        const int tok0 = tgi * ain.tg_size;
        a.M = min(ain.tg_size, ain.M - tok0);
        a.x = static_cast<const uint8_t*>(ain.x) + (int64_t)tok0 * ain.ldx * 2;
        const int ys = ain.ydt == DT_F32 ? 4 : 2;
        if (ain.y) a.y = static_cast<uint8_t*>(ain.y) + (int64_t)tok0 * ain.ldy * ys;
        if (ain.y2) a.y2 = static_cast<uint8_t*>(ain.y2) + (int64_t)tok0 * ain.ldy * ys;
        if (ain.res) a.res = static_cast<const uint8_t*>(ain.res) + (int64_t)tok0 * ain.ld_res * (ain.res_dt == DT_F32 ? 4 : 2);
        a.keys = ain.keys + tok0;
    }
    // k-steps per register buffer (two buffers in flight); fewer where the
    // activation fragments and RMSNorm weights would crowd the registers
    constexpr int U = ((GAM && WF == WF_I8) || (CT == 2 && (GAM || WF == WF_I8))) ? 2 : 4;
    constexpr int KE = WTraits<WF>::KE;
    // tiles per item: a gate/up pair (GLU), or ArgmaxTiles consecutive tiles
    // for the argmax (fewer per-item reductions for the many-tile lm_head)
    constexpr int RT = GLU ? 2 : (ARGMAX ? ArgmaxTiles<WF>::v : 1);
    constexpr int F = RT * CT;
    __shared__ f32x4 red[NW][F][64];
    __shared__ float red_ss[NW][16 * CT];

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const bool want_res = !ARGMAX && (a.flags & EP_RESIDUAL);

    int s = 0, ks0 = 0, ks1 = a.ksteps;
    if (a.S > 1) {
        s = bid % a.S;
        ks0 = (s * a.ksteps) / a.S;
        ks1 = ((s + 1) * a.ksteps) / a.S;
    }
    const int grp_step = a.S > 1 ? gdim / a.S : gdim;
    int kb, kend;
    wave_range<NW>(ks0, ks1, wave_id, kb, kend);
    const int kb0 = kb;

    // weight tiles that exist (the last argmax pair may have only one)
    const int n_tiles = ARGMAX ? (a.N + 15) / 16 : a.n_groups * RT;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)n_tiles * a.ksteps * 1024u));
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2u));
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(GAM ? (const void*)a.gamma : a.x, GAM ? (uint32_t)a.K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)n_tiles * 64u : 0u);
    const int res_size = a.res_dt == DT_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(want_res ? a.res : a.x, want_res ? (uint32_t)((uint64_t)a.M * a.ld_res * res_size) : 0u);

    // this lane's activation rows: token ct*16 + r of each tile (out of range past M)
    uint32_t xrow[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
        xrow[ct] = ct * 16 + r < a.M ? (uint32_t)((ct * 16 + r) * a.ldx + g * KE) * 2u : OOB;
    const uint32_t grow = r < a.M ? (uint32_t)(g * KE) * 4u : OOB;

    unsigned long long best[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) best[ct] = 0ull;
    // two register buffers of U k-steps: the loads of chunk c+1 are in
    // flight while chunk c is multiplied
    u32x4 A0[U][RT], A1[U][RT];
    XFrag<WF, XDT, CT> X0[U], X1[U];
    EpiOps<RT, CT> epi, epi_next;
    int item = bid;
    int grp = a.S > 1 ? bid / a.S : bid;

    auto issue = [&](int grp_, int kb_, int n_, u32x4 (&Ad)[U][RT], XFrag<WF, XDT, CT> (&Xd)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t ko = (uint32_t)(kb_ + u) * 4u * KE;
            uint32_t xo[CT];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) xo[ct] = u < n_ ? xrow[ct] + ko * 2u : OOB;
            load_xfrag<WF, XDT, CT, GAM>(xr, gr, xo, u < n_ ? grow + ko * 4u : OOB, Xd[u]);
        }
        __builtin_amdgcn_sched_barrier(0);
        issue_weights<RT, U>(a, wrs, grp_, kb_, n_, lane, Ad);
    };
    // slots u >= n were loaded out of range: zero operands, so every slot
    // runs unconditionally (branch-free: each load is waited for on its own)
    auto compute = [&](const u32x4 (&As)[U][RT], const XFrag<WF, XDT, CT> (&Xs)[U], f32x4 (&acc)[RT][CT],
                       float (&ss)[CT]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const BOps<WF, XDT> b = make_bops<WF, XDT, CT, NORM, GAM>(Xs[u], ct, ss[ct]);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = unit_mfma<WF, XDT>(As[u][rt], b, acc[rt][ct]);
            }
    };

    // weights first: the epilogue operands (the residual may have just been
    // written by the previous kernel: a slower, coherent fetch) are needed
    // last, and loads retire in order
    issue(grp, kb, item < a.n_items ? min(U, kend - kb) : 0, A0, X0);
    load_epi<RT, CT>(a, sr, rr, grp, item < a.n_items, lane, epi);

    while (item < a.n_items) {
        f32x4 acc[RT][CT];
        float ss[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            ss[ct] = 0.0f;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        // buffer 0 holds the chunk at kb on entry
        for (;;) {
            if (kb + U < kend) issue(grp, kb + U, min(U, kend - kb - U), A1, X1);
            compute(A0, X0, acc, ss);
            kb += U;
            if (kb >= kend) break;
            if (kb + U < kend) issue(grp, kb + U, min(U, kend - kb - U), A0, X0);
            compute(A1, X1, acc, ss);
            kb += U;
            if (kb >= kend) break;
        }
        const int cur_grp = grp;
        item += gdim;
        grp += grp_step;
        kb = kb0;
        if (item < a.n_items) {  // next item's loads fly during this item's reduction
            issue(grp, kb, min(U, kend - kb), A0, X0);
            load_epi<RT, CT>(a, sr, rr, grp, true, lane, epi_next);
        }

        // ---- reduce the NW partial tiles (fixed order, all threads) ----
        if constexpr (NORM) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                ss[ct] += __shfl_xor(ss[ct], 16);
                ss[ct] += __shfl_xor(ss[ct], 32);
                if (g == 0) red_ss[wave_id][ct * 16 + r] = ss[ct];
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) red[wave_id][rt * CT + ct][lane] = acc[rt][ct];
        __syncthreads();
        {
            float* redf = reinterpret_cast<float*>(&red[0][0][0]);
            constexpr int PER_W = F * 64 * 4;
            for (int t = threadIdx.x; t < PER_W; t += NW * 64) {
                float part[NW];
#pragma unroll
                for (int w = 0; w < NW; ++w) part[w] = redf[w * PER_W + t];
                float sum = part[0];
#pragma unroll
                for (int w = 1; w < NW; ++w) sum += part[w];
                redf[t] = sum;
            }
            if constexpr (NORM) {
                if (threadIdx.x < 16 * CT) {
                    float t = red_ss[0][threadIdx.x];
#pragma unroll
                    for (int w = 1; w < NW; ++w) t += red_ss[w][threadIdx.x];
                    red_ss[0][threadIdx.x] = t;
                }
            }
        }
        __syncthreads();
        if (wave_id != 0) {
            __syncthreads();  // wave 0 has read the sums before the next item overwrites them
            continue;
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = red[0][rt * CT + ct][lane];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) ss[ct] = NORM ? red_ss[0][ct * 16 + r] : 0.0f;
        __syncthreads();
        EpiOps<RT, CT> e = epi;
        epi = epi_next;

        const int grp_c = cur_grp;
        bool finish = true;
        if constexpr (!ARGMAX) {
            if (a.S > 1) {
                // split-K hand-off without a fence: agent-scope stores of the
                // partial tile and sums of squares, wait for their completion,
                // then the agent-scope arrival count; the last arriver sums
                // the S partials in split order and re-arms the counter
                constexpr int REC = F * 4 + CT;
                float* P = reinterpret_cast<float*>(a.partials) + ((int64_t)(grp_c + gofs) * a.S * 64 + lane) * REC;
                float* mine = P + (int64_t)s * 64 * REC;
#pragma unroll
                for (int f = 0; f < F; ++f)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        __hip_atomic_store(mine + f * 4 + i, acc[f / CT][f % CT][i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
                    __hip_atomic_store(mine + F * 4 + ct, ss[ct], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                unsigned old = 0;
                if (lane == 0)
                    old = __hip_atomic_fetch_add(&a.counters[grp_c + gofs], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                old = __shfl(old, 0);
                finish = (old == (unsigned)(a.S - 1));
                if (finish) {
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        ss[ct] = 0.0f;
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                    for (int s2 = 0; s2 < a.S; ++s2) {
                        const float* q = P + (int64_t)s2 * 64 * REC;
#pragma unroll
                        for (int f = 0; f < F; ++f)
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                acc[f / CT][f % CT][i] +=
                                    __hip_atomic_load(q + f * 4 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct)
                            ss[ct] += __hip_atomic_load(q + F * 4 + ct, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    if (lane == 0) __hip_atomic_store(&a.counters[grp_c + gofs], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (!finish) continue;

        if constexpr (ARGMAX) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int m = ct * 16 + r;
                if (m >= a.M) continue;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int o = (grp_c * RT + rt) * 16 + g * 4;  // first of this lane's 4 rows
                    f32x4 v = acc[rt][ct];
                    if (a.scales) v *= as_f32x4(e.sc[rt]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (o + i < a.N) {
                            const unsigned long long kk = argmax_key(v[i], (uint32_t)(o + i));
                            best[ct] = kk > best[ct] ? kk : best[ct];
                        }
                    }
                }
            }
            continue;
        }
        const int o = grp_c * 16 + g * 4;  // first of this lane's 4 logical rows
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const float inv = NORM ? 1.0f / sqrtf(ss[ct] / (float)a.K + a.eps) : 1.0f;
            const int m = ct * 16 + r;
            f32x4 v;
            if constexpr (GLU) {
                f32x4 gt = acc[0][ct] * inv;
                f32x4 up = acc[1][ct] * inv;
                if (a.scales) {
                    gt *= as_f32x4(e.sc[0]);
                    up *= as_f32x4(e.sc[1]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
            } else {
                v = acc[0][ct] * inv;
                if (a.scales) v *= as_f32x4(e.sc[0]);
            }
            {
                if (m >= a.M || o >= a.N) continue;
                if (a.vec_store) {
                    if (want_res) v += epi_res(a.res_dt, e.res32[ct], e.res16[ct]);
                    void* dst = a.y;
                    int col = o;
                    if (a.flags & EP_SPLIT) {
                        const int blk = o / a.split_period;
                        dst = (blk & 1) ? a.y2 : a.y;
                        col = (blk >> 1) * a.split_period + (o - blk * a.split_period);
                    }
                    store_act4(dst, a.ydt, (int64_t)m * a.ldy + col, v);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int oi = o + i;
                        if (oi >= a.N) break;
                        float vi = v[i];
                        if (want_res) vi += load_act(a.res, a.res_dt, (int64_t)m * a.ld_res + oi);
                        void* dst = a.y;
                        int col = oi;
                        if (a.flags & EP_SPLIT) {
                            const int blk = oi / a.split_period;
                            dst = (blk & 1) ? a.y2 : a.y;
                            col = (blk >> 1) * a.split_period + (oi - blk * a.split_period);
                        }
                        store_act(dst, a.ydt, (int64_t)m * a.ldy + col, vi);
                    }
                }
            }
        }
    }

    if constexpr (ARGMAX) {
        if (wave_id != 0) return;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
            for (int sh = 16; sh <= 32; sh <<= 1) {
                const unsigned long long other = __shfl_xor(best[ct], sh);
                best[ct] = other > best[ct] ? other : best[ct];
            }
            const int m = ct * 16 + r;
            if (g == 0 && m < a.M && best[ct] != 0ull)
                __hip_atomic_fetch_max(&a.keys[m], best[ct], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // the key updates are agent-scope read-modify-writes performed at the
        // device coherence point; waiting for their completion orders them
        // before this workgroup's completion count
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old == gridDim.x - 1) {
            for (int mm = lane; mm < ain.M; mm += 64) {
                const unsigned long long kk =
                    __hip_atomic_exchange(&ain.keys[mm], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ain.ids[mm] = (int32_t)key_index(kk);
                if (ain.maxv) ain.maxv[mm] = key_value(kk);
            }
            if (lane == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// host-side launch
// ---------------------------------------------------------------------------
int gemv_waves(int wf, int M, bool glu, bool argmax, bool norm, int nw_wanted) {
    if (glu || argmax || M > 16) return 4;
    if (nw_wanted >= 16) return (wf == WF_BF16 && !norm) ? 16 : (norm ? 4 : 8);
    if (nw_wanted >= 8) return norm ? 4 : 8;
    return 4;
}

int gemv_argmax_tiles(int wf) { return wf == WF_I8 ? ArgmaxTiles<WF_I8>::v : ArgmaxTiles<WF_BF16>::v; }

bool gemv_supported(int wf, int xdt, int M, bool norm) {
    if (M < 1 || M > 32 || (M > 16 && norm)) return false;
    return (wf == WF_BF16 && xdt == DT_BF16) || (wf == WF_I8 && (xdt == DT_F16 || xdt == DT_BF16));
}

template <int WF, int XDT, int CT, bool NORM, bool GAM>
static hipError_t launch_n(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    const dim3 gd(grid), bd(nw * 64);
    if (argmax) {
        if (glu || NORM) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemv_kernel<WF, XDT, CT, false, true, 4, false, false>), gd, dim3(256), 0, st, a);
    } else if (glu) {
        if (nw != 4) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemv_kernel<WF, XDT, CT, true, false, 4, NORM, GAM>), gd, dim3(256), 0, st, a);
    } else if (nw == 16) {
        // 16-wave workgroups fit their registers only without the RMSNorm
        // prologue and with BF16 weights
        if constexpr (NORM || WF != WF_BF16 || CT != 1) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((gemv_kernel<WF, XDT, CT, false, false, 16, false, false>), gd, bd, 0, st, a);
    } else if (nw == 8) {
        if constexpr (NORM || CT != 1) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((gemv_kernel<WF, XDT, CT, false, false, 8, false, false>), gd, bd, 0, st, a);
    } else {
        hipLaunchKernelGGL((gemv_kernel<WF, XDT, CT, false, false, 4, NORM, GAM>), gd, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int WF, int XDT, int CT>
static hipError_t launch_c(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    if constexpr (CT == 2) {  // two token tiles leave no registers for the RMSNorm operands
        if (a.flags & EP_NORM) return hipErrorInvalidValue;
        return launch_n<WF, XDT, CT, false, false>(a, glu, argmax, nw, grid, st);
    } else {
        if (a.flags & EP_NORM) {
            if (a.gamma) return launch_n<WF, XDT, CT, true, true>(a, glu, argmax, nw, grid, st);
            return launch_n<WF, XDT, CT, true, false>(a, glu, argmax, nw, grid, st);
        }
        return launch_n<WF, XDT, CT, false, false>(a, glu, argmax, nw, grid, st);
    }
}

template <int WF, int XDT>
static hipError_t launch_x(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    if ((a.tg_grid ? a.tg_size : a.M) <= 16) return launch_c<WF, XDT, 1>(a, glu, argmax, nw, grid, st);
    return launch_c<WF, XDT, 2>(a, glu, argmax, nw, grid, st);
}

hipError_t launch_gemv(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int nw, int grid,
                       hipStream_t stream) {
    const int mg = a.tg_grid ? a.tg_size : a.M;  // tokens one workgroup sees
    if (!gemv_supported(wf, xdt, mg, (a.flags & EP_NORM) != 0)) return hipErrorInvalidValue;
    if (a.tg_grid && (grid % a.tg_grid != 0 || (int64_t)(grid / a.tg_grid) * a.tg_size < a.M))
        return hipErrorInvalidValue;
    if (nw != 4 && nw != 8 && nw != 16) return hipErrorInvalidValue;
    if (a.S < 1 || (a.tg_grid ? a.tg_grid : grid) % a.S != 0) return hipErrorInvalidValue;
    if (wf == WF_BF16) return launch_x<WF_BF16, DT_BF16>(a, glu, argmax, nw, grid, stream);
    if (xdt == DT_F16) return launch_x<WF_I8, DT_F16>(a, glu, argmax, nw, grid, stream);
    return launch_x<WF_I8, DT_BF16>(a, glu, argmax, nw, grid, stream);
}

}  // namespace qwk
