// qw_skinny.hip -- small-M projection kernel for gfx950 (decode GEMV / skinny GEMM,
// tied lm_head with fused greedy argmax).
//
// Data flow.  Weights stream once from HBM straight into MFMA A registers:
// one k-step of a 16-row tile is a single fully coalesced 1 KB wave load in
// the packed tile order of qw_device.hpp.  The activations of up to 32 tokens
// are staged once per workgroup into LDS, already in the MFMA input type
// (bf16, f16 or f32; an FP32 activation feeding a 16-bit MFMA is kept as a
// hi + lo pair), with the RMSNorm weight (1 + gamma) folded in; the per-token
// sums of squares for the RMSNorm are taken during the same staging pass.
// Each k-step then costs one weight load, one or two ds_read_b128 and the
// MFMAs (16 rows x 16 tokens each).  M <= 16 uses one token column tile
// (CT = 1), M <= 32 two.
//
// Work decomposition.  An item is a 16-row output tile (a gate/up tile pair
// for GLU weights) over one K split.  A workgroup of NW waves owns one item at
// a time, its waves take contiguous pieces of the split, and their partial
// tiles meet in LDS (fixed summation order).  Workgroups walk the items
// grid-stride and keep one K split for their whole life, so the activation
// staging happens once per workgroup; the weight loads of the next item are
// issued before the current item's reduction and epilogue.  K is split across
// workgroups only when the host asks for it (few output tiles, or an
// activation slice too large for LDS); the last of the S workgroups of a tile
// (agent-scope counter) sums the S partials in split order -- deterministic --
// and runs the epilogue.  Counters return to zero, so no memset is needed and
// the kernel can be captured in a graph.
//
// Epilogue: per-row INT8 scale, 1/rms of the RMSNorm, SiLU(gate)*up for GLU
// pairs, residual add, Q/gate de-interleave, or -- for the lm_head -- a
// running (logit, index) maximum per token merged across the grid with a
// 64-bit atomic max on an orderable key (ties resolve to the lowest index)
// and decoded by the last workgroup.
//
// Reference operators replaced: cutlass_style_gemv_kernel / _bf16 /
// _fused_silu (cutlass_gemm_wrapper.cuh:41-200), int8_gemv_batch_kernel
// (mlp_cuda.cu:158-180), lm_head_gemv_kernel_optimized (lm_head_cuda.cu:38-99)
// + block_argmax_kernel (gpu_sampler_argmax.cu:14-43), and the thread-per-row
// projection kernels of the attention operators.
#include "qw_stream.hpp"

namespace qwk {

template <int WF, int XDT, int CT, bool GLU, bool ARGMAX, int NW>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(SkinnyArgs ain) {
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
        a.x = static_cast<const uint8_t*>(ain.x) + (int64_t)tok0 * ain.ldx * XSize<XDT>::v;
        const int ys = ain.ydt == DT_F32 ? 4 : 2;
        if (ain.y) a.y = static_cast<uint8_t*>(ain.y) + (int64_t)tok0 * ain.ldy * ys;
        if (ain.y2) a.y2 = static_cast<uint8_t*>(ain.y2) + (int64_t)tok0 * ain.ldy * ys;
        if (ain.res) a.res = static_cast<const uint8_t*>(ain.res) + (int64_t)tok0 * ain.ld_res * (ain.res_dt == DT_F32 ? 4 : 2);
        a.keys = ain.keys + tok0;
    }
    constexpr int U = (GLU && NW == 16) ? 4 : 8;
    constexpr int KE = WTraits<WF>::KE;
    constexpr int RT = GLU ? 2 : 1;
    constexpr int F = RT * CT;
    constexpr int ROWS = CT * 16;
    constexpr int OS = OpSize<WF>::v;
    __shared__ f32x4 red[NW][F][64];
    __shared__ float ss_tok[ROWS];
    __shared__ float ss_scratch[NW * ROWS];
    extern __shared__ uint8_t xs[];  // staged activations

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const bool norm = (a.flags & EP_NORM) != 0;
    const bool want_res = !ARGMAX && (a.flags & EP_RESIDUAL);

    // This workgroup's K split is constant (the host makes gdim % S == 0),
    // so its tile group advances by gdim / S per item: no division in
    // the item loop.
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
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * RT * a.ksteps * 1024u));

    unsigned long long best[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) best[ct] = 0ull;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * XSize<XDT>::v));
    // no gamma (the weight carries it): an empty buffer, every gamma load reads 0
    const __amdgpu_buffer_rsrc_t gr =
        make_rsrc(norm && a.gamma ? (const void*)a.gamma : a.x, norm && a.gamma ? (uint32_t)a.K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)a.n_groups * RT * 64u : 0u);
    const int res_size = a.res_dt == DT_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(want_res ? a.res : a.x, want_res ? (uint32_t)((uint64_t)a.M * a.ld_res * res_size) : 0u);

    u32x4 A[U][RT];
    EpiOps<RT, CT> epi, epi_next;
    int item = bid;
    int grp = a.S > 1 ? bid / a.S : bid;
    int n = min(U, kend - kb);
    // activation loads first, then the epilogue operands, then the weights;
    // the activations are converted into LDS while the weights stream in
    const int kr = (ks1 - ks0) * 4 * KE;
    // chunks of 8 activations each thread stages (1, 2 or 4 up front)
    const int rp = 1 << (32 - __builtin_clz((unsigned)a.M));  // M+1 rounded up to a power of 2
    const int cpt = ((kr / 8) * rp + NW * 64 - 1) / (NW * 64);
    auto prologue = [&](auto sq_tag, auto norm_tag) {
        constexpr int SQ = decltype(sq_tag)::value;
        constexpr bool NORM = decltype(norm_tag)::value;
        XStage<XDT, SQ> st;
        stage_issue<WF, XDT, NW, SQ, NORM>(a, xr, gr, ks0 * 4 * KE, kr, st);
        load_epi<RT, CT>(a, sr, rr, grp, item < a.n_items, lane, epi);
        __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the weight stream
        issue_weights<RT, U>(a, wrs, grp, kb, item < a.n_items ? n : 0, lane, A);
        __builtin_amdgcn_sched_barrier(0);
        stage_finish<WF, XDT, CT, NW, SQ, NORM>(a, xr, gr, ks0 * 4 * KE, kr, st, xs, ss_tok, ss_scratch);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    if (norm) {
        if (cpt <= 1) prologue(I1{}, std::true_type{});
        else if (cpt <= 2) prologue(I2{}, std::true_type{});
        else prologue(I4{}, std::true_type{});
    } else {
        if (cpt <= 1) prologue(I1{}, std::false_type{});
        else if (cpt <= 2) prologue(I2{}, std::false_type{});
        else prologue(I4{}, std::false_type{});
    }
    __syncthreads();

    const int ls = lds_row_elems<WF>(kr);
    const int plane_bytes = (a.M + 1) * ls * OS;
    int xrow[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) xrow[ct] = min(ct * 16 + r, a.M);

    while (item < a.n_items) {
        f32x4 acc[RT][CT];
#pragma unroll
        for (int j = 0; j < CT; ++j)
#pragma unroll
            for (int i = 0; i < RT; ++i) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (;;) {
            if (n == U) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int relk = (kb + u - ks0) * 4 * KE + g * KE;
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        BOps<WF, XDT> b;
                        read_bops<WF, XDT>(b, xs + ((int64_t)xrow[ct] * ls + relk) * OS, plane_bytes);
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = unit_mfma<WF, XDT>(A[u][rt], b, acc[rt][ct]);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (u < n) {
                        const int relk = (kb + u - ks0) * 4 * KE + g * KE;
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct) {
                            BOps<WF, XDT> b;
                            read_bops<WF, XDT>(b, xs + ((int64_t)xrow[ct] * ls + relk) * OS, plane_bytes);
#pragma unroll
                            for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = unit_mfma<WF, XDT>(A[u][rt], b, acc[rt][ct]);
                        }
                    }
                }
            }
            kb += n;
            if (kb >= kend) break;
            n = min(U, kend - kb);
            issue_weights<RT, U>(a, wrs, grp, kb, n, lane, A);
        }
        const int cur_grp = grp;
        item += gdim;
        grp += grp_step;
        kb = kb0;
        n = min(U, kend - kb);
        const bool more = item < a.n_items;
        if (more) {  // uniform; the loop only comes back through this path
            load_epi<RT, CT>(a, sr, rr, grp, true, lane, epi_next);
            issue_weights<RT, U>(a, wrs, grp, kb, n, lane, A);
        }

        // ---- reduce the NW pieces in LDS (fixed order) ----
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) red[wave_id][rt * CT + ct][lane] = acc[rt][ct];
        __syncthreads();
        for (int t = threadIdx.x; t < F * 64; t += NW * 64) {
            const int f = t >> 6, l = t & 63;
            f32x4 sum = red[0][f][l];
#pragma unroll
            for (int w = 1; w < NW; ++w) sum += red[w][f][l];
            red[0][f][l] = sum;
        }
        __syncthreads();
        if (wave_id != 0) continue;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = red[0][rt * CT + ct][lane];
        float ss[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) ss[ct] = norm ? ss_tok[ct * 16 + r] : 0.0f;
        EpiOps<RT, CT> e = epi;
        epi = epi_next;

        const int grp = cur_grp;
        bool finish = true;
        if constexpr (!ARGMAX) {
            if (a.S > 1) {
                // Cross-workgroup split-K hand-off, no fence: the partial tile
                // (and the partial sums of squares) go out as agent-scope
                // atomic stores (written through to the device coherence
                // point), s_waitcnt vmcnt(0) waits for their completion, then
                // the agent-scope counter increment.  The last of the S
                // workgroups reads the S partials back with agent-scope atomic
                // loads, in split order (deterministic), and returns the
                // counter to zero.
                constexpr int REC = F * 4 + CT;  // floats per lane per split
                float* P = reinterpret_cast<float*>(a.partials) + ((int64_t)(grp + gofs) * a.S * 64 + lane) * REC;
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
                    old = __hip_atomic_fetch_add(&a.counters[grp + gofs], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
                                acc[f / CT][f % CT][i] += __hip_atomic_load(q + f * 4 + i, __ATOMIC_RELAXED,
                                                                            __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct)
                            ss[ct] += __hip_atomic_load(q + F * 4 + ct, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    if (lane == 0)
                        __hip_atomic_store(&a.counters[grp + gofs], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (!finish) continue;

        float inv[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) inv[ct] = norm ? 1.0f / sqrtf(ss[ct] / (float)a.K + a.eps) : 1.0f;

        // ---- epilogue (wave 0) ----
        const int o = grp * 16 + g * 4;  // first of this lane's 4 logical rows
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int m = ct * 16 + r;
            f32x4 v;
            if constexpr (GLU) {
                f32x4 gt = acc[0][ct] * inv[ct];
                f32x4 up = acc[1][ct] * inv[ct];
                if (a.scales) {
                    gt *= as_f32x4(e.sc[0]);
                    up *= as_f32x4(e.sc[1]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
            } else {
                v = acc[0][ct] * inv[ct];
                if (a.scales) v *= as_f32x4(e.sc[0]);
            }
            if constexpr (ARGMAX) {
                if (m < a.M) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (o + i < a.N) {
                            unsigned long long kk = argmax_key(v[i], (uint32_t)(o + i));
                            best[ct] = kk > best[ct] ? kk : best[ct];
                        }
                    }
                }
            } else {
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
        // merge the four row groups of each token column, then the grid
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
            for (int sh = 16; sh <= 32; sh <<= 1) {
                unsigned long long other = __shfl_xor(best[ct], sh);
                best[ct] = other > best[ct] ? other : best[ct];
            }
            const int m = ct * 16 + r;
            if (g == 0 && m < a.M && best[ct] != 0ull)
                __hip_atomic_fetch_max(&a.keys[m], best[ct], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // The key updates are agent-scope read-modify-writes, performed at
        // the device coherence point; waiting for their completion orders
        // them before this workgroup's completion count.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old == gridDim.x - 1) {
            for (int m = lane; m < ain.M; m += 64) {
                unsigned long long kk = __hip_atomic_exchange(&ain.keys[m], 0ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
                ain.ids[m] = (int32_t)key_index(kk);
                if (ain.maxv) ain.maxv[m] = key_value(kk);
            }
            if (lane == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// host-side launch
// ---------------------------------------------------------------------------
size_t skinny_lds_bytes(int wf, int xdt, int M, int ksteps_per_split) {
    const int os = wf == WF_F32 ? 4 : 2;
    const int ke = wf == WF_F32 ? 4 : (wf == WF_BF16 ? 8 : 16);
    const bool split = (wf == WF_BF16 && xdt != DT_BF16) || (wf == WF_I8 && xdt == DT_F32);
    const size_t row = (size_t)ksteps_per_split * 4 * ke * os + 16;
    return (split ? 2 : 1) * (size_t)(M + 1) * row;
}

template <typename Kern>
static hipError_t launch_k(Kern k, const SkinnyArgs& a, int nw, int grid, size_t smem, hipStream_t st) {
    {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)kSkinnyMaxLds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(nw * 64), smem, st, a);
    return hipGetLastError();
}

template <int WF, int XDT, int CT>
static hipError_t launch3(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, size_t smem, hipStream_t st) {
    if constexpr (CT == 1) {
        if (!argmax && nw == 16) {
            if (glu) return launch_k(skinny_kernel<WF, XDT, CT, true, false, 16>, a, 16, grid, smem, st);
            return launch_k(skinny_kernel<WF, XDT, CT, false, false, 16>, a, 16, grid, smem, st);
        }
        if (!argmax && nw == 8) {
            if (glu) return launch_k(skinny_kernel<WF, XDT, CT, true, false, 8>, a, 8, grid, smem, st);
            return launch_k(skinny_kernel<WF, XDT, CT, false, false, 8>, a, 8, grid, smem, st);
        }
    }
    if (argmax) {
        if (glu) return hipErrorInvalidValue;
        return launch_k(skinny_kernel<WF, XDT, CT, false, true, 4>, a, 4, grid, smem, st);
    }
    if (glu) return launch_k(skinny_kernel<WF, XDT, CT, true, false, 4>, a, 4, grid, smem, st);
    return launch_k(skinny_kernel<WF, XDT, CT, false, false, 4>, a, 4, grid, smem, st);
}

template <int WF, int XDT>
static hipError_t launch2(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, size_t smem, hipStream_t st) {
    if ((a.tg_grid ? a.tg_size : a.M) <= 16) return launch3<WF, XDT, 1>(a, glu, argmax, nw, grid, smem, st);
    return launch3<WF, XDT, 2>(a, glu, argmax, nw, grid, smem, st);
}

template <int WF>
static hipError_t launch1(const SkinnyArgs& a, int xdt, bool glu, bool argmax, int nw, int grid, size_t smem,
                          hipStream_t st) {
    switch (xdt) {
        case DT_F32: return launch2<WF, DT_F32>(a, glu, argmax, nw, grid, smem, st);
        case DT_BF16: return launch2<WF, DT_BF16>(a, glu, argmax, nw, grid, smem, st);
        case DT_F16: return launch2<WF, DT_F16>(a, glu, argmax, nw, grid, smem, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_skinny(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int nw, int grid,
                         hipStream_t stream) {
    const int mg = a.tg_grid ? a.tg_size : a.M;  // tokens one workgroup sees
    if (a.M < 1 || mg < 1 || mg > 32) return hipErrorInvalidValue;
    if (a.tg_grid && (grid % a.tg_grid != 0 || (int64_t)(grid / a.tg_grid) * a.tg_size < a.M))
        return hipErrorInvalidValue;
    if (nw != 4 && nw != 8 && nw != 16) return hipErrorInvalidValue;
    if (a.S < 1 || (a.tg_grid ? a.tg_grid : grid) % a.S != 0) return hipErrorInvalidValue;
    const size_t smem = skinny_lds_bytes(wf, xdt, mg, (a.ksteps + a.S - 1) / a.S);
    if (smem > kSkinnyMaxLds) return hipErrorInvalidValue;
    switch (wf) {
        case WF_F32: return launch1<WF_F32>(a, xdt, glu, argmax, nw, grid, smem, stream);
        case WF_BF16: return launch1<WF_BF16>(a, xdt, glu, argmax, nw, grid, smem, stream);
        case WF_I8: return launch1<WF_I8>(a, xdt, glu, argmax, nw, grid, smem, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qwk
