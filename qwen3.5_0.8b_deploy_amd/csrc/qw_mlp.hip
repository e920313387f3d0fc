// qw_mlp.hip -- the decoder MLP block in one launch (small M):
//     y = [residual +] down( silu(gate . xn) * (up . xn) ),  xn = RMSNorm(x)*(1+gamma)
//
// Why one launch.  At decode sizes (22 MB of BF16 weights per layer) two
// separate kernels pay two launch/ramp/tail costs, and the down projection
// (1024 rows = 64 tiles) can occupy only a quarter of the chip.  Here the
// gate/up tile pairs ("up tasks") and the down tiles ("down tasks") share one
// grid: a down task issues its weight loads first, then waits for the last up
// task, so the down weights stream in while the gate/up pass still runs.
//
// Scheduling.  Workgroups take tasks from a ticket counter in order: all up
// tickets come before all down tickets.  A down task waits only for up tasks,
// and every up ticket was handed to a workgroup that is already running (and
// never waits), so the wait always ends -- whatever the number of resident
// workgroups.  The wait is still bounded: after ~0.2 s of polling it sets the
// error flag and gives up instead of hanging.  The last workgroup to leave
// returns the counters to zero (no memset, graph-capture safe).
//
// Data hand-off.  Up tasks write the intermediate h (in the MFMA input type
// of the down weights) with agent-scope atomic stores, wait for their
// completion, then count themselves done; down tasks stage h into LDS with
// device-coherent (sc1) loads.  No cache write-back or invalidate is needed.
//
// Replaces CudaMLP::forward / forward_add_residual (mlp_cuda.cu:295-337,
// with the residual added), launch_cutlass_gemv_fused_silu
// (cutlass_gemm_wrapper.cuh:141-200, 240-263) and the post-norm + MLP +
// residual chain of CudaLayer::forward (cuda_engine.cu:119-124).
#include "qw_stream.hpp"

namespace qwk {

constexpr int MLP_NW = 8;

template <int WF, int XDT, int CT, int RT, int U, int NW>
__device__ __forceinline__ void stream_chunks(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t wrs, int grp, int ks0,
                                              int kb, int kend, int n, int lane, u32x4 (&A)[U][RT],
                                              const uint8_t* xs, int ls, int plane_bytes, const int (&xrow)[CT],
                                              f32x4 (&acc)[RT][CT]) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int OS = OpSize<WF>::v;
    const int g = lane >> 4;
    for (;;) {
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
        kb += n;
        if (kb >= kend) break;
        n = min(U, kend - kb);
        issue_weights<RT, U>(a, wrs, grp, kb, n, lane, A);
    }
}

// Sum the NW waves' tiles in LDS (fixed order); every wave gets the result.
// red holds NW * F * 64 f32x4.
template <int NW, int F>
__device__ __forceinline__ void reduce_waves(f32x4* red, f32x4* acc, int wave_id, int lane) {
#pragma unroll
    for (int f = 0; f < F; ++f) red[(wave_id * F + f) * 64 + lane] = acc[f];
    __syncthreads();
    for (int t = threadIdx.x; t < F * 64; t += NW * 64) {
        f32x4 sum = red[t];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[w * F * 64 + t];
        red[t] = sum;
    }
    __syncthreads();
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] = red[f * 64 + lane];
}

// Stage-issue, epilogue operands, weights, stage-finish -- in that order.
template <int WF, int XDT, int CT, int RT, int U, int NW, bool NORM, int XAUX>
__device__ __forceinline__ void prologue(const SkinnyArgs& a, int cpt, __amdgpu_buffer_rsrc_t xr,
                                         __amdgpu_buffer_rsrc_t gr, __amdgpu_buffer_rsrc_t sr,
                                         __amdgpu_buffer_rsrc_t rr, __amdgpu_buffer_rsrc_t wrs, int grp, int kb,
                                         int n, int lane, int kr, EpiOps<RT, CT>& epi, u32x4 (&A)[U][RT],
                                         uint8_t* xs, float* ss_tok, float* ss_scratch, bool weights_first) {
    auto body = [&](auto sq_tag) {
        constexpr int SQ = decltype(sq_tag)::value;
        XStage<XDT, SQ> st;
        if (weights_first) {
            // the activations are not ready yet: weights were issued earlier
            stage_issue<WF, XDT, NW, SQ, NORM, XAUX>(a, xr, gr, 0, kr, st);
        } else {
            stage_issue<WF, XDT, NW, SQ, NORM, XAUX>(a, xr, gr, 0, kr, st);
            load_epi<RT, CT>(a, sr, rr, grp, true, lane, epi);
            __builtin_amdgcn_sched_barrier(0);
            issue_weights<RT, U>(a, wrs, grp, kb, n, lane, A);
            __builtin_amdgcn_sched_barrier(0);
        }
        stage_finish<WF, XDT, CT, NW, SQ, NORM, XAUX>(a, xr, gr, 0, kr, st, xs, ss_tok, ss_scratch);
    };
    if (cpt <= 1) body(std::integral_constant<int, 1>{});
    else if (cpt <= 2) body(std::integral_constant<int, 2>{});
    else body(std::integral_constant<int, 4>{});
}

template <int XDT>
__device__ __forceinline__ int chunks_per_thread(int M, int kr, int nt) {
    const int rp = 1 << (32 - __builtin_clz((unsigned)M));
    return ((kr / 8) * rp + nt - 1) / nt;
}

// WF: weight format (gate/up and down share it); XDT: dtype of x.  The
// intermediate h is held in the MFMA input type of WF.
template <int WF, int XDT, bool NORM>
__global__ __launch_bounds__(MLP_NW * 64) void mlp_kernel(MlpArgs p) {
    constexpr int NW = MLP_NW;
    constexpr int KE = WTraits<WF>::KE;
    constexpr int OS = OpSize<WF>::v;
    constexpr int HDT = WF == WF_BF16 ? DT_BF16 : (WF == WF_I8 ? DT_F16 : DT_F32);
    constexpr int UA = 8, UB = 16;
    __shared__ f32x4 red[NW * 2 * 64];
    __shared__ float ss_tok[16];
    __shared__ float ss_scratch[NW * 16];
    __shared__ int tick_s;
    extern __shared__ uint8_t xs[];

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int total = p.n_up + p.n_down;

    for (;;) {
        if (threadIdx.x == 0)
            tick_s = (int)__hip_atomic_fetch_add(&p.ctl[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int t = tick_s;
        __syncthreads();
        if (t >= total) break;

        if (t < p.n_up) {
            // ---------------- gate/up tile pair t: x -> h ----------------
            const SkinnyArgs& a = p.up;
            int kb, kend;
            wave_range<NW>(0, a.ksteps, wave_id, kb, kend);
            const int n = min(UA, kend - kb);
            const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * 2 * a.ksteps * 1024u));
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * XSize<XDT>::v));
            const __amdgpu_buffer_rsrc_t gr = make_rsrc(NORM && a.gamma ? (const void*)a.gamma : a.x, NORM && a.gamma ? (uint32_t)a.K * 4u : 0u);
            const __amdgpu_buffer_rsrc_t sr =
                make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)a.n_groups * 2 * 64u : 0u);
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.x, 0u);
            const int kr = a.ksteps * 4 * KE;
            EpiOps<2, 1> epi;
            u32x4 A[UA][2];
            prologue<WF, XDT, 1, 2, UA, NW, NORM, 0>(a, chunks_per_thread<XDT>(a.M, kr, NW * 64), xr, gr, sr, rr, wrs,
                                                   t, kb, n, lane, kr, epi, A, xs, ss_tok, ss_scratch, false);
            __syncthreads();
            const int ls = lds_row_elems<WF>(kr);
            const int plane_bytes = (a.M + 1) * ls * OS;
            const int xrow[1] = {min(r, a.M)};
            f32x4 acc[2][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}, {f32x4{0.f, 0.f, 0.f, 0.f}}};
            stream_chunks<WF, XDT, 1, 2, UA, NW>(a, wrs, t, 0, kb, kend, n, lane, A, xs, ls, plane_bytes, xrow, acc);
            f32x4 accf[2] = {acc[0][0], acc[1][0]};
            reduce_waves<NW, 2>(red, accf, wave_id, lane);
            if (wave_id == 0) {
                float inv = 1.0f;
                if (NORM) inv = 1.0f / sqrtf(ss_tok[r] / (float)a.K + a.eps);
                f32x4 gt = accf[0] * inv, up = accf[1] * inv;
                if (a.scales) {
                    gt *= as_f32x4(epi.sc[0]);
                    up *= as_f32x4(epi.sc[1]);
                }
                f32x4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
                const int o = t * 16 + g * 4;
                if (r < a.M && o < a.N) {
                    // device-coherent stores of h (read by other workgroups in this launch)
                    if constexpr (HDT == DT_F32) {
                        float* dst = reinterpret_cast<float*>(a.y) + (int64_t)r * a.ldy + o;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            __hip_atomic_store(dst + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        uint32_t* dst = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned short*>(a.y) + (int64_t)r * a.ldy + o);
                        const uint32_t w0 = op_bits<WF>(v[0]) | (op_bits<WF>(v[1]) << 16);
                        const uint32_t w1 = op_bits<WF>(v[2]) | (op_bits<WF>(v[3]) << 16);
                        __hip_atomic_store(dst, w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(dst + 1, w1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if (lane == 0) __hip_atomic_fetch_add(&p.ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            // ---------------- down tile j: h -> y (+ residual) ----------------
            const int j = t - p.n_up;
            const SkinnyArgs& a = p.down;
            int kb, kend;
            wave_range<NW>(0, a.ksteps, wave_id, kb, kend);
            const int n = min(UB, kend - kb);
            const bool want_res = (a.flags & EP_RESIDUAL) != 0;
            const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * a.ksteps * 1024u));
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * XSize<HDT>::v));
            const __amdgpu_buffer_rsrc_t sr =
                make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)a.n_groups * 64u : 0u);
            const int res_size = a.res_dt == DT_F32 ? 4 : 2;
            const __amdgpu_buffer_rsrc_t rr =
                make_rsrc(want_res ? a.res : a.x, want_res ? (uint32_t)((uint64_t)a.M * a.ld_res * res_size) : 0u);
            // weights and epilogue operands do not depend on h: issue them now
            EpiOps<1, 1> epi;
            u32x4 A[UB][1];
            load_epi<1, 1>(a, sr, rr, j, true, lane, epi);
            issue_weights<1, UB>(a, wrs, j, kb, n, lane, A);
            // wait for every gate/up tile (bounded)
            if (threadIdx.x == 0) {
                unsigned it = 0;
                while (__hip_atomic_load(&p.ctl[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)p.n_up) {
                    __builtin_amdgcn_s_sleep(2);
                    if (++it > (1u << 22)) {
                        __hip_atomic_store(&p.ctl[3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __syncthreads();
            const int kr = a.ksteps * 4 * KE;
            prologue<WF, HDT, 1, 1, UB, NW, false, AUX_SC1>(a, chunks_per_thread<HDT>(a.M, kr, NW * 64), xr, xr, sr, rr,
                                                            wrs, j, kb, n, lane, kr, epi, A, xs, ss_tok, ss_scratch,
                                                            true);
            __syncthreads();
            const int ls = lds_row_elems<WF>(kr);
            const int plane_bytes = (a.M + 1) * ls * OS;
            const int xrow[1] = {min(r, a.M)};
            f32x4 acc[1][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
            stream_chunks<WF, HDT, 1, 1, UB, NW>(a, wrs, j, 0, kb, kend, n, lane, A, xs, ls, plane_bytes, xrow, acc);
            f32x4 accf[1] = {acc[0][0]};
            reduce_waves<NW, 1>(red, accf, wave_id, lane);
            if (wave_id == 0) {
                f32x4 v = accf[0];
                if (a.scales) v *= as_f32x4(epi.sc[0]);
                const int o = j * 16 + g * 4;
                if (r < a.M && o < a.N) {
                    if (a.vec_store) {
                        if (want_res) v += epi_res(a.res_dt, epi.res32[0], epi.res16[0]);
                        store_act4(a.y, a.ydt, (int64_t)r * a.ldy + o, v);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (o + i >= a.N) break;
                            float vi = v[i];
                            if (want_res) vi += load_act(a.res, a.res_dt, (int64_t)r * a.ld_res + o + i);
                            store_act(a.y, a.ydt, (int64_t)r * a.ldy + o + i, vi);
                        }
                    }
                }
            }
        }
    }
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(&p.ctl[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1) {  // last one out: reset for the next launch
            __hip_atomic_store(&p.ctl[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&p.ctl[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&p.ctl[2], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

size_t mlp_fused_lds_bytes(int wf, int xdt, int M, int H, int I) {
    const int hdt = wf == WF_BF16 ? DT_BF16 : (wf == WF_I8 ? DT_F16 : DT_F32);
    const int ke = wf == WF_F32 ? 4 : (wf == WF_BF16 ? 8 : 16);
    const size_t up = skinny_lds_bytes(wf, xdt, M, H / (4 * ke));
    const size_t down = skinny_lds_bytes(wf, hdt, M, I / (4 * ke));
    return up > down ? up : down;
}

template <typename Kern>
static hipError_t launch_mlp_k(Kern k, const MlpArgs& p, int grid, size_t smem, hipStream_t st) {
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSkinnyMaxLds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(MLP_NW * 64), smem, st, p);
    return hipGetLastError();
}

template <int WF, int XDT>
static hipError_t launch_mlp2(const MlpArgs& p, bool norm, int grid, size_t smem, hipStream_t st) {
    if (norm) return launch_mlp_k(mlp_kernel<WF, XDT, true>, p, grid, smem, st);
    return launch_mlp_k(mlp_kernel<WF, XDT, false>, p, grid, smem, st);
}

template <int WF>
static hipError_t launch_mlp1(const MlpArgs& p, int xdt, bool norm, int grid, size_t smem, hipStream_t st) {
    switch (xdt) {
        case DT_F32: return launch_mlp2<WF, DT_F32>(p, norm, grid, smem, st);
        case DT_BF16: return launch_mlp2<WF, DT_BF16>(p, norm, grid, smem, st);
        case DT_F16: return launch_mlp2<WF, DT_F16>(p, norm, grid, smem, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_mlp_fused(const MlpArgs& p, int wf, int xdt, int grid, hipStream_t stream) {
    if (p.up.M < 1 || p.up.M > 16) return hipErrorInvalidValue;
    const size_t smem = mlp_fused_lds_bytes(wf, xdt, p.up.M, p.up.K, p.down.K);
    if (smem > kSkinnyMaxLds) return hipErrorInvalidValue;
    const bool norm = (p.up.flags & EP_NORM) != 0;
    switch (wf) {
        case WF_F32: return launch_mlp1<WF_F32>(p, xdt, norm, grid, smem, stream);
        case WF_BF16: return launch_mlp1<WF_BF16>(p, xdt, norm, grid, smem, stream);
        case WF_I8: return launch_mlp1<WF_I8>(p, xdt, norm, grid, smem, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qwk
