// qw_mlp.hip -- the decoder MLP block in one launch (decode, M <= 16 tokens):
//     y = [residual +] down( silu(gate . xn) * (up . xn) ),  xn = RMSNorm(x)*(1+gamma)
//
// Why one launch.  At decode sizes (22 MB of BF16 weights per layer) the two
// projections are each a few microseconds of streaming, and two launches pay
// two ramp/tail costs with the down weights only requested once the gate/up
// pass is over.  Here every weight byte of the block is requested at the
// start of the launch, so the down weights stream in while the gate/up pass
// still runs, and the block costs one ramp.
//
// Decomposition (no split-K, so the only cross-workgroup hand-off is h).
// Workgroups are 16 waves, one per CU (224 + 32 = 256 at the Qwen shape):
//   * workgroups [0, ceil(n_down/2)): "down" workgroup j owns output rows
//     [32j, 32j+32), two 16-row tiles, 8 waves per tile cutting the K = I
//     reduction in eight; each wave holds ALL its down-weight k-steps in
//     registers from the start;
//   * the rest: "gate/up" workgroup i owns the gate/up tile pair i
//     (intermediate rows [16i, 16i+16)) over the whole K = H, cut in
//     sixteen by wave.
// A CU never hosts a down and a gate/up workgroup together: a gate/up
// workgroup's h stores would otherwise queue behind the down workgroup's
// 224 KB of weight loads in the CU's memory pipeline (measured: the slowest
// gate/up workgroups finished 2 us late with 8-wave workgroups sharing CUs).
// A gate/up workgroup writes its 16 rows of h with agent-scope stores, waits
// for their completion and counts itself done in one of 32 counter slots.
// A down workgroup, its weights already requested, waits until the slots
// sum to n_up, then loads its h fragments with device-coherent loads.  Down
// workgroups come first in the grid so they are resident first; gate/up
// workgroups never wait, so the wait always ends (whatever the number of
// resident workgroups, as long as the waiting ones fit).  The wait is still
// bounded: after 0.2 s by the constant 100 MHz real-time counter it sets the
// error flag (read with qw_device_error, which also returns the counters to
// zero, since late gate/up arrivals of such a launch leave counts behind)
// instead of hanging.  The last down workgroup to leave returns the counters
// to zero (no memset: graph-capture safe).
//
// Operands follow the register-direct GEMV (qw_gemv.hip): each lane loads
// its MFMA B operand straight from global memory in the packed weights'
// k order; RMSNorm rides along as per-token sums of squares and a final
// 1/rms scale; INT8 weights carry per-row scales applied to the tile.
//
// Replaces CudaMLP::forward / forward_add_residual (mlp_cuda.cu:295-337,
// with the residual added), launch_cutlass_gemv_fused_silu
// (cutlass_gemm_wrapper.cuh:141-200, 240-263) and the post-norm + MLP +
// residual chain of CudaLayer::forward (cuda_engine.cu:119-124).
#include "qw_stream.hpp"

namespace qwk {

constexpr int MLP_NW = 16;     // waves per workgroup
constexpr int MLP_DG = 2;      // down tiles per down workgroup (MLP_NW / MLP_DG waves each)
constexpr int MLP_NWD = MLP_NW / MLP_DG;
// Counters (self-resetting): gate/up completions are spread over MLP_SLOTS
// slots and the down workgroups' exits over MLP_EXIT_SLOTS slots plus one
// top counter, each on its own 256-byte line, so that no single address
// takes hundreds of atomics at once (they serialize at the coherence point).
constexpr int MLP_SLOTS = 32, MLP_EXIT_SLOTS = 8, MLP_SLOT_STRIDE = 64;
// out-projection tiles done (qw_layer_tail), after the exit slots and the top counter
constexpr int MLP_PRE_SLOTS = 8, MLP_PRE_BASE = (MLP_SLOTS + MLP_EXIT_SLOTS + 1) * MLP_SLOT_STRIDE;
// FP32 activations (the engine's residual stream) are staged into LDS as
// hi + lo planes of the MFMA input type, for up to this many tokens
constexpr int MLP_F32_MAX_M = 4, MLP_MAX_K = 1024;
constexpr int MLP_F32_LDS = (MLP_F32_MAX_M + 1) * (MLP_MAX_K + 8) * 2 * 2;

int mlp_fused_max_m(int xdt) { return xdt == DT_F32 ? MLP_F32_MAX_M : 16; }

// k-steps per wave: gate/up (K = H, 16 waves) and down (K = I, 8 waves per
// tile) at the Qwen3.5-0.8B shape (H = 1024, I = 3584); smaller shapes
// leave slots empty
template <int WF> struct MlpUnits;
template <> struct MlpUnits<WF_BF16> { static constexpr int UA = 2, UB = 14; };
template <> struct MlpUnits<WF_I8> { static constexpr int UA = 1, UB = 7; };

int mlp_counter_words() { return MLP_PRE_BASE + MLP_PRE_SLOTS * MLP_SLOT_STRIDE; }

// the out-projection ahead of the block: one 16-row tile over the whole K per
// workgroup, K cut in sixteen by wave
template <int WF> struct MlpPreUnits { static constexpr int U = 2 * MlpUnits<WF>::UA; };
int mlp_pre_max_ksteps(int wf) {
    if (wf == WF_BF16) return MLP_NW * MlpPreUnits<WF_BF16>::U;
    if (wf == WF_I8) return MLP_NW * MlpPreUnits<WF_I8>::U;
    return 0;
}

int mlp_fused_max_ksteps(int wf, bool down) {
    if (wf == WF_BF16) return down ? MLP_NWD * MlpUnits<WF_BF16>::UB : MLP_NW * MlpUnits<WF_BF16>::UA;
    if (wf == WF_I8) return down ? MLP_NWD * MlpUnits<WF_I8>::UB : MLP_NW * MlpUnits<WF_I8>::UA;
    return 0;
}

// 16-bit activation fragment loads of U k-steps with cache policy AUX
template <int WF, int XDT, int U, int AUX>
__device__ __forceinline__ void load_frags(__amdgpu_buffer_rsrc_t xr, uint32_t xrow, int kb, int n,
                                           XFrag<WF, XDT, 1> (&X)[U]) {
    constexpr int KE = WTraits<WF>::KE;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t xo = u < n ? xrow + (uint32_t)(kb + u) * 4u * KE * 2u : OOB;
#pragma unroll
        for (int h = 0; h < XFrag<WF, XDT, 1>::N16; ++h)
            X[u].v[0][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 16 * h, 0, AUX));
    }
}

// Sum the F tiles (and per-token sums of squares) of each run of GW waves
// in LDS in a fixed order; the first wave of the run gets the result.
template <int NW, int GW, int F, bool SS>
__device__ __forceinline__ void reduce_runs(f32x4 (&red)[NW][2][64], float (&red_ss)[NW][16], f32x4 (&acc)[F],
                                            float& ss, int wave_id, int lane) {
    const int r = lane & 15, g = lane >> 4;
    if constexpr (SS) {
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (g == 0) red_ss[wave_id][r] = ss;
    }
#pragma unroll
    for (int f = 0; f < F; ++f) red[wave_id][f][lane] = acc[f];
    __syncthreads();
    if (wave_id % GW == 0) {
#pragma unroll
        for (int f = 0; f < F; ++f) {
            f32x4 s = red[wave_id][f][lane];
#pragma unroll
            for (int w = 1; w < GW; ++w) s += red[wave_id + w][f][lane];
            acc[f] = s;
        }
        if constexpr (SS) {
            float t = red_ss[wave_id][r];
#pragma unroll
            for (int w = 1; w < GW; ++w) t += red_ss[wave_id + w][r];
            ss = t;
        }
    }
}

// Out-projection tile t of qw_layer_tail (a gate/up workgroup, before its own
// work): x_mid rows [16t, 16t+16) = x + W_o . core, FP32, K (the core width)
// cut in sixteen by wave and reduced in a fixed order, the residual added as
// the separate projection's epilogue adds it.  Wave 0 stores the rows with
// device-coherent stores, waits for them and counts the tile done.
template <int WF>
__device__ __forceinline__ void mlp_pre_tile(const MlpArgs& p, int t, int wave_id, int lane, f32x4 (&red)[MLP_NW][2][64],
                                             float (&red_ss)[MLP_NW][16]) {
    constexpr int U = MlpPreUnits<WF>::U;
    constexpr int KE = WTraits<WF>::KE;
    const SkinnyArgs& o = p.pre;
    const int r = lane & 15, g = lane >> 4;
    int kb, kend;
    wave_range<MLP_NW>(0, o.ksteps, wave_id, kb, kend);
    const int n = kend - kb;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(o.w, (uint32_t)((uint64_t)o.n_groups * o.ksteps * 1024u));
    const __amdgpu_buffer_rsrc_t cr = make_rsrc(o.x, (uint32_t)((uint64_t)o.M * o.ldx * 2u));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(o.scales ? (const void*)o.scales : o.x, o.scales ? (uint32_t)o.n_groups * 64u : 0u);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(o.res, (uint32_t)((uint64_t)o.M * o.ld_res * 4u));
    const uint32_t crow = r < o.M ? (uint32_t)(r * o.ldx + g * KE) * 2u : OOB;
    // the core fragments (small, needed first), the weights, the scales and the residual rows
    XFrag<WF, DT_BF16, 1> X[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t xo[1] = {u < n ? crow + (uint32_t)(kb + u) * 4u * KE * 2u : OOB};
        load_xfrag<WF, DT_BF16, 1, false>(cr, cr, xo, OOB, X[u]);
    }
    u32x4 A[U][1];
    issue_weights<1, U>(o, wrs, t, kb, n, lane, A);
    u32x4 sc = u32x4{0u, 0u, 0u, 0u};
    if constexpr (WF == WF_I8)
        sc = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, (uint32_t)((t * 16 + g * 4) * 4), 0, 0));
    const int ro = t * 16 + g * 4;
    const bool mine = r < o.M && ro < o.N;
    const u32x4 xin = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, mine ? (uint32_t)(r * o.ld_res + ro) * 4u : OOB, 0, 0));
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const BOps<WF, DT_BF16> b = make_bops<WF, DT_BF16, 1, false, false>(X[u], 0, ss);
        acc[0] = unit_mfma<WF, DT_BF16>(A[u][0], b, acc[0]);
    }
    reduce_runs<MLP_NW, MLP_NW, 1, false>(red, red_ss, acc, ss, wave_id, lane);
    if (wave_id == 0) {
        f32x4 v = acc[0];
        if constexpr (WF == WF_I8) v *= as_f32x4(sc);
        v += as_f32x4(xin);
        if (mine) {
            unsigned* dst = reinterpret_cast<unsigned*>(p.xmid + (int64_t)r * o.ldy + ro);
#pragma unroll
            for (int i = 0; i < 4; ++i) __hip_atomic_store(dst + i, __float_as_uint(v[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0)
            __hip_atomic_fetch_add(&p.cnt[MLP_PRE_BASE + (t % MLP_PRE_SLOTS) * MLP_SLOT_STRIDE], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Bounded wait (wave 0, then the workgroup) until every out-projection tile is done.
__device__ __forceinline__ void mlp_pre_wait(const MlpArgs& p, int wave_id, int lane) {
    if (wave_id == 0) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
            unsigned v = lane < MLP_PRE_SLOTS ? __hip_atomic_load(&p.cnt[MLP_PRE_BASE + lane * MLP_SLOT_STRIDE],
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                              : 0u;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
            if (v >= (unsigned)p.pre.n_groups) break;
            __builtin_amdgcn_s_sleep(1);
            if (__builtin_amdgcn_s_memrealtime() - t0 > 20000000ull) {
                if (lane == 0) __hip_atomic_store(&p.ctl[3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

// WF: weight format (gate/up and down share it); XDT: dtype of x (16-bit
// read straight into registers, FP32 staged through LDS).
// The intermediate h is held in the MFMA input type of WF (BF16, or F16 for
// INT8 weights), which is what the down projection consumes.
// PRE (FP32 x only): the out-projection of qw_layer_tail runs first (gate/up
// workgroups [0, pre.n_groups) take one tile each), and the block reads x_mid.
template <int WF, int XDT, bool NORM, bool GAM, bool PRE>
__global__ __launch_bounds__(MLP_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void mlp_kernel(MlpArgs p) {
    static_assert(!PRE || XDT == DT_F32, "the out-projection stage feeds the FP32 staging");
    const int n_dwg = (p.n_down + MLP_DG - 1) / MLP_DG;
    constexpr int NW = MLP_NW;
    constexpr int KE = WTraits<WF>::KE;
    constexpr int UA = MlpUnits<WF>::UA, UB = MlpUnits<WF>::UB;
    constexpr int HDT = WF == WF_BF16 ? DT_BF16 : DT_F16;
    __shared__ f32x4 red[NW][2][64];
    __shared__ float red_ss[NW][16];
    __shared__ __attribute__((aligned(16))) uint8_t xs_f32[XDT == DT_F32 ? MLP_F32_LDS : 16];
    __shared__ float ss_tok[16];
    __shared__ float ss_scratch[XDT == DT_F32 ? MLP_NW * 16 : 1];

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int bid = blockIdx.x;

    if (bid >= n_dwg) {
        // ---------------- gate/up tile pair grp: x -> h ----------------
        const SkinnyArgs& a = p.up;
        const int grp = bid - n_dwg;
        int kb, kend;
        wave_range<NW>(0, a.ksteps, wave_id, kb, kend);
        const int n = kend - kb;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * 2 * a.ksteps * 1024u));
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(GAM ? (const void*)a.gamma : a.x, GAM ? (uint32_t)a.K * 4u : 0u);
        const __amdgpu_buffer_rsrc_t sr =
            make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)a.n_groups * 2 * 64u : 0u);
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        float ss = 0.0f;
        u32x4 sc[2];  // per-row scales (INT8 weights only)
        u32x4 A[UA][2];
        auto issue_rest = [&]() {
            issue_weights<2, UA>(a, wrs, grp, kb, n, lane, A);
            if constexpr (WF == WF_I8) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    sc[rt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                           sr, (uint32_t)(((grp * 2 + rt) * 16 + g * 4) * 4), 0, 0));
            }
        };
        if constexpr (XDT == DT_F32) {
            // x (times 1 + gamma) staged into LDS as hi + lo planes; the weight
            // loads are issued between the staging's loads and its LDS writes.
            // PRE: the out-projection tile first (if this workgroup has one),
            // then the weights, the wait for every tile, and x_mid staged with
            // device-coherent loads (written in this launch)
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(PRE ? (const void*)p.xmid : a.x, (uint32_t)((uint64_t)a.M * a.ldx * 4u));
            const int kr = a.K;
            if constexpr (PRE) {
                if (grp < p.pre.n_groups) mlp_pre_tile<WF>(p, grp, wave_id, lane, red, red_ss);
                issue_rest();
                mlp_pre_wait(p, wave_id, lane);
            }
            auto stage = [&](auto sq_tag) {
                constexpr int SQ = decltype(sq_tag)::value;
                constexpr int XA = PRE ? AUX_SC1 : 0;
                XStage<XDT, SQ> st;
                stage_issue<WF, XDT, NW, SQ, NORM, XA>(a, xr, gr, 0, kr, st);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (!PRE) issue_rest();
                __builtin_amdgcn_sched_barrier(0);
                stage_finish<WF, XDT, 1, NW, SQ, NORM, XA>(a, xr, gr, 0, kr, st, xs_f32, ss_tok, ss_scratch);
            };
            const int rp = 1 << (32 - __builtin_clz((unsigned)a.M));
            const int cpt = ((kr / 8) * rp + NW * 64 - 1) / (NW * 64);
            if (cpt <= 1) stage(std::integral_constant<int, 1>{});
            else stage(std::integral_constant<int, 2>{});
            __syncthreads();
            constexpr int OS = OpSize<WF>::v;
            const int ls = lds_row_elems<WF>(kr);
            const int plane_bytes = (a.M + 1) * ls * OS;
            const int xrow = min(r, a.M);  // row M of the staging is zero
#pragma unroll
            for (int u = 0; u < UA; ++u) {
                BOps<WF, XDT> b;
                const int relk = (kb + u) * 4 * KE + g * KE;
                read_bops<WF, XDT>(b, xs_f32 + ((int64_t)xrow * ls + relk) * OS, plane_bytes);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) acc[rt] = unit_mfma<WF, XDT>(A[u][rt], b, acc[rt]);
            }
            if (NORM && r < 16) ss = ss_tok[r];
        } else {
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2u));
            const uint32_t xrow = r < a.M ? (uint32_t)(r * a.ldx + g * KE) * 2u : OOB;
            const uint32_t grow = r < a.M ? (uint32_t)(g * KE) * 4u : OOB;
            // activations (small, needed first), then the weights, then the scales
            XFrag<WF, XDT, 1> X[UA];
#pragma unroll
            for (int u = 0; u < UA; ++u) {
                const uint32_t ko = (uint32_t)(kb + u) * 4u * KE;
                const uint32_t xo[1] = {u < n ? xrow + ko * 2u : OOB};
                load_xfrag<WF, XDT, 1, GAM>(xr, gr, xo, u < n ? grow + ko * 4u : OOB, X[u]);
            }
            __builtin_amdgcn_sched_barrier(0);
            issue_rest();
            __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first wait
#pragma unroll
            for (int u = 0; u < UA; ++u) {
                const BOps<WF, XDT> b = make_bops<WF, XDT, 1, NORM, GAM>(X[u], 0, ss);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) acc[rt] = unit_mfma<WF, XDT>(A[u][rt], b, acc[rt]);
            }
        }
        reduce_runs<NW, NW, 2, NORM && XDT != DT_F32>(red, red_ss, acc, ss, wave_id, lane);
        if (wave_id == 0) {
            const float inv = NORM ? 1.0f / sqrtf(ss / (float)a.K + a.eps) : 1.0f;
            f32x4 gt = acc[0] * inv, up = acc[1] * inv;
            if constexpr (WF == WF_I8) {
                gt *= as_f32x4(sc[0]);
                up *= as_f32x4(sc[1]);
            }
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
            const int o = grp * 16 + g * 4;
            if (r < a.M && o < a.N) {
                // device-coherent stores of h (read by the down workgroups of this launch)
                uint32_t* dst = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned short*>(a.y) + (int64_t)r * a.ldy + o);
                const uint32_t w0 = op_bits<WF>(v[0]) | (op_bits<WF>(v[1]) << 16);
                const uint32_t w1 = op_bits<WF>(v[2]) | (op_bits<WF>(v[3]) << 16);
                __hip_atomic_store(dst, w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(dst + 1, w1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (lane == 0)
                __hip_atomic_fetch_add(&p.cnt[(grp % MLP_SLOTS) * MLP_SLOT_STRIDE], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        // ---------------- down tile j: h -> y (+ residual) ----------------
        const SkinnyArgs& a = p.down;
        const int j = bid * MLP_DG + wave_id / MLP_NWD;  // this wave's down tile
        const bool has_tile = j < p.n_down;
        int kb, kend;
        wave_range<MLP_NWD>(0, a.ksteps, wave_id % MLP_NWD, kb, kend);
        const int n = has_tile ? kend - kb : 0;
        const bool want_res = (a.flags & EP_RESIDUAL) != 0;
        const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * a.ksteps * 1024u));
        const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2u));
        const __amdgpu_buffer_rsrc_t sr =
            make_rsrc(a.scales ? (const void*)a.scales : a.x, a.scales ? (uint32_t)a.n_groups * 64u : 0u);
        const int res_size = a.res_dt == DT_F32 ? 4 : 2;
        const __amdgpu_buffer_rsrc_t rr =
            make_rsrc(want_res ? a.res : a.x, want_res ? (uint32_t)((uint64_t)a.M * a.ld_res * res_size) : 0u);
        // every weight k-step of this wave, and the epilogue operands: none depends on h
        u32x4 A[UB][1];
        issue_weights<1, UB>(a, wrs, j, kb, n, lane, A);
        u32x4 sc;  // per-row scales (INT8 weights only)
        if constexpr (WF == WF_I8)
            sc = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, (uint32_t)((j * 16 + g * 4) * 4), 0, 0));
        // the residual of this lane's 4 rows (issued empty without a residual)
        const int ro = j * 16 + g * 4;
        const bool res_ok = want_res && a.vec_store && has_tile && r < a.M && ro < a.N;
        const uint32_t ri = (uint32_t)((int64_t)r * a.ld_res + ro);
        const bool res32 = a.res_dt == DT_F32;
        // PRE: the residual is x_mid, written in this launch: loaded after the wait
        u32x4 rv32 = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, res_ok && res32 && !PRE ? ri * 4 : OOB, 0, 0));
        const u32x2 rv16 = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rr, res_ok && !res32 ? ri * 2 : OOB, 0, 0));
        __builtin_amdgcn_sched_barrier(0);
        // wait for every gate/up tile pair (bounded): wave 0 sums the done slots
        if (wave_id == 0) {
            // s_memrealtime counts at a constant 100 MHz: 20M ticks = 0.2 s
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                unsigned v = lane < MLP_SLOTS
                                 ? __hip_atomic_load(&p.cnt[lane * MLP_SLOT_STRIDE], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : 0u;
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
                if (v >= (unsigned)p.n_up) break;
                __builtin_amdgcn_s_sleep(1);
                if (__builtin_amdgcn_s_memrealtime() - t0 > 20000000ull) {
                    if (lane == 0) __hip_atomic_store(&p.ctl[3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        __syncthreads();
        if constexpr (PRE)
            rv32 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, res_ok && res32 ? ri * 4 : OOB, 0, AUX_SC1));
        const uint32_t xrow = r < a.M ? (uint32_t)(r * a.ldx + g * KE) * 2u : OOB;
        XFrag<WF, HDT, 1> X[UB];
        load_frags<WF, HDT, UB, AUX_SC1>(hr, xrow, kb, n, X);
        __builtin_amdgcn_sched_barrier(0);  // all h fragments in flight before the first MFMA
        f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            // h bits pass straight through as the B operand (its type is the MFMA input type)
            const BOps<WF, HDT> b = make_bops<WF, HDT, 1, false, false>(X[u], 0, ss);
            acc[0] = unit_mfma<WF, HDT>(A[u][0], b, acc[0]);
        }
        reduce_runs<NW, MLP_NWD, 1, false>(red, red_ss, acc, ss, wave_id, lane);
        if (wave_id % MLP_NWD == 0 && has_tile) {
            f32x4 v = acc[0];
            if constexpr (WF == WF_I8) v *= as_f32x4(sc);
            const int o = ro;
            if (r < a.M && o < a.N) {
                if (a.vec_store) {
                    if (want_res) v += epi_res(a.res_dt, rv32, rv16);
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
        // leave: two-level count of the down workgroups; the last one out
        // (every wait has ended) returns all slots to zero for the next launch
        if (threadIdx.x == 0) {
            const int s = bid % MLP_EXIT_SLOTS;
            const unsigned per = (unsigned)((n_dwg - s + MLP_EXIT_SLOTS - 1) / MLP_EXIT_SLOTS);
            const unsigned used = (unsigned)min(MLP_EXIT_SLOTS, n_dwg);
            unsigned* ex = p.cnt + MLP_SLOTS * MLP_SLOT_STRIDE;
            const unsigned old = __hip_atomic_fetch_add(&ex[s * MLP_SLOT_STRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == per - 1) {
                unsigned* top = ex + MLP_EXIT_SLOTS * MLP_SLOT_STRIDE;
                const unsigned o2 = __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (o2 == used - 1) {
                    for (int q = 0; q < MLP_SLOTS; ++q)
                        __hip_atomic_store(&p.cnt[q * MLP_SLOT_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    for (int q = 0; q < MLP_EXIT_SLOTS; ++q)
                        __hip_atomic_store(&ex[q * MLP_SLOT_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if constexpr (PRE) {
                        for (int q = 0; q < MLP_PRE_SLOTS; ++q)
                            __hip_atomic_store(&p.cnt[MLP_PRE_BASE + q * MLP_SLOT_STRIDE], 0u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    }
                    __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

template <int WF, int XDT, bool PRE = false>
static hipError_t launch_mlp2(const MlpArgs& p, bool norm, bool gam, hipStream_t st) {
    const dim3 grid((p.n_down + MLP_DG - 1) / MLP_DG + p.n_up), block(MLP_NW * 64);
    if (norm && gam) hipLaunchKernelGGL((mlp_kernel<WF, XDT, true, true, PRE>), grid, block, 0, st, p);
    else if (norm) hipLaunchKernelGGL((mlp_kernel<WF, XDT, true, false, PRE>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((mlp_kernel<WF, XDT, false, false, PRE>), grid, block, 0, st, p);
    return hipGetLastError();
}

hipError_t launch_mlp_fused(const MlpArgs& p, int wf, int xdt, hipStream_t stream) {
    if (p.up.M < 1 || p.up.M > mlp_fused_max_m(xdt) || p.up.K > MLP_MAX_K) return hipErrorInvalidValue;
    if (p.up.ksteps > mlp_fused_max_ksteps(wf, false) || p.down.ksteps > mlp_fused_max_ksteps(wf, true))
        return hipErrorInvalidValue;
    const bool norm = (p.up.flags & EP_NORM) != 0;
    const bool gam = norm && p.up.gamma != nullptr;
    if (p.pre.w) {
        // the out-projection stage: FP32 x, BF16 core, one tile per gate/up workgroup
        if (xdt != DT_F32 || !p.xmid || p.pre.n_groups > p.n_up || p.pre.ksteps > mlp_pre_max_ksteps(wf) ||
            p.pre.M != p.up.M || p.pre.N != p.up.K || p.up.x != p.pre.res || p.down.res != p.xmid ||
            p.pre.ldy != p.up.ldx || p.pre.ld_res != p.up.ldx)
            return hipErrorInvalidValue;
        if (wf == WF_BF16) return launch_mlp2<WF_BF16, DT_F32, true>(p, norm, gam, stream);
        if (wf == WF_I8) return launch_mlp2<WF_I8, DT_F32, true>(p, norm, gam, stream);
        return hipErrorInvalidValue;
    }
    if (wf == WF_BF16 && xdt == DT_BF16) return launch_mlp2<WF_BF16, DT_BF16>(p, norm, gam, stream);
    if (wf == WF_I8 && xdt == DT_F16) return launch_mlp2<WF_I8, DT_F16>(p, norm, gam, stream);
    if (wf == WF_I8 && xdt == DT_BF16) return launch_mlp2<WF_I8, DT_BF16>(p, norm, gam, stream);
    if (wf == WF_BF16 && xdt == DT_F32) return launch_mlp2<WF_BF16, DT_F32>(p, norm, gam, stream);
    if (wf == WF_I8 && xdt == DT_F32) return launch_mlp2<WF_I8, DT_F32>(p, norm, gam, stream);
    return hipErrorInvalidValue;
}

}  // namespace qwk
