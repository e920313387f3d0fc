// qw_skinny.hip -- small-M projection kernel for gfx950 (decode GEMV / skinny GEMM,
// tied lm_head with fused greedy argmax).
//
// Work decomposition.  The unit of work is one wave64 "item": a 16-row output
// tile (or a gate/up tile pair for GLU weights) over one slice of K.  Waves
// are independent: a wave streams its weight k-steps straight from HBM into
// MFMA A registers (1 KB fully coalesced non-temporal loads, see
// qw_device.hpp), reads the matching activation fragment (L2 resident) as the
// B operand, and accumulates 16 rows x 16 tokens per MFMA.  M <= 16 uses one
// token column tile (CT=1), M <= 32 two.  When a tile has fewer rows than the
// chip has waves to fill, K is split S ways; each split wave writes its FP32
// partial tile to the workspace and the last of the S waves to arrive (an
// agent-scope counter) sums the S partials in split order -- deterministic --
// and runs the epilogue.  Counters are returned to zero by that wave, so the
// kernel needs no memset and is safe to capture in a graph.
//
// Epilogue: per-row INT8 scale, RMSNorm of x (gamma folded into the B operand,
// 1/rms applied to the accumulator), SiLU(gate)*up for GLU pairs, residual
// add, Q/gate de-interleave, or -- for the lm_head -- a running (logit, index)
// maximum per token that is merged across the grid with 64-bit atomic max on
// an orderable key (ties resolve to the lowest index) and decoded by the last
// wave of the grid.
//
// Reference operators replaced: cutlass_style_gemv_kernel / _bf16 /
// _fused_silu (cutlass_gemm_wrapper.cuh:41-200), int8_gemv_batch_kernel
// (mlp_cuda.cu:158-180), lm_head_gemv_kernel_optimized (lm_head_cuda.cu:38-99)
// + block_argmax_kernel (gpu_sampler_argmax.cu:14-43), and the thread-per-row
// projection kernels of the attention operators.
#include "qw_device.hpp"
#include "qw_kernels.hpp"

namespace qwk {

constexpr unsigned EP_RESIDUAL = 1u, EP_NORM = 2u, EP_SPLIT = 4u;

template <int XDT> struct XSize { static constexpr int v = (XDT == DT_F32) ? 4 : 2; };

// Raw activation bits of one lane for one k-step unit (KE elements).
template <int XDT, int KE> struct XRaw {
    static constexpr int BYTES = KE * XSize<XDT>::v;
    static constexpr int NW = BYTES / 4;
    uint32_t w[NW];
};

template <int XDT, int KE>
__device__ __forceinline__ void load_xraw(XRaw<XDT, KE>& r, const uint8_t* p) {
    constexpr int B = XRaw<XDT, KE>::BYTES;
    if constexpr (B >= 16) {
#pragma unroll
        for (int i = 0; i < B / 16; ++i) {
            u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
            r.w[4 * i + 0] = v[0]; r.w[4 * i + 1] = v[1];
            r.w[4 * i + 2] = v[2]; r.w[4 * i + 3] = v[3];
        }
    } else {
        u32x2 v = *reinterpret_cast<const u32x2*>(p);
        r.w[0] = v[0]; r.w[1] = v[1];
    }
}

template <int XDT, int KE>
__device__ __forceinline__ void zero_xraw(XRaw<XDT, KE>& r) {
#pragma unroll
    for (int i = 0; i < XRaw<XDT, KE>::NW; ++i) r.w[i] = 0u;
}

template <int XDT, int KE>
__device__ __forceinline__ float xraw_elem(const XRaw<XDT, KE>& r, int e) {
    if constexpr (XDT == DT_F32) {
        return __uint_as_float(r.w[e]);
    } else {
        uint32_t h = (r.w[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        return XDT == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    }
}

// Whether x needs a hi/lo split to keep its precision through the MFMA input type.
template <int WF, int XDT> struct XSplit {
    static constexpr bool v = (WF == WF_BF16 && XDT != DT_BF16) || (WF == WF_I8 && XDT == DT_F32);
};
// Whether the raw x bits already are the MFMA input type.
template <int WF, int XDT> struct XDirect {
    static constexpr bool v = (WF == WF_BF16 && XDT == DT_BF16) || (WF == WF_I8 && XDT == DT_F16);
};

// B operands of one unit for one token tile.
template <int WF, int XDT> struct BOps;
template <int XDT> struct BOps<WF_BF16, XDT> { bf16x8 hi, lo; };
template <int XDT> struct BOps<WF_I8, XDT> { f16x8 hi0, hi1, lo0, lo1; };
template <int XDT> struct BOps<WF_F32, XDT> { float v[4]; };

template <int WF, int XDT, int KE>
__device__ __forceinline__ void make_bops(BOps<WF, XDT>& b, const XRaw<XDT, KE>& r, bool norm,
                                          const float* gam) {
    if constexpr (WF == WF_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float f = xraw_elem(r, e);
            b.v[e] = norm ? f * (1.0f + gam[e]) : f;
        }
    } else if constexpr (WF == WF_BF16) {
        if (XDirect<WF, XDT>::v && !norm) {
            u32x4 t = {r.w[0], r.w[1], r.w[2], r.w[3]};
            b.hi = __builtin_bit_cast(bf16x8, t);
            return;
        }
        u32x4 th, tl;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float f0 = xraw_elem(r, 2 * p), f1 = xraw_elem(r, 2 * p + 1);
            if (norm) { f0 *= 1.0f + gam[2 * p]; f1 *= 1.0f + gam[2 * p + 1]; }
            uint32_t h0 = f32_to_bf16_bits(f0), h1 = f32_to_bf16_bits(f1);
            th[p] = h0 | (h1 << 16);
            if constexpr (XSplit<WF, XDT>::v) {
                uint32_t l0 = f32_to_bf16_bits(f0 - bf16_bits_to_f32(h0));
                uint32_t l1 = f32_to_bf16_bits(f1 - bf16_bits_to_f32(h1));
                tl[p] = l0 | (l1 << 16);
            }
        }
        b.hi = __builtin_bit_cast(bf16x8, th);
        if constexpr (XSplit<WF, XDT>::v) b.lo = __builtin_bit_cast(bf16x8, tl);
    } else {  // WF_I8: f16 MFMA, 16 elements -> two operands
        if (XDirect<WF, XDT>::v && !norm) {
            u32x4 t0 = {r.w[0], r.w[1], r.w[2], r.w[3]};
            u32x4 t1 = {r.w[4], r.w[5], r.w[6], r.w[7]};
            b.hi0 = __builtin_bit_cast(f16x8, t0);
            b.hi1 = __builtin_bit_cast(f16x8, t1);
            return;
        }
        u32x4 th0, th1, tl0, tl1;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            float f0 = xraw_elem(r, 2 * p), f1 = xraw_elem(r, 2 * p + 1);
            if (norm) { f0 *= 1.0f + gam[2 * p]; f1 *= 1.0f + gam[2 * p + 1]; }
            uint32_t h0 = f32_to_f16_bits(f0), h1 = f32_to_f16_bits(f1);
            uint32_t hv = h0 | (h1 << 16);
            uint32_t lv = 0;
            if constexpr (XSplit<WF, XDT>::v) {
                uint32_t l0 = f32_to_f16_bits(f0 - f16_bits_to_f32(h0));
                uint32_t l1 = f32_to_f16_bits(f1 - f16_bits_to_f32(h1));
                lv = l0 | (l1 << 16);
            }
            if (p < 4) { th0[p] = hv; tl0[p] = lv; } else { th1[p - 4] = hv; tl1[p - 4] = lv; }
        }
        b.hi0 = __builtin_bit_cast(f16x8, th0);
        b.hi1 = __builtin_bit_cast(f16x8, th1);
        if constexpr (XSplit<WF, XDT>::v) {
            b.lo0 = __builtin_bit_cast(f16x8, tl0);
            b.lo1 = __builtin_bit_cast(f16x8, tl1);
        }
    }
}

// acc += A(unit) x B(unit)
template <int WF, int XDT>
__device__ __forceinline__ f32x4 unit_mfma(u32x4 a, const BOps<WF, XDT>& b, f32x4 acc) {
    if constexpr (WF == WF_BF16) {
        bf16x8 av = __builtin_bit_cast(bf16x8, a);
        acc = mfma_bf16(av, b.hi, acc);
        if constexpr (XSplit<WF, XDT>::v) acc = mfma_bf16(av, b.lo, acc);
    } else if constexpr (WF == WF_I8) {
        f16x8 a0, a1;
        i8unit_to_f16(a, a0, a1);
        acc = mfma_f16(a0, b.hi0, acc);
        acc = mfma_f16(a1, b.hi1, acc);
        if constexpr (XSplit<WF, XDT>::v) {
            acc = mfma_f16(a0, b.lo0, acc);
            acc = mfma_f16(a1, b.lo1, acc);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = mfma_f32(__uint_as_float(a[e]), b.v[e], acc);
    }
    return acc;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // raw (untyped) buffer: stride 0, num_records = bytes; loads past the end return 0
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int AUX_NT = 2;  // non-temporal (streamed once)

template <int XDT, int KE>
__device__ __forceinline__ void buf_load_xraw(XRaw<XDT, KE>& r, __amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                              uint32_t soff) {
    constexpr int B = XRaw<XDT, KE>::BYTES;
    if constexpr (B >= 16) {
#pragma unroll
        for (int i = 0; i < B / 16; ++i) {
            u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 * i, soff, 0));
            r.w[4 * i + 0] = v[0]; r.w[4 * i + 1] = v[1];
            r.w[4 * i + 2] = v[2]; r.w[4 * i + 3] = v[3];
        }
    } else {
        u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0));
        r.w[0] = v[0]; r.w[1] = v[1];
    }
}

// Per-item epilogue operands, loaded before the item's weights so that they
// never form a dependent memory round trip after the weight stream.
template <int RT, int CT>
struct EpiOps {
    f32x4 sc[RT];
    f32x4 res[CT];
};

template <int RT, int CT>
__device__ __forceinline__ void load_epi(const SkinnyArgs& a, int grp, int lane, bool want_res,
                                         EpiOps<RT, CT>& e) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        e.sc[rt] = a.scales ? *reinterpret_cast<const f32x4*>(a.scales + (int64_t)(grp * RT + rt) * 16 + g * 4)
                            : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        e.res[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int m = ct * 16 + r;
        const int o = grp * 16 + g * 4;
        if (want_res && m < a.M && o < a.N) {
            if (a.vec_store) {
                e.res[ct] = load_act4(a.res, a.res_dt, (int64_t)m * a.ld_res + o);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (o + i < a.N) e.res[ct][i] = load_act(a.res, a.res_dt, (int64_t)m * a.ld_res + o + i);
            }
        }
    }
}

// This wave's k sub-range [kb, kend) of an item: the item's K split is cut
// into NW contiguous pieces, one per wave of the workgroup.
template <int NW>
__device__ __forceinline__ void item_range(const SkinnyArgs& a, int item, int wave_id, int& kb, int& kend) {
    const int grp = item / a.S;
    const int s = item - grp * a.S;
    const int ks0 = (int)(((int64_t)s * a.ksteps) / a.S);
    const int ks1 = (int)(((int64_t)(s + 1) * a.ksteps) / a.S);
    const int cnt = ks1 - ks0;
    kb = ks0 + (wave_id * cnt) / NW;
    kend = ks0 + ((wave_id + 1) * cnt) / NW;
}

// Issue the loads of k-steps [kb, kb+n) (n <= U) of tile group grp.
template <int WF, int XDT, int CT, int RT, int U>
__device__ __forceinline__ void issue_chunk(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t wrs,
                                            __amdgpu_buffer_rsrc_t xrs, uint32_t xvoff[CT], int grp,
                                            int kb, int n, int lane, u32x4 (&A)[U][RT],
                                            XRaw<XDT, WTraits<WF>::KE> (&X)[U][CT]) {
    constexpr int KE = WTraits<WF>::KE;
    const uint32_t tile_bytes = (uint32_t)a.ksteps * 1024u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (u < n) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                A[u][rt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         wrs, lane * 16, (uint32_t)(grp * RT + rt) * tile_bytes + (uint32_t)(kb + u) * 1024u, AUX_NT));
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                buf_load_xraw<XDT, KE>(X[u][ct], xrs, xvoff[ct], (uint32_t)(kb + u) * (4 * KE) * XSize<XDT>::v);
        }
    }
}

// Work decomposition (see the file header): a workgroup of NW waves owns one
// item at a time -- a 16-row tile (two for GLU) over one K split -- and its
// waves take contiguous pieces of that split; partial tiles meet in LDS.
// Workgroups walk the items grid-stride, and the loads of the next item are
// issued before the current item's reduction and epilogue.  The RMSNorm
// statistics come from the activation fragments already in registers.
template <int WF, int XDT, int CT, bool GLU, bool ARGMAX, int NW>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(SkinnyArgs a) {
    constexpr int U = NW == 16 ? (WF == WF_I8 ? 2 : 4) : skinny_unroll(WF, XDT, CT, GLU);
    constexpr int KE = WTraits<WF>::KE;
    constexpr int RT = GLU ? 2 : 1;
    constexpr int F = RT * CT;
    using XR = XRaw<XDT, KE>;
    __shared__ f32x4 red[NW][F][64];
    __shared__ float ssred[NW][CT][64];
    extern __shared__ float gam_s[];  // K floats when the norm prologue is on

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const bool norm = (a.flags & EP_NORM) != 0;
    const bool want_res = !ARGMAX && (a.flags & EP_RESIDUAL);

    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_groups * RT * a.ksteps * 1024u));
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * XSize<XDT>::v));
    uint32_t xvoff[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)   // tokens >= M fall outside the buffer and read as 0
        xvoff[ct] = (uint32_t)(((ct * 16 + r) * a.ldx + g * KE) * XSize<XDT>::v);

    if (norm) {
        for (int i = threadIdx.x; i < a.K / 4; i += NW * 64)
            reinterpret_cast<f32x4*>(gam_s)[i] = reinterpret_cast<const f32x4*>(a.gamma)[i];
    }

    unsigned long long best[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) best[ct] = 0ull;

    u32x4 A[U][RT];
    XR X[U][CT];
    EpiOps<RT, CT> epi, epi_next;
    int kb = 0, kend = 0, n = 0;
    int item = blockIdx.x;
    if (item < a.n_items) {
        if (wave_id == 0) load_epi<RT, CT>(a, item / a.S, lane, want_res, epi);
        item_range<NW>(a, item, wave_id, kb, kend);
        n = min(U, kend - kb);
        issue_chunk<WF, XDT, CT, RT, U>(a, wrs, xrs, xvoff, item / a.S, kb, n, lane, A, X);
    }
    __syncthreads();  // gamma staged

    while (item < a.n_items) {
        f32x4 acc[RT][CT];
        float ss[CT];
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            ss[j] = 0.0f;
#pragma unroll
            for (int i = 0; i < RT; ++i) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        for (;;) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u < n) {
                    float gam[KE];
                    if (norm) {
                        const float* gp = gam_s + (kb + u) * (4 * KE) + g * KE;
#pragma unroll
                        for (int e = 0; e < KE; e += 4) {
                            f32x4 gv = *reinterpret_cast<const f32x4*>(gp + e);
                            gam[e] = gv[0]; gam[e + 1] = gv[1]; gam[e + 2] = gv[2]; gam[e + 3] = gv[3];
                        }
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                            for (int e = 0; e < KE; ++e) {
                                const float xv = xraw_elem(X[u][ct], e);
                                ss[ct] += xv * xv;
                            }
                    }
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        BOps<WF, XDT> b;
                        make_bops<WF, XDT, KE>(b, X[u][ct], norm, gam);
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = unit_mfma<WF, XDT>(A[u][rt], b, acc[rt][ct]);
                    }
                }
            }
            kb += n;
            if (kb >= kend) break;
            n = min(U, kend - kb);
            issue_chunk<WF, XDT, CT, RT, U>(a, wrs, xrs, xvoff, item / a.S, kb, n, lane, A, X);
        }
        const int cur = item;
        item += gridDim.x;
        if (item < a.n_items) {
            if (wave_id == 0) load_epi<RT, CT>(a, item / a.S, lane, want_res, epi_next);
            item_range<NW>(a, item, wave_id, kb, kend);
            n = min(U, kend - kb);
            issue_chunk<WF, XDT, CT, RT, U>(a, wrs, xrs, xvoff, item / a.S, kb, n, lane, A, X);
        }

        // ---- reduce the NW pieces in LDS (fixed order) ----
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) red[wave_id][rt * CT + ct][lane] = acc[rt][ct];
        if (norm) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) ssred[wave_id][ct][lane] = ss[ct];
        }
        __syncthreads();
        if (NW > 1) {
            for (int t = threadIdx.x; t < F * 64; t += NW * 64) {
                const int f = t >> 6, l = t & 63;
                f32x4 sum = red[0][f][l];
#pragma unroll
                for (int w = 1; w < NW; ++w) sum += red[w][f][l];
                red[0][f][l] = sum;
            }
            if (norm) {
                for (int t = threadIdx.x; t < CT * 64; t += NW * 64) {
                    const int c = t >> 6, l = t & 63;
                    float sum = ssred[0][c][l];
#pragma unroll
                    for (int w = 1; w < NW; ++w) sum += ssred[w][c][l];
                    ssred[0][c][l] = sum;
                }
            }
            __syncthreads();
        }
        if (wave_id != 0) continue;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = red[0][rt * CT + ct][lane];
        if (norm) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) ss[ct] = ssred[0][ct][lane];
        }
        EpiOps<RT, CT> e = epi;
        epi = epi_next;

        const int grp = cur / a.S;
        bool finish = true;
        if constexpr (!ARGMAX) {
            if (a.S > 1) {
                // Cross-workgroup split-K hand-off, no fence: the partial tile
                // (and the partial sum of squares) go out as agent-scope atomic
                // stores (written through to the device coherence point),
                // s_waitcnt vmcnt(0) waits for their completion, then the
                // agent-scope counter increment.  The last of the S workgroups
                // reads the S partials back with agent-scope atomic loads, in
                // split order (deterministic), and returns the counter to 0.
                const int s = cur - grp * a.S;
                constexpr int REC = F * 4 + CT;  // floats per lane per split
                float* P = reinterpret_cast<float*>(a.partials) + ((int64_t)grp * a.S * 64 + lane) * REC;
                float* mine = P + (int64_t)s * 64 * REC;
#pragma unroll
                for (int f = 0; f < F; ++f)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        __hip_atomic_store(mine + f * 4 + i, acc[f / CT][f % CT][i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                if (norm) {
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct)
                        __hip_atomic_store(mine + F * 4 + ct, ss[ct], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                unsigned old = 0;
                if (lane == 0)
                    old = __hip_atomic_fetch_add(&a.counters[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
                        if (norm) {
#pragma unroll
                            for (int ct = 0; ct < CT; ++ct)
                                ss[ct] += __hip_atomic_load(q + F * 4 + ct, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                    if (lane == 0)
                        __hip_atomic_store(&a.counters[grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (!finish) continue;

        float inv[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            inv[ct] = 1.0f;
            if (norm) {
                float t = ss[ct];
                t += __shfl_xor(t, 16);
                t += __shfl_xor(t, 32);
                inv[ct] = 1.0f / sqrtf(t / (float)a.K + a.eps);
            }
        }

        // ---- epilogue (wave 0) ----
        const int o = grp * 16 + g * 4;  // first of this lane's 4 logical rows
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int m = ct * 16 + r;
            f32x4 v;
            if constexpr (GLU) {
                f32x4 gt = acc[0][ct] * e.sc[0] * inv[ct];
                f32x4 up = acc[1][ct] * e.sc[1] * inv[ct];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
            } else {
                v = acc[0][ct] * e.sc[0] * inv[ct];
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
                if (want_res) v += e.res[ct];
                if (a.vec_store) {
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
                        void* dst = a.y;
                        int col = oi;
                        if (a.flags & EP_SPLIT) {
                            const int blk = oi / a.split_period;
                            dst = (blk & 1) ? a.y2 : a.y;
                            col = (blk >> 1) * a.split_period + (oi - blk * a.split_period);
                        }
                        store_act(dst, a.ydt, (int64_t)m * a.ldy + col, v[i]);
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
            for (int m = lane; m < a.M; m += 64) {
                unsigned long long kk = __hip_atomic_exchange(&a.keys[m], 0ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
                a.ids[m] = (int32_t)key_index(kk);
                if (a.maxv) a.maxv[m] = key_value(kk);
            }
            if (lane == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int WF, int XDT, int CT, int NW>
static hipError_t launch4(const SkinnyArgs& a, bool glu, bool argmax, int grid, hipStream_t st) {
    const size_t smem = (a.flags & EP_NORM) ? (size_t)a.K * sizeof(float) : 0;
    if (argmax) {
        if (glu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, false, true, NW>), dim3(grid), dim3(NW * 64), smem, st, a);
    } else if (glu) {
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, true, false, NW>), dim3(grid), dim3(NW * 64), smem, st, a);
    } else {
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, false, false, NW>), dim3(grid), dim3(NW * 64), smem, st, a);
    }
    return hipGetLastError();
}

template <int WF, int XDT, int CT>
static hipError_t launch3(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    // 16-wave workgroups serve plain (non-GLU) projections of up to 16
    // tokens whose activation already has the MFMA input type
    if constexpr (CT == 1 && ((WF == WF_BF16 && XDT == DT_BF16) || (WF == WF_I8 && XDT == DT_F16) ||
                              (WF == WF_F32 && XDT == DT_F32))) {
        if (nw == 16 && !glu && !argmax) {
            const size_t smem = (a.flags & EP_NORM) ? (size_t)a.K * sizeof(float) : 0;
            hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, false, false, 16>), dim3(grid), dim3(1024), smem, st, a);
            return hipGetLastError();
        }
    }
    return launch4<WF, XDT, CT, 4>(a, glu, argmax, grid, st);
}

template <int WF, int XDT>
static hipError_t launch2(const SkinnyArgs& a, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    if (a.M <= 16) return launch3<WF, XDT, 1>(a, glu, argmax, nw, grid, st);
    return launch3<WF, XDT, 2>(a, glu, argmax, nw, grid, st);
}

template <int WF>
static hipError_t launch1(const SkinnyArgs& a, int xdt, bool glu, bool argmax, int nw, int grid, hipStream_t st) {
    switch (xdt) {
        case DT_F32: return launch2<WF, DT_F32>(a, glu, argmax, nw, grid, st);
        case DT_BF16: return launch2<WF, DT_BF16>(a, glu, argmax, nw, grid, st);
        case DT_F16: return launch2<WF, DT_F16>(a, glu, argmax, nw, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_skinny(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int nw, int grid,
                         hipStream_t stream) {
    if (a.M < 1 || a.M > 32) return hipErrorInvalidValue;
    if (nw != 4 && nw != 16) return hipErrorInvalidValue;
    switch (wf) {
        case WF_F32: return launch1<WF_F32>(a, xdt, glu, argmax, nw, grid, stream);
        case WF_BF16: return launch1<WF_BF16>(a, xdt, glu, argmax, nw, grid, stream);
        case WF_I8: return launch1<WF_I8>(a, xdt, glu, argmax, nw, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qwk
