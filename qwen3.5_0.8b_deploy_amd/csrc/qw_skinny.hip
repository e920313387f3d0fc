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

// 1/sqrt(mean(x[m]^2)+eps) for the token of this lane (lane & 15 within
// token tile ct); all 64 lanes must call it.
template <int XDT>
__device__ __forceinline__ float lane_inv_rms(const SkinnyArgs& a, int m, int lane) {
    const int g = lane >> 4;
    const int kq = a.K >> 2;  // multiple of 16
    float ss = 0.0f;
    if (m < a.M) {
        const uint8_t* base = reinterpret_cast<const uint8_t*>(a.x) +
                              ((int64_t)m * a.ldx + (int64_t)g * kq) * XSize<XDT>::v;
        constexpr int EPV = 16 / XSize<XDT>::v;  // elements per 16 B
        for (int k = 0; k < kq; k += EPV) {
            u32x4 v = *reinterpret_cast<const u32x4*>(base + (int64_t)k * XSize<XDT>::v);
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                float f;
                if constexpr (XDT == DT_F32) f = __uint_as_float(v[e]);
                else {
                    uint32_t h = (v[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
                    f = XDT == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
                }
                ss += f * f;
            }
        }
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    return 1.0f / sqrtf(ss / (float)a.K + a.eps);
}

template <int WF, int XDT, int CT, bool GLU, bool ARGMAX>
__global__ __launch_bounds__(256) void skinny_kernel(SkinnyArgs a) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int RT = GLU ? 2 : 1;
    using XR = XRaw<XDT, KE>;
    constexpr int PER_UNIT_REGS = RT * 4 + CT * XR::NW;
    constexpr int U0 = 96 / PER_UNIT_REGS;
    constexpr int U = U0 < 2 ? 2 : (U0 > 8 ? 8 : U0);

    const int lane = threadIdx.x & 63;
    const int wave_id = threadIdx.x >> 6;
    const int total_waves = gridDim.x * 4;
    const int gw = blockIdx.x * 4 + wave_id;
    const int r = lane & 15;
    const int g = lane >> 4;
    const bool norm = (a.flags & EP_NORM) != 0;
    const int64_t tile_bytes = (int64_t)a.ksteps * 1024;

    float inv[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) inv[ct] = 1.0f;
    unsigned long long best[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) best[ct] = 0ull;
    if constexpr (ARGMAX) {
        if (norm) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) inv[ct] = lane_inv_rms<XDT>(a, ct * 16 + r, lane);
        }
    }

    for (int item = gw; item < a.n_items; item += total_waves) {
        const int grp = item / a.S;
        const int s = item - grp * a.S;
        const int ks0 = (int)(((int64_t)s * a.ksteps) / a.S);
        const int ks1 = (int)(((int64_t)(s + 1) * a.ksteps) / a.S);

        f32x4 acc[RT][CT];
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

        const uint8_t* wbase[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            wbase[rt] = a.w + (int64_t)(grp * RT + rt) * tile_bytes + lane * 16;

        for (int kb = ks0; kb < ks1; kb += U) {
            const int n = ks1 - kb;
            u32x4 A[U][RT];
            XR X[U][CT];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u < n) {
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        A[u][rt] = load_w16(wbase[rt] + (int64_t)(kb + u) * 1024);
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        const int m = ct * 16 + r;
                        if (m < a.M) {
                            const int64_t k = (int64_t)(kb + u) * (4 * KE) + g * KE;
                            load_xraw<XDT, KE>(X[u][ct], reinterpret_cast<const uint8_t*>(a.x) +
                                                             ((int64_t)m * a.ldx + k) * XSize<XDT>::v);
                        } else {
                            zero_xraw<XDT, KE>(X[u][ct]);
                        }
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u < n) {
                    float gam[KE];
                    if (norm) {
                        const float* gp = a.gamma + (int64_t)(kb + u) * (4 * KE) + g * KE;
#pragma unroll
                        for (int e = 0; e < KE; e += 4) {
                            f32x4 gv = *reinterpret_cast<const f32x4*>(gp + e);
                            gam[e] = gv[0]; gam[e + 1] = gv[1]; gam[e + 2] = gv[2]; gam[e + 3] = gv[3];
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
        }

        if constexpr (!ARGMAX) {
            if (a.S > 1) {
                float4* P = a.partials + (int64_t)grp * a.S * (RT * CT) * 64 + lane;
                float4* mine = P + (int64_t)s * (RT * CT) * 64;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        f32x4 v = acc[rt][ct];
                        mine[(rt * CT + ct) * 64] = make_float4(v[0], v[1], v[2], v[3]);
                    }
                __threadfence();
                unsigned old = 0;
                if (lane == 0) old = atomicAdd(&a.counters[grp], 1u);
                old = __shfl(old, 0);
                if (old != (unsigned)(a.S - 1)) continue;
                __threadfence();
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int s2 = 0; s2 < a.S; ++s2) {
                    const float4* q = P + (int64_t)s2 * (RT * CT) * 64;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct) {
                            float4 v = q[(rt * CT + ct) * 64];
                            acc[rt][ct] += f32x4{v.x, v.y, v.z, v.w};
                        }
                }
                if (lane == 0) atomicExch(&a.counters[grp], 0u);
            }
            if (norm) {
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) inv[ct] = lane_inv_rms<XDT>(a, ct * 16 + r, lane);
            }
        }

        // ---- epilogue ----
        const int o = grp * 16 + g * 4;  // first of this lane's 4 logical rows
        f32x4 sc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if (a.scales) {
                sc[rt] = *reinterpret_cast<const f32x4*>(a.scales + (int64_t)(grp * RT + rt) * 16 + g * 4);
            } else {
                sc[rt] = f32x4{1.f, 1.f, 1.f, 1.f};
            }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int m = ct * 16 + r;
            f32x4 v;
            if constexpr (GLU) {
                f32x4 gt = acc[0][ct] * sc[0] * inv[ct];
                f32x4 up = acc[1][ct] * sc[1] * inv[ct];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu_f(gt[i]) * up[i];
            } else {
                v = acc[0][ct] * sc[0] * inv[ct];
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
                    if (a.flags & EP_RESIDUAL) v += load_act4(a.res, a.res_dt, (int64_t)m * a.ld_res + o);
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
                        if (a.flags & EP_RESIDUAL) vi += load_act(a.res, a.res_dt, (int64_t)m * a.ld_res + oi);
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
        __threadfence();
        unsigned old = 0;
        if (lane == 0) old = atomicAdd(a.done, 1u);
        old = __shfl(old, 0);
        if (old == (unsigned)(total_waves - 1)) {
            __threadfence();
            for (int m = lane; m < a.M; m += 64) {
                unsigned long long kk = __hip_atomic_exchange(&a.keys[m], 0ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
                a.ids[m] = (int32_t)key_index(kk);
                if (a.maxv) a.maxv[m] = key_value(kk);
            }
            if (lane == 0) atomicExch(a.done, 0u);
        }
    }
}

template <int WF, int XDT, int CT>
static hipError_t launch3(const SkinnyArgs& a, bool glu, bool argmax, int grid, hipStream_t st) {
    if (argmax) {
        if (glu) return hipErrorInvalidValue;
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, false, true>), dim3(grid), dim3(256), 0, st, a);
    } else if (glu) {
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, true, false>), dim3(grid), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((skinny_kernel<WF, XDT, CT, false, false>), dim3(grid), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int WF, int XDT>
static hipError_t launch2(const SkinnyArgs& a, bool glu, bool argmax, int grid, hipStream_t st) {
    if (a.M <= 16) return launch3<WF, XDT, 1>(a, glu, argmax, grid, st);
    return launch3<WF, XDT, 2>(a, glu, argmax, grid, st);
}

template <int WF>
static hipError_t launch1(const SkinnyArgs& a, int xdt, bool glu, bool argmax, int grid, hipStream_t st) {
    switch (xdt) {
        case DT_F32: return launch2<WF, DT_F32>(a, glu, argmax, grid, st);
        case DT_BF16: return launch2<WF, DT_BF16>(a, glu, argmax, grid, st);
        case DT_F16: return launch2<WF, DT_F16>(a, glu, argmax, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_skinny(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int grid,
                         hipStream_t stream) {
    if (a.M < 1 || a.M > 32) return hipErrorInvalidValue;
    switch (wf) {
        case WF_F32: return launch1<WF_F32>(a, xdt, glu, argmax, grid, stream);
        case WF_BF16: return launch1<WF_BF16>(a, xdt, glu, argmax, grid, stream);
        case WF_I8: return launch1<WF_I8>(a, xdt, glu, argmax, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qwk
