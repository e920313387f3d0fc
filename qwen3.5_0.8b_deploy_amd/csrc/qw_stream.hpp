// qw_stream.hpp -- device building blocks of the weight-streaming kernels
// (qw_skinny.hip, qw_mlp.hip): activation staging into LDS in the MFMA input
// type, branch-free weight / epilogue-operand loads, and the MFMA step.
//
// Load discipline.  Vector-memory counters retire in issue order, so a
// consumer of a load waits for everything issued before it.  The kernels
// therefore issue the small loads (activations, gamma, scales, residual)
// first and the weight stream last, and issue every load unconditionally:
// an unwanted load gets an out-of-range VGPR offset (zeros, no traffic),
// which keeps the number of outstanding loads identical on every path so the
// compiler can wait for each load separately.
#pragma once

#include <type_traits>

#include "qw_device.hpp"
#include "qw_kernels.hpp"

namespace qwk {

constexpr unsigned EP_RESIDUAL = 1u, EP_NORM = 2u, EP_SPLIT = 4u;
constexpr int AUX_NT = 2;   // buffer-load cache policy: non-temporal (streamed once)
constexpr int AUX_SC1 = 16; // buffer-load cache policy: device-coherent (data written in this kernel)

template <int XDT> struct XSize { static constexpr int v = (XDT == DT_F32) ? 4 : 2; };

// MFMA input type of a weight format: bf16 for BF16 weights, f16 for INT8
// weights (exact for |q| <= 127), f32 for FP32 weights.
template <int WF> struct OpSize { static constexpr int v = WF == WF_F32 ? 4 : 2; };

// Whether the activation needs a hi + lo pair to keep its precision through a
// 16-bit MFMA input.
template <int WF, int XDT> struct XSplit {
    static constexpr bool v = (WF == WF_BF16 && XDT != DT_BF16) || (WF == WF_I8 && XDT == DT_F32);
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // raw (untyped) buffer: stride 0, num_records = bytes; loads past the end return 0
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations are outstanding, leaving the other counters alone
constexpr unsigned vm_wait(int n) { return 0x0F70u | ((unsigned)n & 15u) | (((unsigned)n >> 4) << 14); }

// One 1 KB unit global -> LDS (buffer_load_dwordx4 ... lds; M0 = LDS base of
// the unit, lane l lands at +16*l).  Written as inline assembly so that the
// compiler does not treat the asynchronous LDS write as a hazard for the
// later LDS reads and wait for every load in flight: the K-loop waits for
// exactly the stage it consumes (vector-memory counters retire in order)
// and a barrier publishes it.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds_unit, uint32_t voff) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds_unit;
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs)
                 : "memory", "m0");
}

// Epoch wrap of the persistent kernels' tagged hand-off words.  A word is
// (tag << 32 | payload) with the launch epoch in the tag's high bits; once
// the epoch's field wraps, a word written 2^bits launches earlier (a token
// slot unused since, when M varies) would carry the tag a consumer now waits
// for.  The launch at which the field wraps calls this first, with every
// thread of every workgroup: each workgroup zeroes its share of the words
// (tag 0 never matches a live tag), and a grid barrier on the monotonic
// counter `bar` (+gridDim.x per wrap, so it never needs a reset) keeps every
// producer's first store behind every clear.  All workgroups are resident
// (the callers' launch contract), so the barrier completes; the wait is
// bounded (0.2 s) and raises the error flag on expiry.  `flag` is an LDS word
// the caller initializes afterwards (it carries the outcome to every wave).
__device__ __forceinline__ void wrap_clear_words(uint64_t* words, size_t n, unsigned* bar, unsigned* err, unsigned* flag,
                                                 bool& dead) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        __hip_atomic_store(words + i, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (threadIdx.x == 0) {
        // release: this workgroup's clears are visible before its arrival
        const unsigned old = __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned target = (old / gridDim.x + 1u) * gridDim.x;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        unsigned d = 0u;
        while (__hip_atomic_load(bar, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > 20000000ull) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                d = 1u;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        *flag = d;
    }
    __syncthreads();
    if (*flag) dead = true;
    __syncthreads();
}

// ---------------------------------------------------------------------------
// LDS layout of the staged activations: nops planes (hi, lo) of (M + 1) rows
// of `ls` op-elements; row M is all zero and serves tokens >= M.  The row
// stride carries a 16-byte pad to spread the rows over the LDS banks.
// ---------------------------------------------------------------------------
template <int WF>
__device__ __forceinline__ int lds_row_elems(int kr) { return kr + 16 / OpSize<WF>::v; }

template <int WF>
__device__ __forceinline__ uint32_t op_bits(float f) {
    if constexpr (WF == WF_BF16) return f32_to_bf16_bits(f);
    else if constexpr (WF == WF_I8) return f32_to_f16_bits(f);
    else return __float_as_uint(f);
}
template <int WF>
__device__ __forceinline__ float op_value(uint32_t h) {
    if constexpr (WF == WF_BF16) return bf16_bits_to_f32(h);
    else if constexpr (WF == WF_I8) return f16_bits_to_f32(h);
    else return __uint_as_float(h);
}

// Activation staging, split in two so the small activation loads are issued
// BEFORE the weight stream (vector-memory counters retire in order: a load
// issued after the weights could only be consumed after all of them).
// Thread t owns row t % RP (RP = M+1 rounded up to a power of two) and the
// row's 8-element chunks j0, j0 + NT/RP, ...; the first SQ chunks are loaded
// by stage_issue, stage_finish converts them (times 1 + gamma), writes them
// to LDS and handles any further chunks.  Row M is all zero.
template <int XDT, int SQ>
struct XStage {
    static constexpr int XB = 8 * XSize<XDT>::v;  // bytes of one raw chunk
    u32x4 raw[SQ][XB / 16];
    f32x4 gam[SQ][2];
    int m, j0, tpr, nchunk;
    float ss;
};
template <int XDT> struct XChunk { static constexpr int XB = 8 * XSize<XDT>::v; };

// Buffer loads are range-checked on their VGPR offset only (the scalar
// offset is not part of the check); a VGPR offset with the top bit set is out
// of range and returns zeros without a memory access.  Loads that are not
// wanted are issued that way instead of being skipped, so every path issues
// the same number of loads and the compiler can wait for each one precisely.
constexpr uint32_t OOB = 0x80000000u;

template <int XDT, bool NORM, int XAUX = 0>
__device__ __forceinline__ void stage_load(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t gr,
                                           int k0, int c, int m, bool valid, u32x4 (&raw)[XChunk<XDT>::XB / 16],
                                           f32x4 (&gam)[2]) {
    constexpr int XB = XChunk<XDT>::XB;
    const uint32_t xo = valid && m < a.M ? (uint32_t)(((int64_t)m * a.ldx + k0 + c * 8) * XSize<XDT>::v) : OOB;
#pragma unroll
    for (int h = 0; h < XB / 16; ++h)
        raw[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 16 * h, 0, XAUX));
    if constexpr (NORM) {
        const uint32_t go = valid ? (uint32_t)((k0 + c * 8) * 4) : OOB;
        gam[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, go, 0, 0));
        gam[1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, go + 16, 0, 0));
    }
}

template <int WF, int XDT, int NW, int SQ, bool NORM, int XAUX = 0>
__device__ __forceinline__ void stage_issue(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t gr,
                                            int k0, int kr, XStage<XDT, SQ>& st) {
    constexpr int NT = NW * 64;
    const int rp = 1 << (32 - __builtin_clz((unsigned)a.M));  // M+1 rounded up to a power of 2 (<= 64)
    st.m = threadIdx.x & (rp - 1);
    st.tpr = NT / rp;
    st.j0 = threadIdx.x / rp;
    st.nchunk = kr / 8;
    st.ss = 0.0f;
#pragma unroll
    for (int q = 0; q < SQ; ++q) {
        const int c = st.j0 + q * st.tpr;
        stage_load<XDT, NORM, XAUX>(a, xr, gr, k0, c, st.m, c < st.nchunk && st.m <= a.M, st.raw[q], st.gam[q]);
    }
}

template <int WF, int XDT, bool NORM>
__device__ __forceinline__ void stage_store(const SkinnyArgs& a, int c, int ls, int plane, uint8_t* xs,
                                            const u32x4 (&raw)[XChunk<XDT>::XB / 16], const f32x4 (&gam)[2], int m,
                                            float& ss) {
    constexpr int OS = OpSize<WF>::v;
    constexpr bool SPLIT = XSplit<WF, XDT>::v;
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (XDT == DT_F32) {
            f[e] = __uint_as_float(raw[e >> 2][e & 3]);
        } else {
            const uint32_t hb = (raw[0][e >> 1] >> ((e & 1) * 16)) & 0xffffu;
            f[e] = XDT == DT_BF16 ? bf16_bits_to_f32(hb) : f16_bits_to_f32(hb);
        }
    }
    if constexpr (NORM) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= 1.0f + gam[e >> 2][e & 3];
    }
    uint8_t* dst = xs + ((int64_t)m * ls + c * 8) * OS;
    if constexpr (OS == 4) {
        reinterpret_cast<f32x4*>(dst)[0] = f32x4{f[0], f[1], f[2], f[3]};
        reinterpret_cast<f32x4*>(dst)[1] = f32x4{f[4], f[5], f[6], f[7]};
    } else {
        u32x4 hi, lo;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t h0 = op_bits<WF>(f[2 * p]), h1 = op_bits<WF>(f[2 * p + 1]);
            hi[p] = h0 | (h1 << 16);
            if constexpr (SPLIT) {
                const uint32_t l0 = op_bits<WF>(f[2 * p] - op_value<WF>(h0));
                const uint32_t l1 = op_bits<WF>(f[2 * p + 1] - op_value<WF>(h1));
                lo[p] = l0 | (l1 << 16);
            }
        }
        *reinterpret_cast<u32x4*>(dst) = hi;
        if constexpr (SPLIT) *reinterpret_cast<u32x4*>(dst + (int64_t)plane * OS) = lo;
    }
}

// Finish the staging; per-token sums of squares of the raw activations over
// the range go to ss_tok (LDS), reduced in a fixed order.
template <int WF, int XDT, int CT, int NW, int SQ, bool NORM, int XAUX = 0>
__device__ void stage_finish(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t gr, int k0,
                             int kr, XStage<XDT, SQ>& st, uint8_t* xs, float* ss_tok, float* ss_scratch) {
    constexpr int ROWS = CT * 16;
    const int ls = lds_row_elems<WF>(kr);
    const int plane = (a.M + 1) * ls;
    if (st.m <= a.M) {
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
            const int c = st.j0 + q * st.tpr;
            if (c < st.nchunk) stage_store<WF, XDT, NORM>(a, c, ls, plane, xs, st.raw[q], st.gam[q], st.m, st.ss);
        }
        for (int c = st.j0 + SQ * st.tpr; c < st.nchunk; c += st.tpr) {
            u32x4 raw[XChunk<XDT>::XB / 16];
            f32x4 gam[2];
            stage_load<XDT, NORM, XAUX>(a, xr, gr, k0, c, st.m, true, raw, gam);
            stage_store<WF, XDT, NORM>(a, c, ls, plane, xs, raw, gam, st.m, st.ss);
        }
    }
    if constexpr (NORM) {
        const int rp = 1 << (32 - __builtin_clz((unsigned)a.M));
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        float ss = st.ss;
        for (int off = rp; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
        if (lane < rp && lane < ROWS) ss_scratch[wave * ROWS + lane] = ss;
        __syncthreads();
        if (threadIdx.x < ROWS) {
            float t = 0.0f;
            for (int w = 0; w < NW; ++w) t += (threadIdx.x < rp) ? ss_scratch[w * ROWS + threadIdx.x] : 0.0f;
            ss_tok[threadIdx.x] = t;
        }
    }
}

// B operands of one k-step unit for one token tile, read from LDS.
template <int WF, int XDT> struct BOps;
template <int XDT> struct BOps<WF_BF16, XDT> { bf16x8 hi, lo; };
template <int XDT> struct BOps<WF_I8, XDT> { f16x8 hi0, hi1, lo0, lo1; };
template <int XDT> struct BOps<WF_F32, XDT> { f32x4 v; };

template <int WF, int XDT>
__device__ __forceinline__ void read_bops(BOps<WF, XDT>& b, const uint8_t* p, int plane_bytes) {
    constexpr bool SPLIT = XSplit<WF, XDT>::v;
    if constexpr (WF == WF_BF16) {
        b.hi = *reinterpret_cast<const bf16x8*>(p);
        if constexpr (SPLIT) b.lo = *reinterpret_cast<const bf16x8*>(p + plane_bytes);
    } else if constexpr (WF == WF_I8) {
        b.hi0 = reinterpret_cast<const f16x8*>(p)[0];
        b.hi1 = reinterpret_cast<const f16x8*>(p)[1];
        if constexpr (SPLIT) {
            b.lo0 = reinterpret_cast<const f16x8*>(p + plane_bytes)[0];
            b.lo1 = reinterpret_cast<const f16x8*>(p + plane_bytes)[1];
        }
    } else {
        b.v = *reinterpret_cast<const f32x4*>(p);
    }
}

// acc += A(unit) x B(unit)
template <int WF, int XDT>
__device__ __forceinline__ f32x4 unit_mfma(u32x4 a, const BOps<WF, XDT>& b, f32x4 acc) {
    constexpr bool SPLIT = XSplit<WF, XDT>::v;
    if constexpr (WF == WF_BF16) {
        bf16x8 av = __builtin_bit_cast(bf16x8, a);
        acc = mfma_bf16(av, b.hi, acc);
        if constexpr (SPLIT) acc = mfma_bf16(av, b.lo, acc);
    } else if constexpr (WF == WF_I8) {
        f16x8 a0, a1;
        i8unit_to_f16(a, a0, a1);
        acc = mfma_f16(a0, b.hi0, acc);
        acc = mfma_f16(a1, b.hi1, acc);
        if constexpr (SPLIT) {
            acc = mfma_f16(a0, b.lo0, acc);
            acc = mfma_f16(a1, b.lo1, acc);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = mfma_f32(__uint_as_float(a[e]), b.v[e], acc);
    }
    return acc;
}

// ---------------------------------------------------------------------------
// epilogue operands, issued with the weights and kept as raw bits until used
// ---------------------------------------------------------------------------
template <int RT, int CT>
struct EpiOps {
    u32x4 sc[RT];     // 4 FP32 scales of this lane's rows
    u32x4 res32[CT];  // residual, FP32 rows
    u32x2 res16[CT];  // residual, 16-bit rows
};

template <int RT, int CT>
__device__ __forceinline__ void load_epi(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t rr,
                                         int grp, bool valid, int lane, EpiOps<RT, CT>& e) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {  // the scale buffer is empty for non-INT8 weights
        const uint32_t so = valid ? (uint32_t)(((grp * RT + rt) * 16 + g * 4) * 4) : OOB;
        e.sc[rt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, so, 0, 0));
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {  // the residual buffer is empty without a residual
        const int m = ct * 16 + r;
        const int o = grp * 16 + g * 4;
        const bool ok = valid && a.vec_store && m < a.M && o < a.N;
        const uint32_t i = (uint32_t)((int64_t)m * a.ld_res + o);
        const bool f32 = a.res_dt == DT_F32;
        e.res32[ct] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, ok && f32 ? i * 4 : OOB, 0, 0));
        e.res16[ct] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rr, ok && !f32 ? i * 2 : OOB, 0, 0));
    }
}

__device__ __forceinline__ f32x4 as_f32x4(u32x4 v) {
    return f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}

__device__ __forceinline__ f32x4 epi_res(int dt, u32x4 r32, u32x2 r16) {
    if (dt == DT_F32) return as_f32x4(r32);
    f32x4 v;
    if (dt == DT_BF16) {
        v[0] = bf16_bits_to_f32(r16[0] & 0xffffu); v[1] = bf16_bits_to_f32(r16[0] >> 16);
        v[2] = bf16_bits_to_f32(r16[1] & 0xffffu); v[3] = bf16_bits_to_f32(r16[1] >> 16);
    } else {
        v[0] = f16_bits_to_f32(r16[0] & 0xffffu); v[1] = f16_bits_to_f32(r16[0] >> 16);
        v[2] = f16_bits_to_f32(r16[1] & 0xffffu); v[3] = f16_bits_to_f32(r16[1] >> 16);
    }
    return v;
}

// This wave's k-step range [kb, kend) within the split [ks0, ks1).
template <int NW>
__device__ __forceinline__ void wave_range(int ks0, int ks1, int wave_id, int& kb, int& kend) {
    const int cnt = ks1 - ks0;
    kb = ks0 + (wave_id * cnt) / NW;
    kend = ks0 + ((wave_id + 1) * cnt) / NW;
}

// Issue the weight loads of k-steps [kb, kb+n) (n <= U) of tile group grp;
// the U - n unused slots are issued out of range (zeros, no traffic).
template <int RT, int U>
__device__ __forceinline__ void issue_weights(const SkinnyArgs& a, __amdgpu_buffer_rsrc_t wrs, int grp, int kb,
                                              int n, int lane, u32x4 (&A)[U][RT]) {
    const uint32_t tile_bytes = (uint32_t)a.ksteps * 1024u;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            A[u][rt] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           wrs, u < n ? lane * 16 : OOB,
                           (uint32_t)(grp * RT + rt) * tile_bytes + (uint32_t)(kb + u) * 1024u, AUX_NT));
}

// ---------------------------------------------------------------------------
// register-direct activation operands (qw_gemv.hip, qw_mlp.hip)
// ---------------------------------------------------------------------------
// Activation fragments of one k-step as loaded: KE elements of XDT for each
// of the CT token tiles of the lane, and the matching (1 + gamma) weights
// (shared by the tiles).
template <int WF, int XDT, int CT> struct XFrag {
    static constexpr int KE = WTraits<WF>::KE;
    static constexpr int N16 = KE * 2 / 16;  // 16-byte loads per lane and tile (XDT is 16-bit)
    u32x4 v[CT][N16];
    f32x4 gam[KE / 4];
};

template <int WF, int XDT, int CT, bool GAM>
__device__ __forceinline__ void load_xfrag(__amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t gr, const uint32_t (&xoff)[CT],
                                           uint32_t goff, XFrag<WF, XDT, CT>& f) {
    constexpr int KE = WTraits<WF>::KE;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < XFrag<WF, XDT, CT>::N16; ++h)
            f.v[ct][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[ct] + 16 * h, 0, 0));
    if constexpr (GAM) {
#pragma unroll
        for (int h = 0; h < KE / 4; ++h)
            f.gam[h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, goff + 16 * h, 0, 0));
    }
}

// B operand of one token tile from a loaded fragment.  NORM: accumulate the
// squares; GAM: multiply by (1 + gamma) (without GAM the weight carries the
// norm weight and the activation bits pass through).
template <int WF, int XDT, int CT, bool NORM, bool GAM>
__device__ __forceinline__ BOps<WF, XDT> make_bops(const XFrag<WF, XDT, CT>& f, int ct, float& ss) {
    constexpr int KE = WTraits<WF>::KE;
    BOps<WF, XDT> b;
    constexpr bool SAME = (WF == WF_BF16 && XDT == DT_BF16) || (WF == WF_I8 && XDT == DT_F16);
    constexpr bool RAW = !GAM && SAME;
    if constexpr (NORM && RAW) {
#pragma unroll
        for (int p = 0; p < KE / 2; ++p) {
            const uint32_t w = f.v[ct][p >> 2][p & 3];
            const float e0 = XDT == DT_BF16 ? bf16_bits_to_f32(w & 0xffffu) : f16_bits_to_f32(w & 0xffffu);
            const float e1 = XDT == DT_BF16 ? bf16_bits_to_f32(w >> 16) : f16_bits_to_f32(w >> 16);
            ss += e0 * e0 + e1 * e1;
        }
    }
    if constexpr (RAW) {
        if constexpr (WF == WF_BF16) {
            b.hi = __builtin_bit_cast(bf16x8, f.v[ct][0]);
        } else {
            b.hi0 = __builtin_bit_cast(f16x8, f.v[ct][0]);
            b.hi1 = __builtin_bit_cast(f16x8, f.v[ct][1]);
        }
    } else {
        uint32_t out[KE / 2];
#pragma unroll
        for (int p = 0; p < KE / 2; ++p) {
            const uint32_t w = f.v[ct][p >> 2][p & 3];
            float e0, e1;
            if constexpr (XDT == DT_BF16) {
                e0 = bf16_bits_to_f32(w & 0xffffu);
                e1 = bf16_bits_to_f32(w >> 16);
            } else {
                e0 = f16_bits_to_f32(w & 0xffffu);
                e1 = f16_bits_to_f32(w >> 16);
            }
            if constexpr (NORM) ss += e0 * e0 + e1 * e1;
            if constexpr (GAM) {
                e0 *= 1.0f + f.gam[(2 * p) >> 2][(2 * p) & 3];
                e1 *= 1.0f + f.gam[(2 * p + 1) >> 2][(2 * p + 1) & 3];
            }
            out[p] = op_bits<WF>(e0) | (op_bits<WF>(e1) << 16);
        }
        if constexpr (WF == WF_BF16) {
            b.hi = __builtin_bit_cast(bf16x8, u32x4{out[0], out[1], out[2], out[3]});
        } else {
            b.hi0 = __builtin_bit_cast(f16x8, u32x4{out[0], out[1], out[2], out[3]});
            b.hi1 = __builtin_bit_cast(f16x8, u32x4{out[4], out[5], out[6], out[7]});
        }
    }
    return b;
}

}  // namespace qwk
