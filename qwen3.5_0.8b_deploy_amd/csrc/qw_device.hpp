// qw_device.hpp -- device-side building blocks shared by the gfx950 kernels.
//
// Packed weight layout ("tile order").  A weight W[N][K] is cut into tiles of
// 16 rows.  Along K, each row is cut into 16-byte units of KE elements
// (KE = 4 for FP32, 8 for BF16, 16 for INT8).  One "k-step" of a tile is the
// 64 units that one wave64 loads with a single 16-byte-per-lane instruction:
// lane l = r + 16*g (r = row within the tile, g = 0..3) holds
//     W[16*t + r][ks*4*KE + g*KE + e],  e = 0..KE-1.
// The k-step blocks of a tile are contiguous (1 KB each), tiles follow each
// other.  This is exactly the A-operand register layout of the gfx950 MFMA
// instructions used here (row = lane % 16, k-group = lane / 16), so a weight
// k-step goes from HBM into MFMA registers with one fully coalesced 1 KB
// wave load and no LDS round trip.  The activation operand B is read with the
// same k permutation: lane (j = token, g) holds x[j][ks*4*KE + g*KE + e].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qwk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_I8 = 3 };
enum WFmt { WF_F32 = 0, WF_BF16 = 1, WF_I8 = 2 };

// elements of a weight per 16-byte unit
template <int WF> struct WTraits;
template <> struct WTraits<WF_F32> { static constexpr int KE = 4; };
template <> struct WTraits<WF_BF16> { static constexpr int KE = 8; };
template <> struct WTraits<WF_I8> { static constexpr int KE = 16; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    // round to nearest even; gfx950 converts in hardware (v_cvt_pk_bf16_f32)
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (unsigned short)h);
    return (float)v;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 v = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(unsigned short, v);
}

// Scalar load of element i of an activation array of dtype dt, as float.
__device__ __forceinline__ float load_act(const void* p, int dt, int64_t i) {
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    uint32_t h = reinterpret_cast<const unsigned short*>(p)[i];
    return dt == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

__device__ __forceinline__ void store_act(void* p, int dt, int64_t i, float v) {
    if (dt == DT_F32) {
        reinterpret_cast<float*>(p)[i] = v;
    } else {
        uint32_t h = dt == DT_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        reinterpret_cast<unsigned short*>(p)[i] = (unsigned short)h;
    }
}

// Four consecutive outputs (16 B for F32, 8 B for 16-bit types); caller
// guarantees alignment (ldy and o multiples of 4).
__device__ __forceinline__ void store_act4(void* p, int dt, int64_t i, f32x4 v) {
    if (dt == DT_F32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p) + i) = v;
    } else {
        uint32_t h0, h1, h2, h3;
        if (dt == DT_BF16) {
            h0 = f32_to_bf16_bits(v[0]); h1 = f32_to_bf16_bits(v[1]);
            h2 = f32_to_bf16_bits(v[2]); h3 = f32_to_bf16_bits(v[3]);
        } else {
            h0 = f32_to_f16_bits(v[0]); h1 = f32_to_f16_bits(v[1]);
            h2 = f32_to_f16_bits(v[2]); h3 = f32_to_f16_bits(v[3]);
        }
        u32x2 w;
        w[0] = h0 | (h1 << 16);
        w[1] = h2 | (h3 << 16);
        *reinterpret_cast<u32x2*>(reinterpret_cast<unsigned short*>(p) + i) = w;
    }
}

__device__ __forceinline__ f32x4 load_act4(const void* p, int dt, int64_t i) {
    f32x4 r;
    if (dt == DT_F32) {
        r = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + i);
    } else {
        u32x2 w = *reinterpret_cast<const u32x2*>(reinterpret_cast<const unsigned short*>(p) + i);
        if (dt == DT_BF16) {
            r[0] = bf16_bits_to_f32(w[0] & 0xffffu); r[1] = bf16_bits_to_f32(w[0] >> 16);
            r[2] = bf16_bits_to_f32(w[1] & 0xffffu); r[3] = bf16_bits_to_f32(w[1] >> 16);
        } else {
            r[0] = f16_bits_to_f32(w[0] & 0xffffu); r[1] = f16_bits_to_f32(w[0] >> 16);
            r[2] = f16_bits_to_f32(w[1] & 0xffffu); r[3] = f16_bits_to_f32(w[1] >> 16);
        }
    }
    return r;
}

// Streaming 16-byte weight load: read once per pass, so mark it non-temporal.
__device__ __forceinline__ u32x4 load_w16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Four signed bytes -> four exact halves.  u = b + 128 is placed in the low
// mantissa bits of 1024.0h (bits 0x6400), giving 1024 + u; subtracting 1152
// leaves b exactly (|b| <= 128 is far inside binary16's exact-integer range).
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    uint32_t u = w ^ 0x80808080u;
    uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0,64,u1,64
    uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2,64,u3,64
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    f16x2 a = __builtin_bit_cast(f16x2, p0) - bias;
    f16x2 b = __builtin_bit_cast(f16x2, p1) - bias;
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
}

// 16 int8 weights of one unit -> two f16x8 MFMA operands (k order kept).
__device__ __forceinline__ void i8unit_to_f16(u32x4 w, f16x8& a0, f16x8& a1) {
    u32x4 o0, o1;
    uint32_t l, h;
    i8x4_to_f16(w[0], l, h); o0[0] = l; o0[1] = h;
    i8x4_to_f16(w[1], l, h); o0[2] = l; o0[3] = h;
    i8x4_to_f16(w[2], l, h); o1[0] = l; o1[1] = h;
    i8x4_to_f16(w[3], l, h); o1[2] = l; o1[3] = h;
    a0 = __builtin_bit_cast(f16x8, o0);
    a1 = __builtin_bit_cast(f16x8, o1);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sum over the 64 lanes of a wave with DPP moves only (no LDS crossbar, unlike
// __shfl_xor's ds_bpermute): pairs, quads, half rows and rows by quad_perm /
// row_half_mirror / row_mirror (every lane then holds its row's sum), then
// row_bcast:15 and row_bcast:31 carry the row sums upward, so lane 63 holds
// the total (the other lanes hold partial sums).  Fixed order: deterministic.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false);
    return v + __builtin_bit_cast(float, o);
}
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xF>(v);  // row_mirror
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + __expf(-v)); }

// Orderable key of (value, index): larger value wins, then LOWER index wins.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - idx);
}
__device__ __forceinline__ float key_value(unsigned long long key) {
    uint32_t ord = (uint32_t)(key >> 32);
    uint32_t u = (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord;
    return __uint_as_float(u);
}
__device__ __forceinline__ uint32_t key_index(unsigned long long key) {
    return 0xffffffffu - (uint32_t)(key & 0xffffffffull);
}

}  // namespace qwk
