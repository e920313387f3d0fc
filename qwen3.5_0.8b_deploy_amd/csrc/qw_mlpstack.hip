// qw_mlpstack.hip -- L consecutive decoder MLP blocks in one persistent launch
// (decode, M <= 8 tokens, Qwen3.5-0.8B shape H = 1024, I = 3584):
//     for l < L:  x = x + down_l( silu(gate_l . n_l(x)) * (up_l . n_l(x)) ),
//                 n_l(x) = RMSNorm(x) * (1 + gamma_l),  x rounded to its dtype
// -- the result of L calls of qw_mlp_fused(y = residual = x), with the
// FP32 partial sums grouped differently (8 K slices of 4 k-steps for
// gate/up).
//
// Why.  One MLP block streams 22 MB of BF16 weights, about 3.5 us at the
// HBM rate, but a launch per block pays its start/end (~3 us) and its two
// data hand-offs serially, and no weight of block l+1 moves while block l
// waits for its hand-offs.  Here each block's weights are requested as soon
// as the registers that hold them are free, so they stream while the
// previous block's hand-offs are in flight.
//
// Work split (grid = 256 workgroups of 16 waves, one per CU, all resident):
//   * workgroups 0..191: gate/up.  Waves 8g..8g+7 own tile pair wg + 192 g
//     (intermediate rows [16p, 16p+16) of gate and up; the second group
//     exists in workgroups 0..31 only), the K = H reduction cut in eight
//     128-wide slices, one per wave;
//   * workgroups 192..255: down tile wg - 192 (output rows [16t, 16t+16))
//     over the full K = I, cut in eight 448-wide slices (waves 8..15); waves
//     0..7 poll the h slices of waves 8..15 and hand them over through LDS,
//     so the waves that stream weights never poll (vector-memory loads retire
//     in order: a poll issued behind a weight stream waits for all of it).
//     With INT8 weights and one token the down waves poll their own slices
//     instead (their weights have landed by the time h can arrive).
// A workgroup barrier is used once, at the start; the eight waves of a tile
// reduce their partial tiles through LDS, and the last of them to arrive (an
// LDS counter) runs the epilogue.  The others issue the next block's weight
// loads only after that epilogue's stores (loads issued just before would
// hold them up in the CU's memory pipeline).
//
// Hand-offs carry their own validity: every word written for another
// workgroup is a 64-bit agent-scope store of (tag << 32 | payload), tag =
// epoch * 64 + layer + 1, and a consumer polls the words it needs until
// every tag is the expected one -- no counters, no fences, no memset (a
// 64-bit store is seen whole or not at all).  `epoch` is a device word read
// by every wave at the start and advanced by workgroup 0 at the very end, so
// words of earlier launches never match; the tag keeps 26 bits of it, and
// the launch at which those wrap to zero clears every word first
// (wrap_clear_words).  Payloads, two 16-bit values each:
//   * h (gate/up -> down): h_buf[layer & 1][m][I/2], the down MFMA input type;
//   * x (down -> gate/up of the next block): x_buf[layer & 1][m][H/2], the
//     block output rounded to the activation dtype (the last block's is also
//     written to y).
// Buffers alternate by layer parity: a slot of layer l+2 is written only
// after every reader of layer l has passed (each layer's hand-offs depend on
// all of the previous one's).  A poll reads only the words the wave needs
// (one to four per lane), since poll traffic slows every other access.
//
// Every wait is bounded (0.2 s of the 100 MHz real-time counter): on expiry
// it raises the error flag (qw_device_error) and the launch's abort word, and
// every wave stops waiting, so the grid always drains.  Workgroups must all be
// resident: the launcher takes one workgroup per CU and refuses devices with
// fewer than 256 CUs.
//
// Reference: the post-norm + MLP + residual chain of CudaLayer::forward
// (cuda_engine.cu:119-124) over consecutive layers, i.e. CudaMLP::forward_add_
// residual (mlp_cuda.cu:295-337, the residual added) with RMSNorm
// (language_common.cpp:21-36) per block.
#include "qw_stream.hpp"

namespace qwk {

constexpr int MS_NW = 16;          // waves per workgroup: 8 gate/up + 8 down
constexpr int MS_RW = 8;           // waves per role
constexpr int MS_MAXM = 8;         // tokens (the MFMA's 16 token lanes, register budget 8)
constexpr int MS_H = 1024, MS_I = 3584;
constexpr int MS_GRID = 256;       // workgroups: one per CU
constexpr int MS_DT = MS_H / 16;   // down tiles (64), on workgroups [MS_D0, MS_GRID)
constexpr int MS_D0 = MS_GRID - MS_DT;
constexpr int MS_SPAN = 128;       // K values per wave slice (both roles, both formats)
constexpr int MS_LROW = MS_SPAN + 8;  // LDS row of a wave's B slice (16-byte pad)
constexpr int MS_DSPAN = MS_I / MS_RW;  // intermediate rows of a down wave's slice (448)
constexpr int MS_DROW = MS_DSPAN + 8;    // LDS row of a down wave's h slice (16-byte pad)

constexpr size_t MS_HWORDS = (size_t)2 * MS_MAXM * (MS_I / 2);   // h words: [parity][token][I/2]
constexpr size_t MS_XWORDS = (size_t)2 * MS_MAXM * (MS_H / 2);   // x words: [parity][token][H/2]
size_t mlp_stack_ws_bytes() { return (MS_HWORDS + MS_XWORDS) * 8; }
int mlp_stack_max_m() { return MS_MAXM; }
int mlp_stack_grid() { return MS_GRID; }

struct MsLds {
    uint16_t bs[MS_NW][MS_MAXM][MS_LROW];  // gate/up waves' B slices (MFMA input type bits; 16-byte rows)
    uint16_t bd[MS_RW][MS_MAXM][MS_DROW];  // down waves' h slices, deposited by their pollers
    f32x4 red_gu[2][MS_RW][2][64];         // gate/up partial tiles of the workgroup's (up to) two pairs
    f32x4 red_dn[MS_RW][64];               // down partial tiles
    // up to 4 tokens: the M token columns only, [row quad + 4 * token]
    f32x4 rc_gu[2][MS_RW][16][2];
    f32x4 rc_dn[MS_RW][16];
    float red_ss[2][MS_RW][MS_MAXM];
    float xt[MS_MAXM][16];                 // x of this workgroup's down tile rows
    unsigned cnt_gu[2], cnt_dn;            // arrivals at the reductions (reset by the last arriver)
    unsigned done_gu[2], done_dn;          // blocks whose epilogue has been issued
    unsigned hflag[MS_RW];                 // blocks whose h slice has been deposited for down wave d
    unsigned cnt_fin;                      // workgroup 0: gate/up waves that saw the final x
};

__device__ __forceinline__ uint32_t ms_tag(uint32_t epoch, int layer) { return (epoch << 6) | (uint32_t)(layer + 1); }
constexpr uint32_t MS_EFIELD = (1u << 26) - 1u;  // the epoch bits a tag keeps

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

// After a poll that did not find its words (the it-th miss of this wait):
// false once the wait that began at t0 has run 0.2 s of the 100 MHz real-time
// counter (then the error flag and the abort word are raised) or when another
// wave of this launch has aborted.  The clock is read on every 64th miss
// only, and the abort word once a wait has lasted 1 ms (waits last
// microseconds): thousands of waves polling one address would serialize at
// its memory channel and slow every hand-off.
__device__ __forceinline__ bool ms_pause(const MsAbort& ab, uint64_t t0, unsigned& it, bool& dead) {
    if ((++it & 63u) == 0u) {
        const uint64_t el = __builtin_amdgcn_s_memrealtime() - t0;
        if (el > 100000ull) {
            const bool expired = el > 20000000ull;
            const unsigned seen = __hip_atomic_load(ab.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (seen == ab.epoch + 1u || expired) {
                if (expired) {
                    __hip_atomic_store(ab.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(ab.abort, ab.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                dead = true;
                return false;
            }
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
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

// INT8 weight units converted to the f16 MFMA operands ahead of a wait, so
// the conversion is off the hand-off's critical path (24 INT8 blocks at M=1:
// 7.07 -> 6.22 us per block).  ON = false (BF16, or 8 tokens, where the
// converted operands would not fit the registers): converted in the MFMA chain.
template <int WF, int N, bool ON> struct MsConv {
    static constexpr bool C = ON && WF == WF_I8;
    f16x8 a0[C ? N : 1], a1[C ? N : 1];
    __device__ __forceinline__ void convert(const u32x4* A) {
        if constexpr (C) {
#pragma unroll
            for (int u = 0; u < N; ++u) {
                i8unit_to_f16(A[u], a0[u], a1[u]);
                u32x4 v0 = __builtin_bit_cast(u32x4, a0[u]), v1 = __builtin_bit_cast(u32x4, a1[u]);
                asm volatile("" : "+v"(v0), "+v"(v1));  // materialized here, before the wait
                a0[u] = __builtin_bit_cast(f16x8, v0);
                a1[u] = __builtin_bit_cast(f16x8, v1);
            }
        }
    }
    template <int XDT>
    __device__ __forceinline__ f32x4 mfma(int u, const u32x4& A, const BOps<WF, XDT>& b, f32x4 acc) const {
        if constexpr (C) {
            acc = mfma_f16(a0[u], b.hi0, acc);
            return mfma_f16(a1[u], b.hi1, acc);
        } else {
            return unit_mfma<WF, XDT>(A, b, acc);
        }
    }
};

// B operand of one k-step from an LDS slice [token][k] of row stride `ld`
// elements: lane (j, g) reads token j's elements [k + g*KE, +KE) (zeros for
// j >= M).
template <int WF>
__device__ __forceinline__ BOps<WF, (WF == WF_BF16 ? DT_BF16 : DT_F16)> ms_bops(const uint16_t* base, int ld, int k,
                                                                                 int lane, int M) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int XDT = WF == WF_BF16 ? DT_BF16 : DT_F16;
    const int j = lane & 15, g = lane >> 4;
    BOps<WF, XDT> b;
    const uint16_t* p = base + (j < M ? j : 0) * ld + k + g * KE;
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

// Bounded wait until the LDS counter c reaches `target` (deposits by the
// other role of this workgroup).  The clock is read on every 256th miss.
__device__ __forceinline__ void ms_wait_lds(unsigned* c, unsigned target, const MsAbort& ab, bool& dead) {
    uint64_t t0 = 0;
    unsigned it = 0;
    while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if ((it & 255u) == 0u) {
            const uint64_t now = __builtin_amdgcn_s_memrealtime();
            if (it == 0u) {
                t0 = now;
            } else if (now - t0 > 20000000ull) {
                __hip_atomic_store(ab.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(ab.abort, ab.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                dead = true;
                return;
            }
        }
        ++it;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");  // the deposited data is read only after the count
}

// Sum over the eight consecutive lanes of a group (every lane then holds its
// group's sum): quad_perm pairs and quads, then row_half_mirror.  Fixed order.
__device__ __forceinline__ float group8_sum(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    return dpp_add<0x141, 0xF>(v);  // row_half_mirror
}

// One LDS deposit done: the data writes complete, then the counter.
__device__ __forceinline__ void ms_deposit(unsigned* c, int lane) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
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
    constexpr int U_DN = KS_DN / MS_RW;                    // per down wave (14 / 7)
    constexpr int HWD = MS_DSPAN / 2;                      // h words per token of a down wave's slice (224)
    constexpr int NH = (HWD + 63) / 64;                    // per lane (4)
    // INT8 weights, one token: the down waves poll their own h slices (no
    // poller -> LDS -> flag hop; 24 blocks 6.0 -> 5.87 us per block); with
    // BF16 weights (twice the bytes in flight ahead of the first poll) that
    // measured slower (162.5 -> 166 us per 24 blocks), and more tokens spill
    constexpr bool SELF = WF == WF_I8 && MT == 1;
    // Partial-tile reduction up to 4 tokens (CMP): a wave writes only the M
    // token columns of its partial tile to LDS (combo c = row quad + 4 *
    // token, one f32x4 each); the last wave's lane 8 q + v reads wave v's
    // combos q, q + 8 and sums them over v with DPP adds, so the epilogue
    // reads 4 M f32x4 per wave instead of eight full tiles, and stores each
    // round's tokens as soon as they are summed (token 0 first: the pollers
    // wait for it).  24 blocks, us per block, BF16 / INT8: one token 6.74 ->
    // 6.51 / 5.94 -> 5.80, two 7.65 -> 7.20 / 7.13 -> 6.92, four 8.79 -> 8.20
    // / 8.32 -> 7.76.  Eight tokens keep the full tiles (10.36 against 10.77
    // compact, 12.05 with every token's words in one store instruction).
    constexpr bool CMP = MT <= 4;
    constexpr int NC = 4 * MT;            // combos the registers are sized for
    constexpr int NR = (NC + 7) / 8;      // combos per epilogue lane
    extern __shared__ __attribute__((aligned(16))) uint8_t ms_raw[];
    MsLds& S = *reinterpret_cast<MsLds*>(ms_raw);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int gq = MT <= 4 ? ((lane >> 3) & 3) : g;  // row quad of the epilogue lane's rows (scales)
    const int ev = lane & 7, eq = lane >> 3;  // epilogue lane: wave ev, combos eq + 8 r
    const int wg = blockIdx.x;
    const int M = a.M;
    const bool dn_wg = wg >= MS_D0;          // a down workgroup (tile t, full K); else gate/up
    const int t = wg - MS_D0;
    // every wave holds the epoch before the barrier, so workgroup 0 can only
    // advance it (at the very end, after all hand-offs) once all have read it
    const uint32_t epoch = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool dead = false;
    // the epoch's 26-bit tag field wraps every 2^26 launches: that launch
    // zeroes the hand-off words first (grid barrier), so no word written
    // 2^26 launches ago can match a tag of this launch
    if ((epoch & MS_EFIELD) == 0u && epoch != 0u)
        wrap_clear_words(a.hbuf, MS_HWORDS + MS_XWORDS, a.epoch + 2, a.err, &S.cnt_fin, dead);
    if (threadIdx.x < MS_RW) S.hflag[threadIdx.x] = 0u;
    if (threadIdx.x == 0) {
        S.cnt_gu[0] = S.cnt_gu[1] = 0u;
        S.done_gu[0] = S.done_gu[1] = 0u;
        S.cnt_dn = 0u;
        S.done_dn = 0u;
        S.cnt_fin = 0u;
    }
    if (dn_wg && threadIdx.x < 16 * MS_MAXM) {  // the down tile's rows of the first block input
        const int m = threadIdx.x >> 4, r = threadIdx.x & 15;
        S.xt[m][r] = m < M ? load_act(a.x, XDT, (int64_t)m * MS_H + t * 16 + r) : 0.0f;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();  // the only workgroup barrier (besides the wrap clear's)
    const MsAbort ab{a.err, a.epoch + 1, epoch};
    uint64_t* const hbuf = a.hbuf;
    uint64_t* const xbuf = a.xbuf;

    // The h slice of down wave w for block l (intermediate rows [448 w, 448 w +
    // 448)): polled through a buffer descriptor (one per-lane offset, the
    // token and parity in the scalar offset, device-coherent loads) and
    // deposited in the wave's LDS rows once every tag matched.
    auto poll_h = [&](int w, int l) {
        const __amdgpu_buffer_rsrc_t hrs = make_rsrc(hbuf, (uint32_t)(MS_HWORDS * 8));
        const uint32_t vb = (uint32_t)(((MS_DSPAN / 2) * w + lane) * 8);
        const uint32_t tg = ms_tag(epoch, l);
        const int so = (l & 1) * MS_MAXM * (MS_I / 2) * 8;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        unsigned it = 0;
        uint32_t v[MT][NH];  // payloads (the tags are checked as the words arrive)
        if constexpr (MT > 1) {
            // first token 0's words only: a producer stores all tokens'
            // words of its rows with one instruction, so once these
            // arrived the rest follow; polling them all costs every
            // other access MT times the poll traffic
            for (;;) {
                bool ok = true;
#pragma unroll
                for (int i = 0; i < NH; ++i) {
                    const int e = lane + 64 * i;
                    if (e < HWD) {
                        const u32x2 wv = __builtin_amdgcn_raw_buffer_load_b64(hrs, vb + 512 * i, so, AUX_SC1);
                        ok = ok && wv[1] == tg;
                    }
                }
                if (__all(ok) || dead) break;
                if (!ms_pause(ab, t0, it, dead)) break;
            }
        }
        // one token: a word once seen is not loaded again (fewer polls on
        // the lines every down workgroup reads); several tokens reload
        // every word (see the x polls)
        constexpr bool SKIP = MT == 1;
        bool got[MT][NH];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                got[m][i] = !(m < M && lane + 64 * i < HWD);
                v[m][i] = 0u;
            }
        for (;;) {
            bool ok = true;
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int i = 0; i < NH; ++i) {
                    if (SKIP) {
                        if (!got[m][i]) {
                            const u32x2 wv = __builtin_amdgcn_raw_buffer_load_b64(hrs, vb + 512 * i,
                                                                                  so + m * (MS_I / 2) * 8, AUX_SC1);
                            if (wv[1] == tg) {
                                v[m][i] = wv[0];
                                got[m][i] = true;
                            }
                        }
                        ok = ok && got[m][i];
                    } else {
                        const int e = lane + 64 * i;
                        u32x2 wv = u32x2{0u, tg};
                        if (m < M && e < HWD)
                            wv = __builtin_amdgcn_raw_buffer_load_b64(hrs, vb + 512 * i, so + m * (MS_I / 2) * 8,
                                                                      AUX_SC1);
                        ok = ok && wv[1] == tg;
                        v[m][i] = wv[0];
                    }
                }
            if (__all(ok) || dead) break;
            if (!ms_pause(ab, t0, it, dead)) break;
        }
        if (a.trace && lane == 0) {
            const uint64_t now = __builtin_amdgcn_s_memrealtime();
            if (w == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 2] = now;
            a.trace[((size_t)l * MS_GRID + wg) * 16 + 4 + w] = now;  // per poller
        }
        // LDS only once valid: the down wave may still be reading the
        // previous block's slice until then (h of block l+1 exists only
        // after this workgroup's x of block l has been published)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                const int e = lane + 64 * i;
                if (m < M && e < HWD) *reinterpret_cast<uint32_t*>(&S.bd[w][m][2 * e]) = v[m][i];
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
    };

    if (!dn_wg) {
        // ===================== gate/up =====================
        // group grp (waves 8 grp .. 8 grp + 7) owns tile pair p; per block:
        // poll this wave's x slice (the down workgroups' words) -> gate/up
        // partial tiles -> the last of the eight stores h; the next block's
        // weights are requested only after that store (loads issued earlier
        // would hold up the store in the CU's memory pipeline), and they have
        // the whole down half of the block to arrive
        const int grp = wave / MS_RW, w = wave % MS_RW;
        const int p = wg + MS_D0 * grp;
        if (p >= MS_I / 16) return;
        const int k0 = w * MS_SPAN;            // this wave's K slice [k0, k0 + 128)
        const uint32_t tile_bytes = (uint32_t)KS_GU * 1024u;
        u32x4 A[U_GU][2];
        float gm[2] = {0.f, 0.f};
        u32x4 sc[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
        auto issue = [&](int l) {
            const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.gu[l], (uint32_t)(MS_I / 16) * 2u * tile_bytes);
            if (a.dbg & 1) {  // timing probe: no gate/up weight traffic (wrong results)
#pragma unroll
                for (int u = 0; u < U_GU; ++u) A[u][0] = A[u][1] = u32x4{(uint32_t)l, 0u, 0u, 0u};
                return;
            }
            // the k-steps go out a.gap ticks of the 100 MHz clock apart: all
            // of a workgroup's gate/up weights requested at once, right after
            // its epilogue stores, delay the hand-off words then in flight
            // (24 BF16 blocks at M = 1 with a per-call gamma: 184 us per step
            // at once, 162 us at 20 ticks apart, 143 us with no gate/up weight
            // loads at all; 10 to 60 ticks measure alike; INT8, two k-steps
            // per wave: 6.60 / 6.24 / 5.99 us per block at 0 / 20 / 120 ticks)
            const uint64_t tb = __builtin_amdgcn_s_memrealtime();
#pragma unroll
            for (int u = 0; u < U_GU; ++u) {
                if (u > 0 && a.gap > 0)
                    while (__builtin_amdgcn_s_memrealtime() - tb < (uint64_t)(u * a.gap)) __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    A[u][rt] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   wr, lane * 16, (uint32_t)(p * 2 + rt) * tile_bytes + (uint32_t)(w * U_GU + u) * 1024u,
                                   AUX_NT));
            }
            if constexpr (GAM) {
                gm[0] = a.gamma[l][k0 + 2 * lane];
                gm[1] = a.gamma[l][k0 + 2 * lane + 1];
            }
            if constexpr (WF == WF_I8) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    sc[rt] = *reinterpret_cast<const u32x4*>(a.gu_scales[l] + (p * 2 + rt) * 16 + gq * 4);
            }
        };
        // this lane's elements of the slice: k0 + 2*lane + {0, 1} of every token
        float xv[MT][2];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int e = 0; e < 2; ++e) xv[m][e] = m < M ? load_act(a.x, XDT, (int64_t)m * MS_H + k0 + 2 * lane + e) : 0.0f;
        issue(0);
        MsConv<WF, 2 * U_GU, (MT <= 4)> cv;
        for (int l = 0; l <= a.L; ++l) {
            if (l < a.L) cv.convert(&A[0][0]);
            if (l > 0) {
                // x of block l: one word (two rows) per lane and token
                const uint32_t tg = ms_tag(epoch, l - 1);
                const uint64_t* X = xbuf + (size_t)((l - 1) & 1) * MS_MAXM * (MS_H / 2) + k0 / 2 + lane;
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                unsigned it = 0;
                uint64_t v[MT];
                if constexpr (MT > 1) {  // token 0's word first (see the h pollers)
                    for (;;) {
                        const bool ok = (uint32_t)(ms_load(X) >> 32) == tg;
                        if (__all(ok) || dead) break;
                        if (!ms_pause(ab, t0, it, dead)) break;
                    }
                }
                // one token: a word once seen is not loaded again, so the
                // remaining polls are only those of words still in flight
                // (24 BF16 blocks: 159.5 -> 154.7 us); with several tokens the
                // per-word branches cost more than they save (8 tokens: 11.5
                // -> 20.8 us per block), so every round reloads every word
                constexpr bool SKIP = MT == 1;
                bool got[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) got[m] = m >= M;
#pragma unroll
                for (int m = 0; m < MT; ++m) v[m] = (uint64_t)tg << 32;
                for (;;) {
                    bool ok = true;
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (SKIP) {
                            if (!got[m]) {
                                const uint64_t wv = ms_load(X + (size_t)m * (MS_H / 2));
                                if ((uint32_t)(wv >> 32) == tg) {
                                    v[m] = wv;
                                    got[m] = true;
                                }
                            }
                            ok = ok && got[m];
                        } else {
                            v[m] = m < M ? ms_load(X + (size_t)m * (MS_H / 2)) : ((uint64_t)tg << 32);
                            ok = ok && (uint32_t)(v[m] >> 32) == tg;
                        }
                    }
                    if (__all(ok) || dead) break;
                    if (!ms_pause(ab, t0, it, dead)) break;
                }
                if (a.trace && grp == 0 && lane == 0) {
                    const uint64_t now = __builtin_amdgcn_s_memrealtime();
                    if (w == 0) a.trace[((size_t)(l - 1) * MS_GRID + wg) * 16 + 0] = now;
                    a.trace[((size_t)(l - 1) * MS_GRID + wg) * 16 + 4 + w] = now;  // per wave
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const uint32_t w2 = (uint32_t)v[m];
                    xv[m][0] = XDT == DT_BF16 ? bf16_bits_to_f32(w2 & 0xffffu) : f16_bits_to_f32(w2 & 0xffffu);
                    xv[m][1] = XDT == DT_BF16 ? bf16_bits_to_f32(w2 >> 16) : f16_bits_to_f32(w2 >> 16);
                }
            }
            if (l == a.L) {
                // workgroup 0: once all eight slices of the final x have been
                // seen, every workgroup has read the epoch: advance it
                if (wg == 0 && grp == 0) {
                    unsigned old = 0;
                    if (lane == 0) old = __hip_atomic_fetch_add(&S.cnt_fin, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    old = __shfl(old, 0);
                    if (old == MS_RW - 1 && lane == 0)
                        __hip_atomic_store(a.epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                break;
            }
            // B slice: round(x * (1 + gamma)) in the MFMA type; sums of squares per token
            float ss[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float a0 = xv[m][0], a1 = xv[m][1];
                ss[m] = a0 * a0 + a1 * a1;
                if (m < M) {
                    const uint32_t b0 = op_bits<WF>(GAM ? a0 * (1.0f + gm[0]) : a0);
                    const uint32_t b1 = op_bits<WF>(GAM ? a1 * (1.0f + gm[1]) : a1);
                    *reinterpret_cast<uint32_t*>(&S.bs[wave][m][2 * lane]) = b0 | (b1 << 16);
                }
            }
            // per-token sums of squares of the slice: DPP adds, the total in
            // lane 63 (no LDS round trips on the way to the MFMAs)
#pragma unroll
            for (int m = 0; m < MT; ++m) ss[m] = wave_sum_to_lane63(ss[m]);
            lds_fence_wave();
            f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U_GU; ++u) {
                const auto b = ms_bops<WF>(&S.bs[wave][0][0], MS_LROW, u * 4 * KE, lane, M);
                accg = cv.template mfma<OPDT>(2 * u, A[u][0], b, accg);
                accu = cv.template mfma<OPDT>(2 * u + 1, A[u][1], b, accu);
            }
            // reduce the eight slices: the last wave to arrive runs the epilogue
            if constexpr (CMP) {
                if (j < M) {
                    S.rc_gu[grp][w][g + 4 * j][0] = accg;
                    S.rc_gu[grp][w][g + 4 * j][1] = accu;
                }
            } else {
                S.red_gu[grp][w][0][lane] = accg;
                S.red_gu[grp][w][1][lane] = accu;
            }
            if (lane == 63) {
#pragma unroll
                for (int m = 0; m < MT; ++m) S.red_ss[grp][w][m] = ss[m];
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&S.cnt_gu[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __builtin_amdgcn_readfirstlane(old);
            if (old == MS_RW - 1) {
                if (a.trace && grp == 0 && lane == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 12] = __builtin_amdgcn_s_memrealtime();
                if (lane == 0) __hip_atomic_store(&S.cnt_gu[grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                if constexpr (CMP) {
                    const uint32_t tg = ms_tag(epoch, l);
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        const int c = eq + 8 * r, jt = c >> 2;  // combo: rows [4 gq, 4 gq + 4) of token jt
                        const int cc = c < NC ? c : 0;
                        f32x4 gs = S.rc_gu[grp][ev][cc][0], us = S.rc_gu[grp][ev][cc][1];
                        float sst = S.red_ss[grp][ev][jt < MT ? jt : 0];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            gs[i] = group8_sum(gs[i]);
                            us[i] = group8_sum(us[i]);
                        }
                        sst = group8_sum(sst);
                        const float inv = 1.0f / sqrtf(sst / (float)MS_H + a.eps);
                        if constexpr (WF == WF_I8) {
                            gs *= as_f32x4(sc[0]);
                            us *= as_f32x4(sc[1]);
                        }
                        if (ev == 0 && jt < M) {
                            uint32_t hb[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) hb[i] = op_bits<WF>(silu_f(gs[i] * inv) * (us[i] * inv));
                            uint64_t* hw = hbuf + ((size_t)(l & 1) * MS_MAXM + jt) * (MS_I / 2) + (p * 16 + gq * 4) / 2;
                            ms_store(hw, tg, hb[0] | (hb[1] << 16));
                            ms_store(hw + 1, tg, hb[2] | (hb[3] << 16));
                        }
                    }
                } else {
                    // the partials summed in wave order
                    const int jj = j < M ? j : 0;
                    f32x4 pv[MS_RW];
                    float ps[MS_RW];
    #pragma unroll
                    for (int v = 0; v < MS_RW; ++v) {
                        pv[v] = S.red_gu[grp][v][0][lane];
                        ps[v] = S.red_ss[grp][v][jj];
                    }
                    f32x4 gs = pv[0];
                    float sst = ps[0];
    #pragma unroll
                    for (int v = 1; v < MS_RW; ++v) {
                        gs += pv[v];
                        sst += ps[v];
                    }
    #pragma unroll
                    for (int v = 0; v < MS_RW; ++v) pv[v] = S.red_gu[grp][v][1][lane];
                    f32x4 us = pv[0];
    #pragma unroll
                    for (int v = 1; v < MS_RW; ++v) us += pv[v];
                    const float inv = 1.0f / sqrtf(sst / (float)MS_H + a.eps);
                    if constexpr (WF == WF_I8) {
                        gs *= as_f32x4(sc[0]);
                        us *= as_f32x4(sc[1]);
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
                if (a.trace && grp == 0 && lane == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 1] = __builtin_amdgcn_s_memrealtime();
                if (lane == 0) __hip_atomic_store(&S.done_gu[grp], (unsigned)(l + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
                ms_wait_lds(&S.done_gu[grp], (unsigned)(l + 1), ab, dead);
            }
            if (l + 1 < a.L) issue(l + 1);  // the next block's weights stream during the hand-offs
        }
    } else if (wave < MS_RW) {
        // ===================== h pollers of the down waves =====================
        // wave w polls the h slice of down wave w and deposits it in LDS; a
        // poller issues no weight loads, so its polls never wait behind a
        // weight stream
        if constexpr (SELF) return;  // the down waves poll their own slices
        const int w = wave;
        for (int l = 0; l < a.L; ++l) {
            poll_h(w, l);
            if (lane == 0) __hip_atomic_store(&S.hflag[w], (unsigned)(l + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    } else {
        // ===================== down =====================
        // per block: the h slice (LDS, from the poller) -> partial tile ->
        // the last of the eight adds the partials to x of the tile's rows and
        // publishes them as 16-bit pairs (after the last block also as y);
        // the next block's weights are requested after that
        const int d = wave - MS_RW;
        const int kb = d * U_DN;                  // this wave's k-steps [kb, kb + U_DN)
        const uint32_t tile_bytes = (uint32_t)KS_DN * 1024u;
        u32x4 A[U_DN];
        u32x4 sc = u32x4{0u, 0u, 0u, 0u};
        auto issue = [&](int l) {
            const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.dn[l], (uint32_t)(MS_H / 16) * tile_bytes);
            if (a.dbg & 2) {  // timing probe: no down weight traffic (wrong results)
#pragma unroll
                for (int u = 0; u < U_DN; ++u) A[u] = u32x4{(uint32_t)l, 0u, 0u, 0u};
                return;
            }
#pragma unroll
            for (int u = 0; u < U_DN; ++u)
                A[u] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               wr, lane * 16, (uint32_t)t * tile_bytes + (uint32_t)(kb + u) * 1024u, AUX_NT));
            if constexpr (WF == WF_I8) sc = *reinterpret_cast<const u32x4*>(a.dn_scales[l] + t * 16 + gq * 4);
        };
        issue(0);
        MsConv<WF, U_DN, (MT <= 4)> cv;
        for (int l = 0; l < a.L; ++l) {
            const uint32_t tg = ms_tag(epoch, l);
            cv.convert(A);
            if constexpr (SELF) poll_h(d, l);
            else ms_wait_lds(&S.hflag[d], (unsigned)(l + 1), ab, dead);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U_DN; ++u) {
                const auto b = ms_bops<WF>(&S.bd[d][0][0], MS_DROW, u * 4 * KE, lane, M);
                acc = cv.template mfma<OPDT>(u, A[u], b, acc);
            }
            if constexpr (CMP) {
                if (j < M) S.rc_dn[d][g + 4 * j] = acc;
            } else {
                S.red_dn[d][lane] = acc;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&S.cnt_dn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __builtin_amdgcn_readfirstlane(old);
            if (old == MS_RW - 1) {
                if (a.trace && lane == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 12] = __builtin_amdgcn_s_memrealtime();
                if (lane == 0) __hip_atomic_store(&S.cnt_dn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                if constexpr (CMP) {
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        // as the gate/up epilogue: combo c = rows [4 gq, 4 gq + 4) of token jt
                        const int c = eq + 8 * r, jt = c >> 2;
                        f32x4 sv = S.rc_dn[ev][c < NC ? c : 0];
#pragma unroll
                        for (int i = 0; i < 4; ++i) sv[i] = group8_sum(sv[i]);
                        if constexpr (WF == WF_I8) sv *= as_f32x4(sc);
                        if (ev == 0 && jt < M) {
                            uint32_t xb[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const float xn = round_act<XDT>(S.xt[jt][gq * 4 + i] + sv[i]);
                                S.xt[jt][gq * 4 + i] = xn;
                                xb[i] = XDT == DT_BF16 ? f32_to_bf16_bits(xn) : f32_to_f16_bits(xn);
                            }
                            uint64_t* xw = xbuf + ((size_t)(l & 1) * MS_MAXM + jt) * (MS_H / 2) + (t * 16 + gq * 4) / 2;
                            ms_store(xw, tg, xb[0] | (xb[1] << 16));
                            ms_store(xw + 1, tg, xb[2] | (xb[3] << 16));
                            if (a.trace && lane == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 3] = __builtin_amdgcn_s_memrealtime();
                            if (l + 1 == a.L) {
                                uint32_t* yw = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.y) + (size_t)jt * MS_H + t * 16 + gq * 4);
                                yw[0] = xb[0] | (xb[1] << 16);
                                yw[1] = xb[2] | (xb[3] << 16);
                            }
                        }
                    }
                } else {
                    f32x4 pd[MS_RW];
    #pragma unroll
                    for (int v = 0; v < MS_RW; ++v) pd[v] = S.red_dn[v][lane];
                    f32x4 s = pd[0];
    #pragma unroll
                    for (int v = 1; v < MS_RW; ++v) s += pd[v];
                    if constexpr (WF == WF_I8) s *= as_f32x4(sc);
                    if (j < M) {
                        uint32_t xb[4];
    #pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float xn = round_act<XDT>(S.xt[j][g * 4 + i] + s[i]);
                            S.xt[j][g * 4 + i] = xn;
                            xb[i] = XDT == DT_BF16 ? f32_to_bf16_bits(xn) : f32_to_f16_bits(xn);
                        }
                        uint64_t* xw = xbuf + ((size_t)(l & 1) * MS_MAXM + j) * (MS_H / 2) + (t * 16 + g * 4) / 2;
                        ms_store(xw, tg, xb[0] | (xb[1] << 16));
                        ms_store(xw + 1, tg, xb[2] | (xb[3] << 16));
                        if (a.trace && lane == 0) a.trace[((size_t)l * MS_GRID + wg) * 16 + 3] = __builtin_amdgcn_s_memrealtime();
                        if (l + 1 == a.L) {
                            uint32_t* yw = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.y) + (size_t)j * MS_H + t * 16 + g * 4);
                            yw[0] = xb[0] | (xb[1] << 16);
                            yw[1] = xb[2] | (xb[3] << 16);
                        }
                    }
                }
                if (lane == 0) __hip_atomic_store(&S.done_dn, (unsigned)(l + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
                ms_wait_lds(&S.done_dn, (unsigned)(l + 1), ab, dead);
            }
            if (l + 1 < a.L) issue(l + 1);  // the next block's weights stream during the hand-offs
        }
    }
}

template <typename Kern>
static hipError_t launch_ms(Kern k, const MlpStackArgs& a, hipStream_t st) {
    // more than half the CU's LDS: one workgroup per CU
    constexpr size_t lds = ((sizeof(MsLds) + 1023) / 1024 * 1024) > 96 * 1024 ? (sizeof(MsLds) + 1023) / 1024 * 1024
                                                                                : 96 * 1024;
    static_assert(lds <= 160 * 1024, "LDS layout");
    {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(MS_GRID), dim3(MS_NW * 64), lds, st, a);
    return hipGetLastError();
}

template <int WF, int XDT, bool GAM>
static hipError_t launch_ms2(const MlpStackArgs& a, hipStream_t st) {
    if (a.M == 1) return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 1>, a, st);
    if (a.M == 2) return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 2>, a, st);
    if (a.M <= 4) return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 4>, a, st);
    return launch_ms(mlp_stack_kernel<WF, XDT, GAM, 8>, a, st);
}

template <int WF, int XDT>
static hipError_t launch_ms1(const MlpStackArgs& a, hipStream_t st) {
    if (a.gamma[0]) return launch_ms2<WF, XDT, true>(a, st);
    return launch_ms2<WF, XDT, false>(a, st);
}

hipError_t launch_mlp_stack(const MlpStackArgs& a, int wf, int xdt, hipStream_t stream) {
    if (a.L < 1 || a.L > kMlpStackMaxLayers || a.M < 1 || a.M > mlp_stack_max_m()) return hipErrorInvalidValue;
    MlpStackArgs b = a;
    b.xbuf = a.hbuf + MS_HWORDS;  // the x words follow the h words
    if (wf == WF_BF16 && xdt == DT_BF16) return launch_ms1<WF_BF16, DT_BF16>(b, stream);
    if (wf == WF_I8 && xdt == DT_F16) return launch_ms1<WF_I8, DT_F16>(b, stream);
    return hipErrorInvalidValue;
}

}  // namespace qwk
