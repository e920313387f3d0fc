// qw_chain.hip -- a chain of dependent projections in one persistent launch
// (decode, M <= 2 tokens): the layer sequence of the decoder between the
// attention / Gated-DeltaNet cores, e.g. per layer
//     in  : x -> [QKV|Z|a|b]            (norm prologue optional)
//     out : [..][0, 2048) -> x (+ x)    (the core's output in the real model)
//     gate/up : x -> h  (SiLU*mul)      (norm prologue optional)
//     down : h -> x (+ x)
// Each op's input is the previous op's output (a "linear chain"), so every op
// waits for its whole input vector, as a separate launch would, but nothing
// else: no launch gaps, and each wave requests the weights of the next op it
// takes part in as soon as its MFMAs are done, so the weights stream while
// the hand-offs are in flight.
//
// Activations live in "slots" of tagged 64-bit words (tag << 32 | two 16-bit
// values; tag = epoch << 10 | op + 1, 0 for the values imported at launch
// start), written with agent-scope stores and polled until every tag is the
// one expected; `epoch` advances once per launch, so no word needs clearing
// (graph replays included) except when the tag's 22 epoch bits wrap (below).
//
// Work split (grid = 256 workgroups of 16 waves, one per CU, all resident):
// op o's output blocks (16-row tiles, or gate/up tile pairs) go round robin to
// the workgroups starting at workgroup base_o (the host staggers the bases so
// that consecutive small ops land on different CUs); within a workgroup the
// (block, k-step) units are cut into 12 contiguous ranges, one per compute
// wave (at most 10 weight loads each).  Waves 0..3 are pollers: per op they
// wait for the input words, deposit them in LDS (times 1 + gamma, in the MFMA
// type, with the per-token sums of squares), and fetch the residual rows and
// INT8 row scales of the workgroup's blocks; they issue no weight loads, so
// their polls never wait behind a weight stream (vector-memory loads retire in
// order).  The compute waves reduce their partial tiles through LDS; the last
// to arrive (an LDS counter) runs the epilogue (1/rms, scale, SiLU*mul,
// residual, rounding to the slot's 16-bit type) and stores the output words
// (and the plain values to an export buffer); the others request their next
// weights once those stores are issued.  Parity-double-buffered LDS inputs
// are safe because every op depends on all of the previous one.
//
// Every wait is bounded (0.2 s of the 100 MHz real-time counter): on expiry
// it raises the error flag (qw_device_error) and this launch's abort word, and
// every wave stops waiting, so the grid always drains.
//
// Reference: the per-layer projection sequence of CudaLayer::forward
// (cuda_engine.cu:105-124) -- CudaLinearAttention / CudaFullAttention input
// and output projections (linear_attention_cuda.cu:174-187,
// full_attention_cuda.cu:451-600) and CudaMLP::forward_add_residual
// (mlp_cuda.cu:295-337) -- at one or two decode tokens.
#include "qw_stream.hpp"

namespace qwk {

constexpr int CH_NW = 16;             // waves per workgroup
constexpr int CH_NP = 4;              // poller waves
constexpr int CH_CW = CH_NW - CH_NP;  // compute waves
constexpr int CH_GRID = 256;
constexpr int CH_MAXM = 2;
constexpr int CH_LROW = kChainMaxK + 8;  // LDS row of the staged input (16-byte pad)
constexpr int CH_TW = 3;              // output blocks per workgroup and op
// weight loads per compute wave and op, and the ops whose weights a wave
// holds: BF16 one op of up to 10 loads; INT8 (half the k-steps) two ops of up
// to 5, so the weights of the op after next stream during the current one
template <int WF> struct ChBuf {
    static constexpr int ULD = WF == WF_I8 ? 5 : 10;
    static constexpr int NBUF = WF == WF_I8 ? 2 : 1;
};
// input words per poller lane for MT tokens
constexpr int ch_pw(int MT) { return (MT * kChainMaxK / 2 + CH_NP * 64 - 1) / (CH_NP * 64); }

struct ChLds {
    uint16_t xin[2][CH_MAXM][CH_LROW];  // staged input (MFMA type bits), by participation parity
    f32x4 red[CH_TW][CH_CW][2][64];     // partial tiles of the compute waves
    float ss[2][CH_NP][CH_MAXM];        // sums of squares of the input, per poller
    float sc[2][CH_TW][2][16];          // INT8 row scales of the workgroup's blocks
    float res[2][CH_TW][CH_MAXM][16];   // residual rows of the workgroup's blocks
    unsigned ready[2][CH_NP];           // participation + 1 whose input poller p has deposited
    unsigned cnt, done;                 // compute-wave arrivals; participations whose epilogue is issued
    ChainOp ops[kChainMaxOps];          // the op table, copied once (read every op by every wave)
};

__device__ __forceinline__ uint32_t ch_tag(uint32_t epoch, int op_tag) { return (epoch << 10) | (uint32_t)op_tag; }
// The tag keeps 22 bits of the epoch.  The epoch skips the values whose field
// is 0 (an import tag would then be 0, the value of a cleared word), so the
// field runs 1 .. 2^22 - 1, and the launch at which it returns to 1 clears
// every slot word first (wrap_clear_words).
constexpr uint32_t CH_EFIELD = (1u << 22) - 1u;
__device__ __forceinline__ uint32_t ch_next_epoch(uint32_t e) {
    const uint32_t n = e + 1u;
    return (n & CH_EFIELD) == 0u ? n + 1u : n;
}

__device__ __forceinline__ uint64_t ch_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ch_store(uint64_t* p, uint32_t tag, uint32_t payload) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct ChAbort {
    unsigned* err;
    unsigned* abort;
    uint32_t epoch;
};

// After a miss of a bounded wait that began at t0 (see qw_mlpstack.hip):
// false once it has run 0.2 s (error flag and abort word raised) or another
// wave of this launch has aborted.
__device__ __forceinline__ bool ch_pause(const ChAbort& ab, uint64_t t0, unsigned& it, bool& dead) {
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

// Bounded wait until the LDS word reaches `target`.
__device__ __forceinline__ void ch_wait_lds(unsigned* c, unsigned target, const ChAbort& ab, bool& dead) {
    uint64_t t0 = 0;
    unsigned it = 0;
    while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (dead) return;
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
    asm volatile("" ::: "memory");
}

template <int XDT>
__device__ __forceinline__ float ch_val(uint32_t h) {
    return XDT == DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}
template <int XDT>
__device__ __forceinline__ uint32_t ch_bits(float v) {
    return XDT == DT_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// Blocks of op `op` held by workgroup w: the r-th of the round robin, then
// every 256th; count 0 when r >= blocks.
__device__ __forceinline__ int ch_blocks_of(const ChainOp& op, int w, int& r) {
    r = (w - op.base) & (CH_GRID - 1);
    return r < op.n_blk ? (op.n_blk - r + CH_GRID - 1) / CH_GRID : 0;
}

// WF: BF16 (XDT BF16) or INT8 (XDT F16); MT: token count the registers hold.
template <int WF, int XDT, int MT>
__global__ __launch_bounds__(CH_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void chain_kernel(ChainArgs a) {
    constexpr int KE = WTraits<WF>::KE;
    constexpr int KS = 4 * KE;  // K per k-step
    constexpr int CH_PW = ch_pw(MT);
    extern __shared__ __attribute__((aligned(16))) uint8_t ch_raw[];
    ChLds& L = *reinterpret_cast<ChLds*>(ch_raw);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int wg = blockIdx.x;
    const int M = a.M;
    const uint32_t epoch = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool dead = false;
    // the launch at which the epoch field returns to 1 clears the slot words
    if ((epoch & CH_EFIELD) == 1u && epoch > CH_EFIELD) wrap_clear_words(a.words, a.n_words, a.epoch + 2, a.err, &L.cnt, dead);
    if (threadIdx.x < 2 * CH_NP) L.ready[threadIdx.x / CH_NP][threadIdx.x % CH_NP] = 0u;
    if (threadIdx.x == 0) {
        L.cnt = 0u;
        L.done = 0u;
    }
    {
        static_assert(sizeof(ChainOp) % 4 == 0, "op table copy");
        const uint32_t* src = reinterpret_cast<const uint32_t*>(a.ops);
        uint32_t* dst = reinterpret_cast<uint32_t*>(L.ops);
        const int n = a.n_ops * (int)(sizeof(ChainOp) / 4);
        for (int i = threadIdx.x; i < n; i += CH_NW * 64) dst[i] = src[i];
    }
    __syncthreads();  // the only workgroup barrier (besides the wrap clear's)
    const ChAbort ab{a.err, a.epoch + 1, epoch};

    if (wave < CH_NP) {
        // ============================ pollers ============================
        const int p = wave;
        // imports: this workgroup's share of every slot fed at launch start
        for (int s = 0; s < a.n_imports; ++s) {
            const ChainImport& im = a.imports[s];
            const int nw = M * im.words;  // words of the slot
            const int per = (nw + CH_GRID - 1) / CH_GRID;
            for (int i = wg * per + p * 64 + lane; i < min(nw, (wg + 1) * per); i += CH_NP * 64) {
                const int m = i / im.words, e = i - m * im.words;
                const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(im.src) +
                                                                      (size_t)m * im.ld + 2 * e);
                ch_store(im.words_ptr + i, ch_tag(epoch, 0), v);
            }
        }
        int q = 0;
        for (int o = 0; o < a.n_ops; ++o) {
            const ChainOp& op = L.ops[o];
            int r;
            const int nb = ch_blocks_of(op, wg, r);
            if (nb == 0) continue;
            const int par = q & 1;
            // --- input words of this poller: i = p*64 + lane + 256 n ---
            const uint32_t tg = ch_tag(epoch, op.in_tag);
            const int kw = op.K / 2;  // words per token
            const int nw = M * kw;
            uint32_t woff[CH_PW];     // word offset in the slot, or ~0 (none)
#pragma unroll
            for (int n = 0; n < CH_PW; ++n) {
                const int i = p * 64 + lane + CH_NP * 64 * n;
                const int m = i / kw, e = i - m * kw;
                woff[n] = i < nw ? (uint32_t)(m * op.in_ld + op.in_off / 2 + e) : ~0u;
            }
            float gm[CH_PW][2];
            if (op.gamma) {  // issued before the polls: static, they land first
#pragma unroll
                for (int n = 0; n < CH_PW; ++n) {
                    const int i = p * 64 + lane + CH_NP * 64 * n;
                    const int e = i % kw;
                    const bool ok = woff[n] != ~0u;
                    gm[n][0] = ok ? op.gamma[2 * e] : 0.0f;
                    gm[n][1] = ok ? op.gamma[2 * e + 1] : 0.0f;
                }
            }
            // residual rows (poller 0) and INT8 row scales (last poller) of the
            // blocks: issued ahead of the input polls (they were written by an
            // earlier op, or are static), checked after them
            const int rbl = lane >> 4, rm = (lane >> 3) & 1, re = lane & 7;  // block, token, word
            const bool rwant = p == 0 && op.residual && rbl < nb && rm < M;
            const uint32_t rtag = ch_tag(epoch, op.res_tag);
            const uint64_t* rptr = op.out_words + (size_t)rm * op.out_ld + (r + CH_GRID * rbl) * 8 + re;
            uint64_t rv = rwant ? ch_load(rptr) : 0;
            float scv[2] = {1.0f, 1.0f};
            if (p == CH_NP - 1 && op.scales) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int i = lane + 64 * h;
                    const int bl = i / 32, rt = (i / 16) & 1, row = i & 15;
                    const int pt = op.glu ? 2 * (r + CH_GRID * bl) + rt : r + CH_GRID * bl;
                    if (i < nb * 32 && (op.glu || rt == 0)) scv[h] = op.scales[pt * 16 + row];
                }
            }
            uint64_t v[CH_PW];
            {
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                unsigned it = 0;
                for (;;) {
                    bool ok = true;
#pragma unroll
                    for (int n = 0; n < CH_PW; ++n) {
                        if (woff[n] != ~0u) {
                            v[n] = ch_load(op.in_words + woff[n]);
                            ok = ok && (uint32_t)(v[n] >> 32) == tg;
                        }
                    }
                    if (__all(ok) || dead) break;
                    if (!ch_pause(ab, t0, it, dead)) break;
                }
            }
            if (a.trace && p == 0 && lane == 0) a.trace[((size_t)o * 4 + 0) * CH_GRID + wg] = __builtin_amdgcn_s_memrealtime();
            // deposit (times 1 + gamma, in the MFMA type) and the sums of squares
            float ss[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) ss[m] = 0.0f;
#pragma unroll
            for (int n = 0; n < CH_PW; ++n) {
                if (woff[n] != ~0u) {
                    const int i = p * 64 + lane + CH_NP * 64 * n;
                    const int m = i / kw, e = i - m * kw;
                    const uint32_t w2 = (uint32_t)v[n];
                    float x0 = ch_val<XDT>(w2 & 0xffffu), x1 = ch_val<XDT>(w2 >> 16);
                    const float q2 = x0 * x0 + x1 * x1;
#pragma unroll
                    for (int mm = 0; mm < MT; ++mm)
                        if (mm == m) ss[mm] += q2;
                    uint32_t out = w2;
                    if (op.gamma) {
                        x0 *= 1.0f + gm[n][0];
                        x1 *= 1.0f + gm[n][1];
                        out = ch_bits<XDT>(x0) | (ch_bits<XDT>(x1) << 16);
                    }
                    *reinterpret_cast<uint32_t*>(&L.xin[par][m][2 * e]) = out;
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) ss[m] += __shfl_xor(ss[m], off);
                if (lane == 0 && m < M) L.ss[par][p][m] = ss[m];
            }
            if (p == 0 && op.residual) {
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                unsigned it = 0;
                for (;;) {
                    const bool ok = !rwant || (uint32_t)(rv >> 32) == rtag;
                    if (__all(ok) || dead) break;
                    if (!ch_pause(ab, t0, it, dead)) break;
                    if (rwant) rv = ch_load(rptr);
                }
                if (rwant) {
                    L.res[par][rbl][rm][2 * re] = ch_val<XDT>((uint32_t)rv & 0xffffu);
                    L.res[par][rbl][rm][2 * re + 1] = ch_val<XDT>((uint32_t)rv >> 16);
                }
            }
            if (p == CH_NP - 1 && op.scales) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int i = lane + 64 * h;
                    if (i < nb * 32) L.sc[par][i / 32][(i / 16) & 1][i & 15] = scv[h];
                }
            }
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) __hip_atomic_store(&L.ready[par][p], (unsigned)(q + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            ++q;
        }
        // workgroup 0: once the last op's output is complete everywhere,
        // every workgroup has read the epoch: advance it
        if (wg == 0 && p == 0 && a.n_ops > 0) {
            const ChainOp& op = L.ops[a.n_ops - 1];
            const uint32_t tg = ch_tag(epoch, a.n_ops);
            const int nw = M * (op.N / 2);
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            unsigned it = 0;
            for (;;) {
                bool ok = true;
                for (int i = lane; i < nw; i += 64) {
                    const int m = i / (op.N / 2), e = i - m * (op.N / 2);
                    ok = ok && (uint32_t)(ch_load(op.out_words + (size_t)m * op.out_ld + e) >> 32) == tg;
                }
                if (__all(ok) || dead) break;
                if (!ch_pause(ab, t0, it, dead)) break;
            }
            if (lane == 0) __hip_atomic_store(a.epoch, ch_next_epoch(epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // ============================ compute waves ============================
    const int c = wave - CH_NP;
    constexpr int ULD = ChBuf<WF>::ULD, NBUF = ChBuf<WF>::NBUF;
    u32x4 A0[ULD], A1[NBUF == 2 ? ULD : 1];
    // this wave's units of op o: [u0, u1) of the workgroup's nb * ksteps
    auto range = [&](const ChainOp& op, int nb, int& u0, int& u1) {
        const int U = nb * op.ksteps;
        u0 = (c * U) / CH_CW;
        u1 = ((c + 1) * U) / CH_CW;
    };
    // always ULD loads (out-of-range slots read nothing), so the compiler can
    // count the loads in flight and wait for exactly the ones it consumes
    auto issue = [&](int o_req, auto& A) {
        const bool none = o_req >= a.n_ops;
        const int o = none ? a.n_ops - 1 : o_req;
        const ChainOp& op = L.ops[o];
        int r;
        const int nb = ch_blocks_of(op, wg, r);
        int u0, u1;
        range(op, nb, u0, u1);
        const int RT = op.glu ? 2 : 1;
        const int n_pt = op.glu ? 2 * op.n_blk : op.n_blk;
        const uint32_t tile_bytes = (uint32_t)op.ksteps * 1024u;
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(op.w, (uint32_t)((uint64_t)n_pt * tile_bytes));
#pragma unroll
        for (int i = 0; i < ULD; ++i) {
            const int u = u0 + (RT == 2 ? (i >> 1) : i);
            const int rt = RT == 2 ? (i & 1) : 0;
            uint32_t off = OOB;
            if (u < u1 && !none) {
                const int bl = u / op.ksteps, ks = u - bl * op.ksteps;
                const int blk = r + CH_GRID * bl;
                const int pt = op.glu ? 2 * blk + rt : blk;
                off = (uint32_t)pt * tile_bytes + (uint32_t)ks * 1024u + lane * 16;
            }
            A[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, AUX_NT));
        }
    };
    // the next op (after o) this workgroup takes part in, or n_ops
    auto next_op = [&](int o) {
        for (int o2 = o + 1; o2 < a.n_ops; ++o2) {
            int r;
            if (ch_blocks_of(L.ops[o2], wg, r) > 0) return o2;
        }
        return a.n_ops;
    };
    // one participation: op o (the q-th op this workgroup takes part in) with
    // its weights in A; `later` is the op whose weights A takes next
    auto step = [&](int o, int q, auto& A, int later) {
        const ChainOp& op = L.ops[o];
        int r;
        const int nb = ch_blocks_of(op, wg, r);
        int u0, u1;
        range(op, nb, u0, u1);
        const int par = q & 1;
        const int RT = op.glu ? 2 : 1;
        for (int p = 0; p < CH_NP; ++p) ch_wait_lds(&L.ready[par][p], (unsigned)(q + 1), ab, dead);
        if (a.trace && c == 0 && lane == 0) a.trace[((size_t)o * 4 + 1) * CH_GRID + wg] = __builtin_amdgcn_s_memrealtime();
        // partial tiles of (up to) two blocks: bl0 = u0 / ksteps and bl0 + 1
        const int bl0 = u0 / op.ksteps;
        f32x4 acc[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) acc[b][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const uint16_t* xb = &L.xin[par][0][0];
#pragma unroll
        for (int i = 0; i < ULD; ++i) {
            const int u = u0 + (RT == 2 ? (i >> 1) : i);
            const int rt = RT == 2 ? (i & 1) : 0;
            if (u < u1) {
                const int bl = u / op.ksteps, ks = u - bl * op.ksteps;
                const int k = ks * KS;
                BOps<WF, XDT> bo;
                const uint16_t* px = xb + (j < M ? j : 0) * CH_LROW + k + g * KE;
                if constexpr (WF == WF_BF16) {
                    u32x4 v = *reinterpret_cast<const u32x4*>(px);
                    if (j >= M) v = u32x4{0u, 0u, 0u, 0u};
                    bo.hi = __builtin_bit_cast(bf16x8, v);
                } else {
                    u32x4 v0 = reinterpret_cast<const u32x4*>(px)[0], v1 = reinterpret_cast<const u32x4*>(px)[1];
                    if (j >= M) v0 = v1 = u32x4{0u, 0u, 0u, 0u};
                    bo.hi0 = __builtin_bit_cast(f16x8, v0);
                    bo.hi1 = __builtin_bit_cast(f16x8, v1);
                }
                const f32x4 d = unit_mfma<WF, XDT>(A[i], bo, f32x4{0.f, 0.f, 0.f, 0.f});
                if (bl == bl0) {
                    if (rt == 0) acc[0][0] += d;
                    else acc[0][1] += d;
                } else {
                    if (rt == 0) acc[1][0] += d;
                    else acc[1][1] += d;
                }
            }
        }
        if (a.trace && lane == 0)  // the last compute wave's MFMAs
            __hip_atomic_fetch_max(&a.trace[((size_t)o * 4 + 2) * CH_GRID + wg], (uint64_t)__builtin_amdgcn_s_memrealtime(),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // partial tiles to LDS; the last wave to arrive runs the epilogue
        // every block of the workgroup gets this wave's partial (zero where
        // it has no units), so the epilogue sums all waves without branches
#pragma unroll
        for (int bl = 0; bl < CH_TW; ++bl) {
            if (bl < nb) {
                const bool mine0 = u1 > u0 && bl == bl0, mine1 = u1 > u0 && bl == bl0 + 1;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    if (rt < RT)
                        L.red[bl][c][rt][lane] = mine0 ? acc[0][rt] : (mine1 ? acc[1][rt] : f32x4{0.f, 0.f, 0.f, 0.f});
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&L.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __shfl(old, 0);
        if (old == CH_CW - 1) {
            if (lane == 0) __hip_atomic_store(&L.cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            float inv = 1.0f;
            if (op.norm) {
                const int jj = j < M ? j : 0;
                float sst = 0.0f;
#pragma unroll
                for (int p = 0; p < CH_NP; ++p) sst += L.ss[par][p][jj];
                inv = 1.0f / sqrtf(sst / (float)op.K + op.eps);
            }
            const uint32_t tg = ch_tag(epoch, o + 1);
            for (int bl = 0; bl < nb; ++bl) {
                f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
                // all waves' partials, in wave order
#pragma unroll
                for (int c2 = 0; c2 < CH_CW; ++c2) s[0] += L.red[bl][c2][0][lane];
                if (RT == 2) {
#pragma unroll
                    for (int c2 = 0; c2 < CH_CW; ++c2) s[1] += L.red[bl][c2][1][lane];
                }
                const int blk = r + CH_GRID * bl;
                const int o_row = blk * 16 + g * 4;  // first of this lane's 4 output rows
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (op.glu) {
                        const float gt = s[0][i] * inv * (op.scales ? L.sc[par][bl][0][g * 4 + i] : 1.0f);
                        const float up = s[1][i] * inv * (op.scales ? L.sc[par][bl][1][g * 4 + i] : 1.0f);
                        v[i] = silu_f(gt) * up;
                    } else {
                        v[i] = s[0][i] * inv * (op.scales ? L.sc[par][bl][0][g * 4 + i] : 1.0f);
                    }
                    if (op.residual) v[i] += L.res[par][bl][j < M ? j : 0][g * 4 + i];
                }
                if (j < M) {
                    uint32_t hb[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) hb[i] = ch_bits<XDT>(v[i]);
                    uint64_t* ow = op.out_words + (size_t)j * op.out_ld + o_row / 2;
                    ch_store(ow, tg, hb[0] | (hb[1] << 16));
                    ch_store(ow + 1, tg, hb[2] | (hb[3] << 16));
                    if (op.exp) {
                        uint32_t* ew = reinterpret_cast<uint32_t*>(op.exp + (size_t)j * op.exp_ld + o_row);
                        ew[0] = hb[0] | (hb[1] << 16);
                        ew[1] = hb[2] | (hb[3] << 16);
                    }
                }
            }
            if (a.trace && lane == 0) a.trace[((size_t)o * 4 + 3) * CH_GRID + wg] = __builtin_amdgcn_s_memrealtime();
            if (lane == 0) __hip_atomic_store(&L.done, (unsigned)(q + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
            ch_wait_lds(&L.done, (unsigned)(q + 1), ab, dead);
        }
        issue(later, A);  // its weights stream during the hand-offs
    };
    int o = next_op(-1);
    int o1 = next_op(o);
    issue(o, A0);
    if constexpr (NBUF == 2) issue(o1, A1);
    for (int q = 0; o < a.n_ops;) {
        const int o2 = next_op(o1);
        step(o, q++, A0, NBUF == 2 ? o2 : o1);
        o = o1;
        o1 = o2;
        if (o >= a.n_ops) break;
        const int o3 = next_op(o1);
        if constexpr (NBUF == 2) step(o, q++, A1, o3);
        else step(o, q++, A0, o1);
        o = o1;
        o1 = o3;
    }
}

template <typename Kern>
static hipError_t launch_ch(Kern k, const ChainArgs& a, hipStream_t st) {
    constexpr size_t lds = sizeof(ChLds);
    static_assert(sizeof(ChLds) <= 160 * 1024, "LDS layout");
    {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(CH_GRID), dim3(CH_NW * 64), lds, st, a);
    return hipGetLastError();
}

int chain_grid() { return CH_GRID; }
int chain_max_m() { return CH_MAXM; }
int chain_max_blocks() { return CH_TW * CH_GRID; }
int chain_max_loads(int wf) { return wf == WF_I8 ? ChBuf<WF_I8>::ULD : ChBuf<WF_BF16>::ULD; }
int chain_compute_waves() { return CH_CW; }

hipError_t launch_chain(const ChainArgs& a, int wf, int xdt, hipStream_t stream) {
    if (a.M < 1 || a.M > CH_MAXM || a.n_imports > kChainMaxImports || a.n_ops > kChainMaxOps)
        return hipErrorInvalidValue;
    if (wf == WF_BF16 && xdt == DT_BF16) {
        if (a.M == 1) return launch_ch(chain_kernel<WF_BF16, DT_BF16, 1>, a, stream);
        return launch_ch(chain_kernel<WF_BF16, DT_BF16, 2>, a, stream);
    }
    if (wf == WF_I8 && xdt == DT_F16) {
        if (a.M == 1) return launch_ch(chain_kernel<WF_I8, DT_F16, 1>, a, stream);
        return launch_ch(chain_kernel<WF_I8, DT_F16, 2>, a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace qwk
