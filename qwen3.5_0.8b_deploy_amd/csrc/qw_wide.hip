// qw_wide.hip -- weight-stationary projection kernel for 17..256 tokens
// (decode at larger batches, short prefill chunks) on gfx950.
//
// Every weight byte is read from HBM exactly once per launch, for all M
// tokens: a wave holds a block of two 16-row tiles (a gate/up pair for GLU
// weights) of one K range in MFMA A registers, and runs them against every
// token tile of the activations, which sit in LDS.  The tokens are the MFMA
// N side (16 per tile, up to 8 tiles), so the weights are the stationary
// operand and the activations are re-read from LDS, not from HBM.  More than
// 128 tokens run as token groups of at most 128 (workgroups of their own,
// the weights then come from L2 for the later groups).
//
// Work decomposition.  K is cut into S splits so that the activation slice
// [M][K/S] of a split fits the workgroup's LDS.  A workgroup is one split of
// NB blocks; its NB x KW waves split the split's K range KW ways per block.
// The grid is (blocks / NB) x S workgroups, sized on the host to fill the
// CUs once (one workgroup per CU; no grid-stride loop), and workgroup w
// takes split w % S, so the workgroups of one XCD (w % 8) share one
// activation slice in their L2.
//
// Data flow of a workgroup.
//   1. Direct-to-LDS loads (buffer_load_dwordx4 ... lds, no VGPRs) bring the
//      activation slice in MFMA B-operand order: one 1 KB unit per (k-step,
//      token tile) in which lane l = r + 16 g holds the 8 k of token r the
//      MFMA reads from that lane.  The RMSNorm weight slice, the INT8 row
//      scales and the residual rows of the epilogue come the same way.
//   2. The weight k-steps of the wave are issued next (up to U per wave in
//      flight, unconditionally; unused slots read out of range), so the
//      small loads above are ahead of them in the in-order vector-memory
//      counter: one s_waitcnt vmcnt(U*RT) and a barrier publish them.
//   3. MFMAs (16x16x32 bf16, or f16 on exactly converted INT8 units), each
//      weight unit against all token tiles, the B operands read one k-step
//      ahead; further weight chunks are issued after a chunk is consumed.
//   4. RMSNorm prologue (when asked), inside the MFMA stream: the per-token
//      sums of squares are the diagonal of X X^T (one more MFMA per token
//      tile and k-step), and (1 + gamma) scales the weight operand, so the
//      staged activations are used as they are.
//   5. The KW partial tiles of a block meet in LDS (fixed order); the split
//      partials meet through a workspace region whose words hold a sentinel
//      between launches: splits 0..S-2 store theirs (device-coherent, sc1),
//      split S-1 polls them until no word is the sentinel, sums the S
//      partials in split order (deterministic), writes the sentinel back
//      (graph-safe, no memset) and runs the epilogue, spread over its waves.
//   6. Epilogue: 1/rms, INT8 row scale, SiLU(gate)*up, residual, Q/gate
//      de-interleave, 4-wide stores.
//
// Reference operators replaced at these token counts: the grid (N, M)
// int8_gemv_batch_kernel (mlp_cuda.cu:158-180), which reads every weight row
// once per token, and the cuBLAS GemmEx / SGEMM calls of the batch forward
// paths (bf16_gemm.cuh:89, cublas_utils.cuh:60-83).
#include "qw_stream.hpp"

namespace qwk {

constexpr int kWideMaxS = 8;  // K splits per launch: the finishing wave loads all of them at once

template <int WF> struct WideT {
    static constexpr int KS = 4 * WTraits<WF>::KE;  // K elements per k-step
    static constexpr int XU = WF == WF_I8 ? 2 : 1;  // LDS units per (k-step, token tile)
    static constexpr int KEW = WTraits<WF>::KE;     // K elements per lane group of a k-step
};

// Residual region of a block's output tile: [CT*16 tokens][16 rows] elements
// of rs bytes, in 1 KB units of 32 (rs = 2) or 16 (rs = 4) tokens.
__device__ __forceinline__ int res_units(int CT, int rs) { return CT * rs / 4; }

template <int WF, int XDT, int CT, bool GLU, bool NORM, int NB, int KW, int U>
__global__ __launch_bounds__(NB * KW * 64) void wide_kernel(WideArgs wa) {
    constexpr int NW = NB * KW;
    constexpr int RT = 2;                 // physical tiles per block
    constexpr int RO = GLU ? 1 : 2;       // output tiles per block
    constexpr int KS = WideT<WF>::KS, XU = WideT<WF>::XU, KEW = WideT<WF>::KEW;
    static_assert(WF == WF_BF16 || WF == WF_I8, "16-bit MFMA weight formats only");
    static_assert((WF == WF_BF16 && XDT == DT_BF16) || (WF == WF_I8 && XDT == DT_F16),
                  "activations arrive in the MFMA input type");
    const SkinnyArgs& a = wa.s;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float ss_part[KW][CT * 16];  // sums of squares of each K part of the split

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int S = a.S;
    // workgroup -> (block group bg, token group t, split s); the T token
    // groups of a block group sit 8 workgroups apart, i.e. on one XCD, where
    // the later ones find its weights in L2
    const int T = wa.T;
    const int s = (int)blockIdx.x % S;
    const int q = (int)blockIdx.x / S;
    const int t = T > 1 ? (q / 8) % T : 0;
    const int bg = T > 1 ? (q % 8) + 8 * (q / (8 * T)) : q;
    const int M0 = t * wa.Mg;                 // this workgroup's tokens [M0, M0 + Mt)
    const int Mt = min(wa.Mg, a.M - M0);
    const int cgrp = bg * T + t;              // counter / partials group
    const int bl = wave / KW, kw = wave % KW;
    const int blk = bg * NB + bl;
    const bool blk_ok = blk < wa.nblocks;
    constexpr bool norm = NORM;  // the host sets NORM exactly when the call asks for EP_NORM
    const bool gam = NORM && a.gamma != nullptr;
    const bool want_res = (a.flags & EP_RESIDUAL) != 0;

    // this workgroup's split [ks0, ks1) and the wave's part [kb, kend)
    const int ks0 = (s * a.ksteps) / S, ks1 = ((s + 1) * a.ksteps) / S;
    const int nks = ks1 - ks0;
    const int kb0 = ks0 + (kw * nks) / KW, kend = ks0 + ((kw + 1) * nks) / KW;

    // ---- 1. small operands, direct to LDS ----
    const int xunits = CT * nks * XU;
    uint8_t* const xl = lds;
    uint8_t* const gl = lds + wa.off_gamma;
    uint8_t* const rl = lds + wa.off_res;
    uint8_t* const sl = lds + wa.off_scales;
    {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2));
        for (int u = wave; u < ((wa.dbg & 4) ? 0 : xunits); u += NW) {
            const int h = u % XU, t = u / XU;
            const int ct = t % CT, ksr = t / CT;
            const int m = ct * 16 + r;
            const int k = (ks0 + ksr) * KS + g * KEW + h * 8;
            lds_dma16(xr, xl + u * 1024, m < Mt ? (uint32_t)(((M0 + m) * a.ldx + k) * 2) : OOB);
        }
        if (gam) {
            const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.gamma, (uint32_t)a.K * 4u);
            const int gunits = (nks * KS * 4 + 1023) / 1024;
            for (int u = wave; u < gunits; u += NW) {
                const int k = ks0 * KS + u * 256 + lane * 4;
                lds_dma16(gr, gl + u * 1024, k < ks1 * KS ? (uint32_t)(k * 4) : OOB);
            }
        }
        if (wa.res_lds && want_res) {
            // residual rows of the block's output tiles: [token][16 rows]
            const int rs = a.res_dt == DT_F32 ? 4 : 2;
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, (uint32_t)((uint64_t)a.M * a.ld_res * rs));
            const int per = res_units(CT, rs);
            for (int u = wave; u < NB * RO * per; u += NW) {
                const int bt = u / per, j = u % per;  // bt = block-in-group * RO + output tile
                const int b2 = bg * NB + bt / RO;
                const int row0 = (GLU ? b2 : b2 * 2 + bt % RO) * 16;
                const int tpu = 1024 / (16 * rs);  // tokens per unit: 32 (16-bit) or 16 (FP32)
                const int lpt = 64 / tpu;          // lanes per token, 16 / lpt rows each
                const int tok = j * tpu + lane / lpt;
                const int rofs = (lane % lpt) * (16 / lpt);
                const bool ok = b2 < wa.nblocks && tok < Mt && row0 < a.N;
                lds_dma16(rr, rl + u * 1024,
                          ok ? (uint32_t)(((int64_t)(M0 + tok) * a.ld_res + row0 + rofs) * rs) : OOB);
            }
        }
        if (a.scales) {
            const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.scales, (uint32_t)wa.n_ptiles * 64u);
            for (int u = wave; u < NB; u += NW) {
                const int b2 = bg * NB + u;
                lds_dma16(sr, sl + u * 1024, lane < 8 && b2 < wa.nblocks ? (uint32_t)((b2 * 32 + lane * 4) * 4) : OOB);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weights: the first chunk of this wave's k-steps ----
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)wa.n_ptiles * a.ksteps * 1024u));
    const uint32_t tile_bytes = (uint32_t)a.ksteps * 1024u;
    uint32_t tbase[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int pt = blk * 2 + rt;
        tbase[rt] = blk_ok && pt < wa.n_ptiles ? (uint32_t)pt * tile_bytes + lane * 16 : OOB;
    }
    u32x4 A[U][RT];
    auto issue = [&](int k0, int n) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                A[u][rt] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               wrs, (u < n && tbase[rt] != OOB) ? tbase[rt] + (uint32_t)(k0 + u) * 1024u : OOB, 0,
                               AUX_NT));
    };
    int kb = kb0;
    int n = min(U, kend - kb);
    issue(kb, n);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vm_wait(U * RT));  // everything issued before the weights has landed
    __syncthreads();

    // ---- 3. MFMAs (and the RMSNorm prologue) ----
    f32x4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    // B operands (one 16-byte LDS read per token tile and unit) of a k-step
    // are read one k-step ahead, so their LDS latency hides under the MFMAs
    // of the previous k-step.
    u32x4 B[2][CT][XU];
    auto read_b = [&](int buf, int ksr) {
        const uint8_t* xp = xl + (ksr * CT * XU) * 1024 + lane * 16;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int h = 0; h < XU; ++h) B[buf][ct][h] = *reinterpret_cast<const u32x4*>(xp + (ct * XU + h) * 1024);
    };
    // RMSNorm prologue inside the MFMA stream: the sums of squares of the
    // tokens are the diagonal of X X^T, one extra MFMA per token tile and
    // k-step on the B operands already in registers (the block-0 waves of
    // the workgroup take them); (1 + gamma) scales the weight operand of the
    // k-step (A), so the staged activations are used as they are.
    f32x4 accss[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) accss[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool do_ss = NORM && bl == 0;
    auto mma = [&](int u, int buf, int ksr) {
        if constexpr (WF == WF_BF16) {
            u32x4 av[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) av[rt] = A[u][rt];
            if (gam) {
                const float* gp = reinterpret_cast<const float*>(gl) + ksr * KS + g * KEW;
                const f32x4 g0 = reinterpret_cast<const f32x4*>(gp)[0];
                const f32x4 g1 = reinterpret_cast<const f32x4*>(gp)[1];
                float gs[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    gs[e] = 1.0f + g0[e];
                    gs[e + 4] = 1.0f + g1[e];
                }
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int q2 = 0; q2 < 4; ++q2) {
                        const uint32_t w = av[rt][q2];
                        const float lo = bf16_bits_to_f32(w & 0xffffu) * gs[2 * q2];
                        const float hi = bf16_bits_to_f32(w >> 16) * gs[2 * q2 + 1];
                        av[rt][q2] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
                    }
            }
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const bf16x8 b = __builtin_bit_cast(bf16x8, B[buf][ct][0]);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = mfma_bf16(__builtin_bit_cast(bf16x8, av[rt]), b, acc[rt][ct]);
                if (do_ss) accss[ct] = mfma_bf16(b, b, accss[ct]);
            }
        } else {
            f16x8 a0[RT], a1[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) i8unit_to_f16(A[u][rt], a0[rt], a1[rt]);
            if (gam) {
                // (1 + gamma) as f16, multiplied into the exact f16 weights
                const float* gp = reinterpret_cast<const float*>(gl) + ksr * KS + g * KEW;
                f16x8 gs0, gs1;
#pragma unroll
                for (int e4 = 0; e4 < 2; ++e4) {
                    const f32x4 v0 = reinterpret_cast<const f32x4*>(gp)[e4];
                    const f32x4 v1 = reinterpret_cast<const f32x4*>(gp)[e4 + 2];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gs0[e4 * 4 + e] = (_Float16)(1.0f + v0[e]);
                        gs1[e4 * 4 + e] = (_Float16)(1.0f + v1[e]);
                    }
                }
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    a0[rt] = a0[rt] * gs0;
                    a1[rt] = a1[rt] * gs1;
                }
            }
            // the first half-unit's MFMAs of every tile, then the second's
            // (each accumulator sums in the same order, with the other tiles'
            // independent MFMAs between its two)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const f16x8 b0 = __builtin_bit_cast(f16x8, B[buf][ct][0]);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = mfma_f16(a0[rt], b0, acc[rt][ct]);
                if (do_ss) accss[ct] = mfma_f16(b0, b0, accss[ct]);
            }
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const f16x8 b1 = __builtin_bit_cast(f16x8, B[buf][ct][1]);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = mfma_f16(a1[rt], b1, acc[rt][ct]);
                if (do_ss) accss[ct] = mfma_f16(b1, b1, accss[ct]);
            }
        }
    };
    if (kb < kend) read_b(0, kb - ks0);
    for (;;) {
        if (wa.dbg & 1) {
        } else if (n == U) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u + 1 < U || kb + U < kend) read_b((u + 1) & 1, kb + u + 1 - ks0);
                mma(u, u & 1, kb + u - ks0);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u < n) {
                    if (u + 1 < n) read_b((u + 1) & 1, kb + u + 1 - ks0);
                    mma(u, u & 1, kb + u - ks0);
                }
            }
        }
        kb += n;
        if (kb >= kend) break;
        n = min(U, kend - kb);
        issue(kb, n);
    }

    if (do_ss) {
        // diagonal of the 16x16 tile: token r sits in lane (r, r / 4), element r % 4
        if (g == (r >> 2)) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const f32x4 v = accss[ct];
                const int e = r & 3;
                ss_part[kw][ct * 16 + r] = e == 0 ? v[0] : (e == 1 ? v[1] : (e == 2 ? v[2] : v[3]));
            }
        }
    }

    // ---- 5. reduction over the KW parts and the S splits ----
    // The workgroup's output is NB blocks x CT token tiles ("units", each
    // both physical tiles of a block for one token tile).  Every wave writes
    // its accumulators to LDS (over the activations), then wave w owns units
    // w, w + NW, ...: it sums their KW parts in a fixed order and, with S > 1,
    // hands them over through the workspace.  The workgroup of the last
    // split of a block group collects the other S - 1 partials of its units,
    // sums the S in split order and runs their epilogue, so the epilogue is
    // spread over all its waves.
    constexpr int NU = NB * CT;                 // units per workgroup
    constexpr int UPW = (NU + NW - 1) / NW;     // units per wave (upper bound)
    __syncthreads();                            // every wave is done with the activations
    {
        f32x4* red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) red[(((bl * KW + kw) * RT + rt) * CT + ct) * 64 + lane] = acc[rt][ct];
    }
    __syncthreads();
    f32x4 u_acc[UPW][RT];
    float u_ss[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        const int u = wave + i * NW;
        const int ub = u / CT, uc = u % CT;
        const f32x4* red = reinterpret_cast<const f32x4*>(lds);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
            if (u < NU) {
#pragma unroll
                for (int k2 = 0; k2 < KW; ++k2) v += red[(((ub * KW + k2) * RT + rt) * CT + uc) * 64 + lane];
            }
            u_acc[i][rt] = v;
        }
        float sq = 0.0f;
        if (norm && u < NU) {
#pragma unroll
            for (int pp = 0; pp < KW; ++pp) sq += ss_part[pp][uc * 16 + r];
        }
        u_ss[i] = sq;
    }

    if (S > 1 && !(wa.dbg & 2)) {
        // Split-K hand-off without counters: the partials region holds
        // kWideSentinel in every word between launches.  Splits 0..S-2 store
        // their partials (device-coherent, sc1) and are done; split S-1, the
        // finisher, polls each partner's words until none holds the sentinel
        // (each 32-bit word is written whole), sums the S partials in split
        // order -- its own from registers, the same values the others'
        // stores carry, so the sum is the one the arrival-count hand-off
        // formed -- and writes the sentinel back.  One memory round trip
        // after the last partner's stores, instead of store completion, an
        // arrival count and the reloads.
        // Layout: [group][split][unit][lane] RT x 16 bytes, then the sums of
        // squares [group][split][unit][lane] x 4 bytes.
        const int ngrp = wa.ngrp * T;
        const uint64_t vbytes = (uint64_t)ngrp * S * NU * 64 * RT * 16;
        const uint64_t pbytes = vbytes + (uint64_t)ngrp * S * NU * 64 * 4;
        const __amdgpu_buffer_rsrc_t prs = make_rsrc(wa.wpart, (uint32_t)min(pbytes, (uint64_t)0x7fffffff));
        auto voff = [&](int s2, int u, int rt) {
            return (uint32_t)(((((uint64_t)cgrp * S + s2) * NU + u) * 64 + lane) * RT + rt) * 16u;
        };
        auto soff = [&](int s2, int u) {
            return (uint32_t)(vbytes + ((((uint64_t)cgrp * S + s2) * NU + u) * 64 + lane) * 4u);
        };
        auto canon = [](float v) {
            const uint32_t b = __float_as_uint(v);
            return b == kWideSentinel ? 0x7fc00000u : b;
        };
        const int fin = S - 1;
        if (s != fin) {
#pragma unroll
            for (int i = 0; i < UPW; ++i) {
                const int u = wave + i * NW;
                if (u < NU) {
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const f32x4 v = u_acc[i][rt];
                        __builtin_amdgcn_raw_buffer_store_b128(u32x4{canon(v[0]), canon(v[1]), canon(v[2]), canon(v[3])},
                                                               prs, voff(s, u, rt), 0, AUX_SC1);
                    }
                    if (norm) __builtin_amdgcn_raw_buffer_store_b32(canon(u_ss[i]), prs, soff(s, u), 0, AUX_SC1);
                }
            }
            return;
        }
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll
        for (int i = 0; i < UPW; ++i) {
            const int u = wave + i * NW;
            if (u >= NU) continue;
            f32x4 pv[kWideMaxS][RT];
            float ps[kWideMaxS];
            // every partner's words in flight at once, reloaded until all arrived
            for (unsigned it = 0;; ++it) {
                bool ok = true;
#pragma unroll
                for (int s2 = 0; s2 < kWideMaxS; ++s2) {
                    if (s2 < fin) {
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) {
                            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(prs, voff(s2, u, rt), 0, AUX_SC1);
                            ok = ok && w[0] != kWideSentinel && w[1] != kWideSentinel && w[2] != kWideSentinel &&
                                 w[3] != kWideSentinel;
                            pv[s2][rt] = __builtin_bit_cast(f32x4, w);
                        }
                        if (norm) {
                            const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(prs, soff(s2, u), 0, AUX_SC1);
                            ok = ok && w != kWideSentinel;
                            ps[s2] = __uint_as_float(w);
                        } else {
                            ps[s2] = 0.0f;
                        }
                    }
                }
                if (__all(ok)) break;
                // bounded wait (0.2 s of the 100 MHz clock): a partial that
                // never arrives raises the error flag instead of hanging
                if ((it & 63u) == 63u && __builtin_amdgcn_s_memrealtime() - t0 > 20000000ull) {
                    __hip_atomic_store(wa.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            // the S partials summed in split order, the finisher's own last
            f32x4 own[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                own[rt] = u_acc[i][rt];
                u_acc[i][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            const float own_ss = u_ss[i];
            u_ss[i] = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < kWideMaxS; ++s2) {
                if (s2 < fin) {
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) u_acc[i][rt] += pv[s2][rt];
                    u_ss[i] += ps[s2];
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) u_acc[i][rt] += own[rt];
            u_ss[i] += own_ss;
            // the partners' words emptied for the next launch
            const u32x4 e4 = u32x4{kWideSentinel, kWideSentinel, kWideSentinel, kWideSentinel};
#pragma unroll
            for (int s2 = 0; s2 < kWideMaxS; ++s2) {
                if (s2 < fin) {
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        __builtin_amdgcn_raw_buffer_store_b128(e4, prs, voff(s2, u, rt), 0, AUX_SC1);
                    if (norm) __builtin_amdgcn_raw_buffer_store_b32(kWideSentinel, prs, soff(s2, u), 0, AUX_SC1);
                }
            }
        }
    }

    // ---- 6. epilogue of this wave's units ----
    const int rs = a.res_dt == DT_F32 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        const int u = wave + i * NW;
        if (u >= NU) continue;
        const int ub = u / CT, ct = u % CT;
        const int blk2 = bg * NB + ub;
        const int m = ct * 16 + r;
        if (blk2 >= wa.nblocks || m >= Mt) continue;
        const float inv = norm ? 1.0f / sqrtf(u_ss[i] / (float)a.K + a.eps) : 1.0f;
        f32x4 sc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            sc[rt] = a.scales ? *reinterpret_cast<const f32x4*>(sl + ub * 1024 + (rt * 16 + g * 4) * 4)
                              : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int ro = 0; ro < RO; ++ro) {
            const int tile = GLU ? blk2 : blk2 * 2 + ro;
            const int o = tile * 16 + g * 4;
            if (o >= a.N) continue;
            f32x4 v;
            if constexpr (GLU) {
                const f32x4 gt = u_acc[i][0] * inv * sc[0];
                const f32x4 up = u_acc[i][1] * inv * sc[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = silu_f(gt[e]) * up[e];
            } else {
                v = u_acc[i][ro] * inv * sc[ro];
            }
            if (a.vec_store) {
                if (want_res) {
                    const uint8_t* rp = rl + (ub * RO + ro) * res_units(CT, rs) * 1024 + (m * 16 + g * 4) * rs;
                    if (rs == 4) {
                        v += *reinterpret_cast<const f32x4*>(rp);
                    } else {
                        const u32x2 w = *reinterpret_cast<const u32x2*>(rp);
                        v += epi_res(a.res_dt, u32x4{0u, 0u, 0u, 0u}, w);
                    }
                }
                void* dst = a.y;
                int col = o;
                if (a.flags & EP_SPLIT) {
                    const int sb = o / a.split_period;
                    dst = (sb & 1) ? a.y2 : a.y;
                    col = (sb >> 1) * a.split_period + (o - sb * a.split_period);
                }
                store_act4(dst, a.ydt, (int64_t)(M0 + m) * a.ldy + col, v);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int oi = o + e;
                    if (oi >= a.N) break;
                    float vi = v[e];
                    if (want_res) vi += load_act(a.res, a.res_dt, (int64_t)(M0 + m) * a.ld_res + oi);
                    void* dst = a.y;
                    int col = oi;
                    if (a.flags & EP_SPLIT) {
                        const int sb = oi / a.split_period;
                        dst = (sb & 1) ? a.y2 : a.y;
                        col = (sb >> 1) * a.split_period + (oi - sb * a.split_period);
                    }
                    store_act(dst, a.ydt, (int64_t)(M0 + m) * a.ldy + col, vi);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Tied lm_head with the fused greedy argmax at 17..256 tokens.
//
// The same weight-stationary idea for a weight far larger than the grid: the
// activations of a token group (at most 64 tokens) are staged once per
// workgroup (direct-to-LDS, B-operand order), and each of its four waves walks 32-row
// blocks of E (grid stride over all workgroups of its token group) in
// chunks of 8 k-steps, two chunks in flight (the loads of chunk s+2 are
// issued as chunk s is consumed; they are unconditional, so the compiler
// counts them and waits for exactly the chunk it uses).  A block's logits
// never leave the registers: each lane keeps, per token tile, the running
// maximum of the orderable key (logit, ~row) -- ties go to the lowest row.
// At the end the waves' keys meet in LDS, one 64-bit atomic max per
// token and workgroup merges the grid, and the last workgroup (completion
// counter) decodes the keys into ids and returns keys and counter to zero.
// Replaces lm_head_gemv_kernel_optimized + block_argmax_kernel
// (lm_head_cuda.cu:38-99, gpu_sampler_argmax.cu:14-43) at these batches.
// ---------------------------------------------------------------------------
constexpr int kArgU = 8;  // k-steps per chunk

constexpr int kArgNW = 4;  // waves per workgroup at up to 32 tokens per group (eight measured slower: 92 vs 86 us BF16 at 32 tokens)

template <int WF, int XDT, int CT, int NW, int WAUX, int U = kArgU, int NCH = 2>
__global__ __launch_bounds__(NW * 64) void wide_argmax_kernel(WideArgmaxArgs a) {
    constexpr int RT = 2;
    constexpr int KS = WideT<WF>::KS, XU = WideT<WF>::XU, KEW = WideT<WF>::KEW;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ unsigned long long kbest[NW][CT * 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int T = a.T;
    const int b = (int)blockIdx.x;
    const int t = (b / 8) % T;                       // token group (8 workgroups apart: one XCD)
    const int gi = (b % 8) + 8 * (b / (8 * T));      // workgroup within the token group
    const int Gt = (int)gridDim.x / T;
    const int M0 = t * a.Mg, Mt = min(a.Mg, a.M - M0);
    const int nch = a.ksteps / U;                    // chunks per block
    const int gw = gi * NW + wave, stride = Gt * NW;
    const int nblk_w = gw < a.n_blk ? (a.n_blk - gw + stride - 1) / stride : 0;
    const int nseq = nblk_w * nch;

    // ---- activations of the token group -> LDS (issued before the weights) ----
    {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2));
        const int xunits = CT * a.ksteps * XU;
        for (int u = wave; u < xunits; u += NW) {
            const int h = u % XU, q = u / XU;
            const int ct = q % CT, ks = q / CT;
            const int m = ct * 16 + r;
            const int k = ks * KS + g * KEW + h * 8;
            lds_dma16(xr, lds + u * 1024, m < Mt ? (uint32_t)(((M0 + m) * a.ldx + k) * 2) : OOB);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    const uint32_t tile_bytes = (uint32_t)a.ksteps * 1024u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_tiles * tile_bytes));
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.scales ? (const void*)a.scales : a.x,
                                                 a.scales ? (uint32_t)a.n_tiles * 64u : 0u);
    u32x4 AR[NCH][U][RT];  // a ring of NCH chunks in flight
    u32x4 SR[NCH][RT];
    // The wave's chunks in order: block gw + i * stride, k-steps from c * U
    // (c < nch), walked by a cursor (no division).  Loads are unconditional
    // and branch-free: blocks past the end lie beyond the descriptors' ranges
    // and read zeros, so every chunk issues the same loads and the compiler
    // waits for exactly the chunk a body consumes.  The row scales come with
    // every chunk (one 16-byte load per tile, used at a block's first chunk).
    int ib = gw, ic = 0;  // issue cursor
    auto issue = [&](auto& A, auto& S) {
        const uint32_t kb = (uint32_t)ic * U * 1024u + lane * 16;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint32_t pt = 2u * (uint32_t)ib + rt;
#pragma unroll
            for (int u = 0; u < U; ++u)
                A[u][rt] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, pt * tile_bytes + kb + (uint32_t)u * 1024u, 0, WAUX));
            S[rt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (pt * 16 + g * 4) * 4, 0, 0));
        }
        if (++ic == nch) {
            ic = 0;
            ib += stride;
        }
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) issue(AR[c], SR[c]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vm_wait(NCH * RT * (U + 1)));  // the activations have landed
    __syncthreads();
    if constexpr (WF == WF_I8 && XDT == DT_BF16) {
        // BF16 activations for the f16 MFMA of INT8 weights: converted once in
        // LDS (exact in the f16 normal range)
        uint32_t* xw = reinterpret_cast<uint32_t*>(lds);
        const int nwords = CT * a.ksteps * XU * 256;
        for (int i = threadIdx.x; i < nwords; i += NW * 64) {
            const uint32_t v = xw[i];
            xw[i] = f32_to_f16_bits(bf16_bits_to_f32(v & 0xffffu)) | (f32_to_f16_bits(bf16_bits_to_f32(v >> 16)) << 16);
        }
        __syncthreads();
    }

    f32x4 acc[RT][CT];
    f32x4 sc[RT];
    // per token tile: this lane's running maximum and its row.  A lane visits
    // its rows in increasing order, so the strict compare keeps the lowest
    // row of a tie; the keys are formed once, at the end.
    float bv[CT];
    uint32_t bi[CT];
    unsigned long long best[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        bv[ct] = -__builtin_inff();
        bi[ct] = 0xffffffffu;
        best[ct] = 0ull;
    }
    int bb = gw, bc = 0;  // body cursor
    u32x4 Bn[CT][XU];     // B fragments of the next k-step
    auto read_bn = [&](int ks) {
        const uint8_t* xp = lds + (ks * CT * XU) * 1024 + lane * 16;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int h = 0; h < XU; ++h) Bn[ct][h] = *reinterpret_cast<const u32x4*>(xp + (ct * XU + h) * 1024);
    };
    read_bn(0);
    auto body = [&](int s, auto& A, auto& S) {
        const int c = bc, blk = bb;
        if (++bc == nch) {
            bc = 0;
            bb += stride;
        }
        if (a.dbg & 1) {  // timing probe: the weight stream alone
            if (c == nch - 1) best[0] = max(best[0], (unsigned long long)A[0][0][0] + A[U - 1][1][3]);
            return;
        }
        if (c == 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                sc[rt] = a.scales ? as_f32x4(S[rt]) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // this k-step's B fragments were read during the previous one;
            // the next k-step's (the next chunk's or block's first past the
            // end of this one) are read now, under these MFMAs
            const int ks = c * U + u;
            u32x4 Bc[CT][XU];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int h = 0; h < XU; ++h) Bc[ct][h] = Bn[ct][h];
            read_bn(ks + 1 == a.ksteps ? 0 : ks + 1);
            if constexpr (WF == WF_BF16) {
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const bf16x8 bb = __builtin_bit_cast(bf16x8, Bc[ct][0]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[rt][ct] = mfma_bf16(__builtin_bit_cast(bf16x8, A[u][rt]), bb, acc[rt][ct]);
                }
            } else {
                f16x8 a0[RT], a1[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) i8unit_to_f16(A[u][rt], a0[rt], a1[rt]);
                // the first half-unit's MFMAs of every tile, then the second's:
                // RT * CT independent MFMAs between the two of each accumulator
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const f16x8 b0 = __builtin_bit_cast(f16x8, Bc[ct][0]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = mfma_f16(a0[rt], b0, acc[rt][ct]);
                }
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const f16x8 b1 = __builtin_bit_cast(f16x8, Bc[ct][1]);
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = mfma_f16(a1[rt], b1, acc[rt][ct]);
                }
            }
        }
        if (c == nch - 1 && s < nseq) {  // the block's logits: into the running maxima
            const int row0 = blk * 32 + g * 4;
            if (blk * 32 + 32 <= a.V) {  // every row of the block is a vocabulary row
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const f32x4 v = acc[rt][ct] * sc[rt];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const bool gt = v[e] > bv[ct];
                            bv[ct] = gt ? v[e] : bv[ct];
                            bi[ct] = gt ? (uint32_t)(row0 + rt * 16 + e) : bi[ct];
                        }
                    }
            } else {
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const f32x4 v = acc[rt][ct] * sc[rt];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int row = row0 + rt * 16 + e;
                            const bool gt = row < a.V && v[e] > bv[ct];
                            bv[ct] = gt ? v[e] : bv[ct];
                            bi[ct] = gt ? (uint32_t)row : bi[ct];
                        }
                    }
            }
        }
    };
    for (int s = 0; s < nseq; s += NCH) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            body(s + c, AR[c], SR[c]);  // past nseq: zeros, no key update
            issue(AR[c], SR[c]);
        }
    }

    // ---- keys: the four row groups of a lane's token, the waves, the grid ----
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
        if (bi[ct] != 0xffffffffu && ct * 16 + r < Mt) best[ct] = argmax_key(bv[ct], bi[ct]);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int sh = 16; sh <= 32; sh <<= 1) {
            const unsigned long long o = __shfl_xor(best[ct], sh);
            best[ct] = o > best[ct] ? o : best[ct];
        }
        if (g == 0) kbest[wave][ct * 16 + r] = best[ct];
    }
    __syncthreads();
    if (threadIdx.x < CT * 16 && (int)threadIdx.x < Mt) {
        unsigned long long k = kbest[0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < NW; ++w) k = kbest[w][threadIdx.x] > k ? kbest[w][threadIdx.x] : k;
        if (k != 0ull) __hip_atomic_fetch_max(&a.keys[M0 + threadIdx.x], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the key updates are device-scope read-modify-writes, performed at the
    // memory side (past the per-XCD L2s) and complete before the completion
    // count is issued; the last workgroup's exchanges are device-scope RMWs
    // too, so they see every update without a cache maintenance fence (an
    // acquire-release count, whose L2 write-back and invalidate run in every
    // workgroup, measured 45 -> 70 us on the INT8 lm_head at one token)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ unsigned last;
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;
    for (int m = threadIdx.x; m < a.M; m += NW * 64) {
        const unsigned long long kk = __hip_atomic_exchange(&a.keys[m], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.ids[m] = (int32_t)key_index(kk);
        if (a.maxv) a.maxv[m] = key_value(kk);
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Tied lm_head with the fused greedy argmax, activation-stationary, BF16 E,
// 65..128 tokens (K = 1024).
//
// The weight-stationary kernel above holds a token group's activations in LDS,
// so beyond 64 tokens it runs two token groups and every CU pulls its share
// of E into registers twice.  Here the roles flip: each of the 8 waves keeps
// one 16-token tile of the activations in registers for all of K (the MFMA B
// operands, 128 VGPRs), and E streams through an LDS ring exactly once per
// workgroup: direct-to-LDS loads of 32-row chunks (both tiles of a block over
// 16 k-steps, 32 KB), four chunks deep, read by all 8 waves as MFMA A
// operands.  One barrier per chunk publishes it and frees the slot the chunk
// three ahead is loaded into.  Each accumulator sums its k-steps in the order
// the weight-stationary kernel does, so the logits, the maxima and the ids
// are the same bit for bit; a lane visits its rows in increasing order
// (strict compare: the lowest row of a tie), and the keys meet as there (one
// atomic max per token, the last workgroup decodes).
//
// Every wave reads every A fragment of E from LDS, 1 KB per MFMA (the
// weight-stationary kernel reads 0.5 KB of B per MFMA), so the LDS reads, not
// the stream, bound it: 96-98 us at 65..128 tokens against 99-101 us for the
// two weight-stationary passes.  With INT8 E it lost (98 against 78 us, the
// units converted to f16 once per chunk into LDS; 130 us with every wave
// converting them), so INT8 keeps the weight-stationary kernel.
// ---------------------------------------------------------------------------
constexpr int kAsNW = 8;                           // waves: one 16-token tile each
constexpr int kAsKC = 16;                          // k-steps per chunk
constexpr int kAsNS = 4;                           // chunks in the LDS ring
constexpr int kAsChunk = 2 * kAsKC * 1024;         // both tiles' 1 KB units
constexpr size_t kAsLds = (size_t)kAsNS * kAsChunk;

__global__ __launch_bounds__(kAsNW * 64) void as_argmax_kernel(WideArgmaxArgs a) {
    constexpr int KSTEPS = 32;                     // k-steps of K = 1024
    constexpr int CH = KSTEPS / kAsKC;             // chunks per 32-row block
    constexpr int PER = 2 * kAsKC / kAsNW;         // units a wave loads per chunk
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int G = (int)gridDim.x, wg = (int)blockIdx.x;
    const int nb = wg < a.n_blk ? (a.n_blk - wg + G - 1) / G : 0;  // blocks wg, wg + G, ...
    const int nq = nb * CH;                                        // chunks
    const int m = wave * 16 + r;                                   // this lane's token

    // ---- the wave's token tile, all of K, as B operands ----
    u32x4 B[KSTEPS];
    {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2));
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            B[ks] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           xr, m < a.M ? (uint32_t)((m * a.ldx + ks * 32 + g * 8) * 2) : OOB, 0, 0));
    }

    // ---- E through the LDS ring ----
    const uint32_t tile_bytes = (uint32_t)KSTEPS * 1024u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_tiles * tile_bytes));
    // chunk q into slot q % NS: block wg + (q / CH) G, k-steps from (q % CH)
    // KC; unit u of a chunk is tile u / KC, k-step u % KC.  Every wave issues
    // the same loads per chunk (chunks past the end read zeros), so one wait
    // count fits every chunk.
    auto dma = [&](int q) {
        uint8_t* slot = lds + (q % kAsNS) * kAsChunk;
        const int blk = wg + (q / CH) * G;
        const uint32_t k0 = (uint32_t)(q % CH) * kAsKC * 1024u;
        const bool ok = q < nq;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int u = wave * PER + p;
            const int rt = u / kAsKC, kk = u % kAsKC;
            lds_dma16(wrs, slot + u * 1024,
                      ok ? (uint32_t)(2 * blk + rt) * tile_bytes + k0 + (uint32_t)kk * 1024u + lane * 16 : OOB);
        }
    };
#pragma unroll
    for (int q = 0; q < kAsNS - 1; ++q) dma(q);

    float bv = -__builtin_inff();  // this lane's running maximum of its token and its row
    uint32_t bi = 0xffffffffu;
    f32x4 acc[2];
    for (int i = 0; i < nb; ++i) {
        const int blk = wg + i * G;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int q = i * CH + c;
            // chunk q has landed (the NS - 2 after it may still be in flight);
            // the barrier makes every wave's part of it visible and frees the
            // slot of q - 1
            __builtin_amdgcn_s_waitcnt(vm_wait((kAsNS - 2) * PER));
            __syncthreads();
            dma(q + kAsNS - 1);
            const uint8_t* sl = lds + (q % kAsNS) * kAsChunk + lane * 16;
            if (c == 0) acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < kAsKC; ++kk) {
                const u32x4 A0 = *reinterpret_cast<const u32x4*>(sl + kk * 1024);
                const u32x4 A1 = *reinterpret_cast<const u32x4*>(sl + (kAsKC + kk) * 1024);
                const bf16x8 b = __builtin_bit_cast(bf16x8, B[c * kAsKC + kk]);
                acc[0] = mfma_bf16(__builtin_bit_cast(bf16x8, A0), b, acc[0]);
                acc[1] = mfma_bf16(__builtin_bit_cast(bf16x8, A1), b, acc[1]);
            }
            if (c == CH - 1) {  // the block's logits: into the running maximum
                const int row0 = blk * 32 + g * 4;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = row0 + rt * 16 + e;
                        const bool gt = row < a.V && acc[rt][e] > bv;
                        bv = gt ? acc[rt][e] : bv;
                        bi = gt ? (uint32_t)row : bi;
                    }
            }
        }
    }

    // ---- keys: the four row groups of a lane's token, then the grid ----
    unsigned long long best = 0ull;
    if (bi != 0xffffffffu && m < a.M) best = argmax_key(bv, bi);
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
        const unsigned long long o = __shfl_xor(best, sh);
        best = o > best ? o : best;
    }
    if (g == 0 && m < a.M && best != 0ull)
        __hip_atomic_fetch_max(&a.keys[m], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // completion as in the weight-stationary kernel: device-scope RMWs past
    // the L2s, observed by s_waitcnt before the count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ unsigned last;
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;
    for (int mm = threadIdx.x; mm < a.M; mm += kAsNW * 64) {
        const unsigned long long kk = __hip_atomic_exchange(&a.keys[mm], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.ids[mm] = (int32_t)key_index(kk);
        if (a.maxv) a.maxv[mm] = key_value(kk);
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
namespace {

constexpr int kWideU = 8;  // weight k-steps per wave in flight

int ct_of(int M) { return M <= 32 ? 2 : (M <= 64 ? 4 : 8); }  // token tiles of 16 (at most 128 tokens)

// LDS bytes of a configuration: activations (or, after the MFMAs, the KW
// partial tiles), the norm-weight slice, the residual tiles, the scales.
struct WideLayout {
    size_t x, gamma, res, scales, total;
    int off_gamma, off_res, off_scales;
};

WideLayout wide_layout(int wf, int CT, int nks, int NB, int KW, bool glu, bool gamma, bool res, int rs, bool scales) {
    const int KS = wf == WF_I8 ? 64 : 32, XU = wf == WF_I8 ? 2 : 1;
    WideLayout L{};
    const size_t xb = (size_t)CT * nks * XU * 1024;
    const size_t red = (size_t)NB * KW * 2 * CT * 1024;  // every wave's accumulators
    L.x = std::max(xb, red);
    L.gamma = gamma ? (size_t)((nks * KS * 4 + 1023) / 1024) * 1024 : 0;
    L.res = res ? (size_t)NB * (glu ? 1 : 2) * (CT * rs / 4) * 1024 : 0;
    L.scales = scales ? (size_t)NB * 1024 : 0;
    L.off_gamma = (int)L.x;
    L.off_res = (int)(L.x + L.gamma);
    L.off_scales = (int)(L.x + L.gamma + L.res);
    L.total = L.x + L.gamma + L.res + L.scales;
    return L;
}

template <typename Kern>
hipError_t launch_w(Kern k, const WideArgs& a, int nw, int grid, size_t smem, hipStream_t st) {
    {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)kWideMaxLds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(nw * 64), smem, st, a);
    return hipGetLastError();
}

template <int WF, int XDT, int CT, bool GLU, bool NORM>
hipError_t launch_n(const WideArgs& a, int NB, int KW, int grid, size_t smem, hipStream_t st) {
    constexpr int U = kWideU;
    if (NB == 4 && KW == 1) return launch_w(wide_kernel<WF, XDT, CT, GLU, NORM, 4, 1, U>, a, 4, grid, smem, st);
    if (NB == 2 && KW == 2) return launch_w(wide_kernel<WF, XDT, CT, GLU, NORM, 2, 2, U>, a, 4, grid, smem, st);
    if (NB == 1 && KW == 4) return launch_w(wide_kernel<WF, XDT, CT, GLU, NORM, 1, 4, U>, a, 4, grid, smem, st);
    return hipErrorInvalidValue;
}

template <int WF, int XDT, int CT, bool GLU>
hipError_t launch_ct(const WideArgs& a, int NB, int KW, int grid, size_t smem, hipStream_t st) {
    if (a.s.flags & EP_NORM) return launch_n<WF, XDT, CT, GLU, true>(a, NB, KW, grid, smem, st);
    return launch_n<WF, XDT, CT, GLU, false>(a, NB, KW, grid, smem, st);
}

template <int WF, int XDT, bool GLU>
hipError_t launch_glu(const WideArgs& a, int CT, int NB, int KW, int grid, size_t smem, hipStream_t st) {
    switch (CT) {
        case 2: return launch_ct<WF, XDT, 2, GLU>(a, NB, KW, grid, smem, st);
        case 4: return launch_ct<WF, XDT, 4, GLU>(a, NB, KW, grid, smem, st);
        case 8: return launch_ct<WF, XDT, 8, GLU>(a, NB, KW, grid, smem, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool wide_supported(int wf, int xdt, int M) {
    return M >= 1 && M <= kWideMaxM && ((wf == WF_BF16 && xdt == DT_BF16) || (wf == WF_I8 && xdt == DT_F16));
}

bool wide_plan(const SkinnyArgs& s, int wf, bool glu, int num_cus, size_t partials_cap, int max_counters, int force_s,
               int force_cfg, WidePlan& p) {
    const int n_ptiles = glu ? 2 * s.n_groups : s.n_groups;
    const int nblocks = glu ? s.n_groups : (s.n_groups + 1) / 2;
    const bool gamma = (s.flags & EP_NORM) && s.gamma;
    const bool res = (s.flags & EP_RESIDUAL) && s.vec_store;
    const int rs = s.res_dt == DT_F32 ? 4 : 2;
    static const int cfgs[3][2] = {{4, 1}, {2, 2}, {1, 4}};
    const int force_t = force_cfg >> 4;  // token groups (measurement)
    force_cfg &= 15;
    bool found = false;
    // preference: enough workgroups to stream from most CUs, then no K split
    // (no hand-off), then the most workgroups within one per CU, then fewer
    // K splits, then fewer token groups
    auto better = [&](int S, int grid, int T) {
        if (!found) return true;
        const bool full = 4 * grid >= 3 * num_cus, pfull = 4 * p.grid >= 3 * num_cus;
        if (full != pfull) return full;
        if ((S == 1) != (p.S == 1)) return S == 1;
        if (grid != p.grid) return grid > p.grid;
        if (S != p.S) return S < p.S;
        return T < p.T;
    };
    for (int T = 1; T <= 8; T *= 2) {
        if (force_t && T != force_t) continue;
        const int Mg = (s.M + T - 1) / T;
        if (T > 1 && Mg < 16) break;
        if (Mg > 8 * 16) continue;  // at most 8 token tiles per group (16 would spill registers)
        const int CT = ct_of(Mg);
        for (int S = 1; S <= std::min(s.ksteps, kWideMaxS); ++S) {
            if (force_s && S != force_s) continue;
            const int nks = (s.ksteps + S - 1) / S;
            for (int c = 0; c < 3; ++c) {
                if (force_cfg && c + 1 != force_cfg) continue;
                const int NB = cfgs[c][0], KW = cfgs[c][1];
                if (nks < KW) continue;
                const WideLayout L = wide_layout(wf, CT, nks, NB, KW, glu, gamma, res, rs, s.scales != nullptr);
                if (L.total > kWideMaxLds) continue;
                // keep the direct-to-LDS loads of a wave plus its weight loads
                // within the 63 the vector-memory counter holds (past that the
                // wave stalls at issue until the first ones land)
                const int XU = wf == WF_I8 ? 2 : 1, KS = wf == WF_I8 ? 64 : 32;
                const int nw = NB * KW;
                auto per = [nw](int units) { return (units + nw - 1) / nw; };
                const int small = per(CT * nks * XU) + (gamma ? per((nks * KS * 4 + 1023) / 1024) : 0) +
                                  (res ? per(NB * (glu ? 1 : 2) * CT * rs / 4) : 0) + (s.scales ? 1 : 0);
                if (small + 2 * kWideU > 63) continue;
                int ngrp = (nblocks + NB - 1) / NB;
                if (T > 1) ngrp = (ngrp + 7) / 8 * 8;  // token groups 8 workgroups apart
                if (S > 1 && (size_t)ngrp * T * S * NB * CT * 64 * (2 * 16 + 4) > partials_cap) continue;
                if (S > 1 && ngrp * T > max_counters) continue;
                const int grid = ngrp * T * S;
                if (grid > num_cus && !(force_s || force_cfg || force_t)) continue;
                if (better(S, grid, T)) {
                    found = true;
                    p.S = S;
                    p.T = T;
                    p.Mg = Mg;
                    p.ngrp = ngrp;
                    p.NB = NB;
                    p.KW = KW;
                    p.CT = CT;
                    p.grid = grid;
                    p.smem = L.total;
                    p.off_gamma = L.off_gamma;
                    p.off_res = L.off_res;
                    p.off_scales = L.off_scales;
                    p.nblocks = nblocks;
                    p.n_ptiles = n_ptiles;
                    p.res_lds = res ? 1 : 0;
                }
            }
        }
    }
    return found;
}

bool wide_argmax_plan(int wf, int xdt, int M, int K, int num_cus, WideArgmaxArgs& a, int& grid, size_t& smem) {
    if (!((wf == WF_BF16 && xdt == DT_BF16) || (wf == WF_I8 && (xdt == DT_F16 || xdt == DT_BF16))) || M < 1 ||
        M > 256)
        return false;
    const int ks = K / (wf == WF_I8 ? 64 : 32);
    if (ks % kArgU != 0) return false;
    const int T = (M + 63) / 64;
    const int Mg = (M + T - 1) / T;
    const int CT = Mg <= 32 ? 2 : 4;
    smem = (size_t)CT * ks * (wf == WF_I8 ? 2 : 1) * 1024;
    if (smem > kWideMaxLds) return false;
    grid = num_cus / (8 * T) * (8 * T);
    if (grid < 8 * T) return false;
    a.T = T;
    a.Mg = Mg;
    a.CT = CT;
    a.ksteps = ks;
    // waves per workgroup: 64-token groups fill the LDS (one workgroup per
    // CU); with INT8 weights 8 waves give each SIMD two, to overlap one's
    // MFMAs with the other's conversions and LDS reads (128 tokens: 110 ->
    // 93 us); BF16 weights measured better with 4 (128 -> 145 us with 8).
    // Smaller groups run two 4-wave workgroups per CU
    if (a.nw == 0) a.nw = CT == 4 && wf == WF_I8 ? 8 : 4;
    if (a.wcache < 0) a.wcache = T > 1 ? 1 : 0;
    return true;
}

hipError_t launch_wide_argmax(const WideArgmaxArgs& a, int wf, int xdt, int grid, size_t smem, hipStream_t stream) {
    auto go = [&](auto kern) {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(kern), (int)kWideMaxLds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, dim3(grid), dim3(a.nw * 64), smem, stream, a);
        return hipGetLastError();
    };
    if (a.nw != 4 && a.nw != 8) return hipErrorInvalidValue;
    // 16-token-tile pairs run one token group (weights streamed once,
    // non-temporal); 64-token groups may be several, whose later groups read
    // the weights from L2 if the loads keep the default cache policy
    auto pick = [&](auto wfc, auto xdtc) {
        constexpr int W = decltype(wfc)::value, X = decltype(xdtc)::value;
        if (a.CT == 2) return a.nw == 8 ? go(wide_argmax_kernel<W, X, 2, 8, AUX_NT>) : go(wide_argmax_kernel<W, X, 2, 4, AUX_NT>);
        if (a.wcache)
            return a.nw == 8 ? go(wide_argmax_kernel<W, X, 4, 8, 0>) : go(wide_argmax_kernel<W, X, 4, 4, 0>);
        return a.nw == 8 ? go(wide_argmax_kernel<W, X, 4, 8, AUX_NT>) : go(wide_argmax_kernel<W, X, 4, 4, AUX_NT>);
    };
    using I = std::integral_constant<int, WF_I8>;
    if (wf == WF_BF16) return pick(std::integral_constant<int, WF_BF16>{}, std::integral_constant<int, DT_BF16>{});
    if (xdt == DT_BF16) return pick(I{}, std::integral_constant<int, DT_BF16>{});
    return pick(I{}, std::integral_constant<int, DT_F16>{});
}

bool as_argmax_plan(int wf, int xdt, int M, int K, int num_cus, int& grid, size_t& smem) {
    if (!(wf == WF_BF16 && xdt == DT_BF16) || K != 1024 || M < 1 || M > kAsNW * 16 || num_cus < 8) return false;
    grid = num_cus;
    smem = kAsLds;
    return true;
}

hipError_t launch_as_argmax(const WideArgmaxArgs& a, int wf, int xdt, int grid, size_t smem, hipStream_t stream) {
    if (!(wf == WF_BF16 && xdt == DT_BF16) || a.K != 1024 || a.M < 1 || a.M > kAsNW * 16 || smem != kAsLds ||
        a.scales)
        return hipErrorInvalidValue;
    hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(as_argmax_kernel), (int)smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(as_argmax_kernel, dim3(grid), dim3(kAsNW * 64), smem, stream, a);
    return hipGetLastError();
}

hipError_t launch_wide(const WideArgs& a, const WidePlan& p, int wf, int xdt, bool glu, hipStream_t stream) {
    if (!wide_supported(wf, xdt, a.s.M) || p.smem > kWideMaxLds) return hipErrorInvalidValue;
    if (wf == WF_BF16) {
        if (glu) return launch_glu<WF_BF16, DT_BF16, true>(a, p.CT, p.NB, p.KW, p.grid, p.smem, stream);
        return launch_glu<WF_BF16, DT_BF16, false>(a, p.CT, p.NB, p.KW, p.grid, p.smem, stream);
    }
    if (glu) return launch_glu<WF_I8, DT_F16, true>(a, p.CT, p.NB, p.KW, p.grid, p.smem, stream);
    return launch_glu<WF_I8, DT_F16, false>(a, p.CT, p.NB, p.KW, p.grid, p.smem, stream);
}

}  // namespace qwk
