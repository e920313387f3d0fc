// qw_gemm.hip -- LDS double-buffered MFMA GEMM for gfx950 (prefill and
// large-batch decode):  y[m][n] = sum_k W[n][k] * x[m][k]  (+ epilogue).
//
// Tiling.  A workgroup computes RW = 256 (or 64) weight rows x BM tokens with 32 x 32 x 16
// MFMAs (weights are the A operand, tokens the B operand; FP32
// accumulators); K advances in blocks of one k-step of the packed weight
// (32 deep for BF16, 64 for INT8).  Shapes:
//   - BM = 256, 8 waves (once the 256-token blocks fill the chip): each wave
//     128 rows x 64 tokens, two waves per SIMD, half the L2->LDS bytes per
//     FLOP of the 128-token block;
//   - BM = 128: BF16 with 4 waves (each 128 x 64; two workgroups share a CU,
//     so one's barrier and LDS waits are covered by the other), INT8 with 8
//     waves (each 128 x 32);
//   - BM = 256, 4 waves (BF16): each wave 128 x 128 (one wave per SIMD);
//   - RW = 64, BM = 128, 4 waves (both formats): each wave 64 x 32, for few
//     tokens on few weight rows, where 256-row blocks leave CUs idle.
// Weight formats: BF16 weights use the bf16 MFMA on BF16 activations.  INT8
// weights (per-row scales) reach LDS as INT8, half the bytes; each lane
// converts its 8-byte fragment exactly to f16 (qw_device.hpp i8x4_to_f16)
// for the f16 MFMA, BF16 activations are converted to f16 when read, and the
// row scale is applied in the epilogue -- y = s * sum q*x, the reference's
// dequantize-then-multiply.
//
// Loads.  Both operands reach LDS through direct buffer->LDS loads
// (buffer_load_dwordx4 ... lds): one wave instruction moves one 1 KB unit.
// The weights are already stored in the packed tile order (qw_device.hpp),
// and the activations are fetched so that they land in the same order: lane
// (r, g) of a unit carries x[token r][8 k starting at group g].  A 32 x 32 x 16
// fragment of either operand is then one conflict-free ds_read_b128 per lane.
// Three (BM = 128: 3 x 24 KB) or four (BM = 256: 4 x 32 KB) LDS stages keep
// the next K-blocks' loads in flight while one is multiplied; a wave waits
// only for its own loads of the block it is about to use, then one barrier
// per block publishes them, placed mid-block so that no barrier sits between
// a fragment read and its MFMAs.  The loads of a block are issued one per MFMA
// pair so the matrix pipe never waits on a burst of load issues.
//
// Epilogue.  In a 32-row weight block, rows i and i+16 of a token land in the
// same lane (accumulator items q and q+8), so a GLU weight -- gate and up
// tiles interleaved by the packer -- becomes silu(gate)*up in registers.
// Residual add, Q/gate de-interleave and BF16/F16/F32 stores as in the skinny
// kernel, or a per-token (logit, index) maximum for the lm_head (lowest index
// on ties) merged with a 64-bit atomic max.
//
// Reference operators replaced: the cuBLAS SGEMM / GemmEx projections of the
// batched paths (full_attention_cuda.cu:708-714, linear_attention_cuda.cu:
// 589-615,664-669, cublas_utils.cuh:48-93, bf16_gemm.cuh:82-122) and the
// per-token loops of CudaMLP (mlp_cuda.cu:295-330 and the lossy base's
// per-token launches, lossy_optimization/04_weight_int8/kernels/mlp_cuda.cu:
// 372-391).
#include "qw_stream.hpp"

namespace qwk {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int G_GROUP_M = 8;               // token blocks per raster group
constexpr int G_EPI_PITCH = 68;            // epilogue LDS row pitch (floats): 64 rows + pad

// Stage geometry for a block of RW weight rows x BM tokens, NW waves and
// weight format WF.  A K-block is one k-step of the packed weight: 32 deep
// for BF16, 64 for INT8 (KSUB 32-deep activation sub-steps).  A stage holds
// the block's RW/16 weight units and KSUB * BM/16 activation units (after the
// weight units); UPW units per wave;
// NS stages in flight (fewer where the stage is larger or two workgroups
// share a CU).
template <int BM, int NW, int WF, int RW> struct GTile {
    static constexpr int WR = RW == 256 ? 2 : 1;      // waves along the rows
    static constexpr int WM = NW / WR;                // waves along the tokens
    static constexpr int WT = BM / WM;                // tokens per wave
    static constexpr int MB = WT / 32;                // 32-token MFMA blocks per wave
    static constexpr int NBW = RW / WR / 32;          // 32-row MFMA blocks per wave
    static constexpr int WU = RW / 16;                // weight units (16-row tiles) per stage
    static constexpr int KSUB = WF == WF_I8 ? 2 : 1;
    static constexpr int KSL = 2 * KSUB;              // 16-deep MFMA slices per K-block
    static constexpr int XU = BM / 16;                // activation units per sub-step
    static constexpr int UNITS = WU + KSUB * XU;
    static constexpr int UPW = UNITS / NW;
    static constexpr int STAGE = UNITS * 1024;
    static constexpr int NS = (BM == 256 && WF != WF_I8) ? 4 : 3;
    static_assert(MB >= 1 && UPW >= 1 && UNITS % NW == 0, "tile shape");
    static constexpr size_t lds_bytes() {
        const size_t epi = (size_t)NW * WT * G_EPI_PITCH * sizeof(float);
        const size_t pipe = (size_t)NS * STAGE;
        return epi > pipe ? epi : pipe;
    }
};

// Element-wise store for outputs whose row count or alignment rules out the
// 4-wide stores.
__device__ __forceinline__ void gemm_store_slow(const GemmArgs& a, int m, int row, f32x4 o4) {
    for (int e = 0; e < 4; ++e) {
        const int oi = row + e;
        if (oi >= a.N) break;
        float vi = o4[e];
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

// Fragment registers: 8 halves (bf16 or f16) as raw bits.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// WF: BF16 (bf16 MFMA) or INT8 (weights converted exactly to f16 in registers,
// f16 MFMA; BF16 activations are converted to f16 as well).  XDT: activation
// type (BF16, or F16 with INT8 weights).
template <int WF, int XDT, bool GLU, bool ARGMAX, int BM, int NW, int RW>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(BM == 256 && NW == 4 ? 1 : 2, BM == 256 && NW == 4 ? 1 : 2)))
void gemm_kernel(GemmArgs a) {
    using T = GTile<BM, NW, WF, RW>;
    constexpr int MB = T::MB, UPW = T::UPW, G_NS = T::NS, G_STAGE = T::STAGE, WM = T::WM, WT = T::WT;
    constexpr int KSUB = T::KSUB, KSL = T::KSL, XU = T::XU, NBW = T::NBW, WU = T::WU, WR = T::WR;
    constexpr int G_XOFF = WU * 1024;       // activation units follow the weight units
    constexpr bool I8 = WF == WF_I8;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ unsigned long long best_s[WR][BM];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn = wave / WM, wm = wave % WM;   // 32*NBW rows x WT tokens of this wave

    // XCD-aware order: consecutive workgroup ids go to different XCDs; give
    // each XCD a contiguous range of tiles (M fastest) so the tiles that
    // share a weight block run on the same L2.
    const int nwg = gridDim.x;
    int b = blockIdx.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    // split-K (64-row blocks only): consecutive ids after the XCD order are
    // the splits of one tile
    constexpr bool SPLITK = RW == 64 && !ARGMAX;
    const int S = SPLITK ? max(1, a.splitk) : 1;
    const int sk = b % S;
    b /= S;
    const int tile = b;
    // grouped raster: G_GROUP_M token blocks x all weight blocks per group,
    // token block fastest, so the workgroups resident on one XCD at a time
    // share both their activation blocks and their weight blocks in its L2
    const int per_group = G_GROUP_M * a.nblk_n;
    const int group = b / per_group;
    const int first_m = group * G_GROUP_M;
    const int gm = min(G_GROUP_M, a.nblk_m - first_m);
    const int in_group = b - group * per_group;
    const int bm = first_m + in_group % gm, bn = in_group / gm;
    const int nt0 = bn * WU;                   // first physical 16-row tile
    const int m0 = bm * BM;

    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_tiles * a.ksteps * 1024u));
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2u));
    // K-blocks (one 32-deep k-step each) of this workgroup's split
    const int kb_lo = (int)((int64_t)sk * a.ksteps / S);
    const int nkb = (int)((int64_t)(sk + 1) * a.ksteps / S) - kb_lo;

    // The UPW units this wave moves per K-block: unit u = wave*UPW + q of the
    // stage is weight tile u (u < WU) or activation unit v = u - WU (sub-step
    // v / XU, token group v % XU), and lands at byte u*1024.  The buffer and
    // per-block stride of each unit are chosen once (wave-uniform selects),
    // so issuing a load inside the K-loop is branch-free.
    uint32_t vbase[UPW], vstep[UPW];
    __amdgpu_buffer_rsrc_t rsq[UPW];
#pragma unroll
    for (int q = 0; q < UPW; ++q) {
        const int u = wave * UPW + q;
        const bool isw = u < WU;
        const int pt = nt0 + u;
        const int v = u - WU;
        const int row = m0 + (v % XU) * 16 + (lane & 15);
        const uint32_t wo = pt < a.n_tiles ? (uint32_t)(pt * a.ksteps * 1024 + lane * 16) : OOB;
        const uint32_t xo = row < a.M ? (uint32_t)((row * a.ldx + (lane >> 4) * 8) * 2 + (v / XU) * 64) : OOB;
        vbase[q] = isw ? wo : xo;
        vstep[q] = isw ? 1024u : (uint32_t)(KSUB * 64);
        rsq[q] = isw ? wrs : xrs;
    }
    auto dma = [&](int kb, int q) {
        uint8_t* dst = lds + (kb % G_NS) * G_STAGE + (wave * UPW + q) * 1024;
        lds_dma16(rsq[q], dst, vbase[q] + (uint32_t)(kb + kb_lo) * vstep[q]);
    };

    f32x16 acc[NBW][MB];
#pragma unroll
    for (int i = 0; i < NBW; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = f32x16{};

    // lane -> fragment address: row l%32 of a 32-row block = tile (l%32)/16,
    // row l%16.  BF16 unit (32 k): k-group 2*slice + l/32 of 8 -> 16 bytes at
    // ((l%16) + 16*(l/32))*16 + slice*512.  INT8 unit (64 k): lane group g of
    // the unit holds 16 k from 16g, so slice s, half l/32 is the 8 bytes at
    // ((l%16) + 16*s)*16 + 8*(l/32).  Activation units as BF16 weight units.
    const int frag_tile = (lane & 31) >> 4;
    const int frag_off = ((lane & 15) + 16 * (lane >> 5)) * 16;
    const int frag_off8 = (lane & 15) * 16 + 8 * (lane >> 5);

    // fragments of one 16-deep slice (raw 16-bit bits)
    u32x4v A[2][NBW], B[2][MB];
    auto read_frags = [&](const uint8_t* st, int sl, u32x4v (&Ad)[NBW], u32x4v (&Bd)[MB]) {
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const int t = wn * 2 * NBW + nb * 2 + frag_tile;
            if constexpr (I8) {
                const uint2 w8 = *reinterpret_cast<const uint2*>(st + t * 1024 + frag_off8 + sl * 256);
                uint32_t l0, h0, l1, h1;
                i8x4_to_f16(w8.x, l0, h0);
                i8x4_to_f16(w8.y, l1, h1);
                Ad[nb] = u32x4v{l0, h0, l1, h1};
            } else {
                Ad[nb] = *reinterpret_cast<const u32x4v*>(st + t * 1024 + frag_off + sl * 512);
            }
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int t = (sl >> 1) * XU + wm * 2 * MB + mb * 2 + frag_tile;
            u32x4v xv = *reinterpret_cast<const u32x4v*>(st + G_XOFF + t * 1024 + frag_off + (sl & 1) * 512);
            if constexpr (I8 && XDT == DT_BF16) {  // exact for |x| in the f16 normal range
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    xv[e] = f32_to_f16_bits(bf16_bits_to_f32(xv[e] & 0xffffu)) |
                            (f32_to_f16_bits(bf16_bits_to_f32(xv[e] >> 16)) << 16);
            }
            Bd[mb] = xv;
        }
    };
    auto mfma = [&](const u32x4v& av, const u32x4v& bv, f32x16& c) {
        if constexpr (I8)
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv),
                                                       c, 0, 0, 0);
        else
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv),
                                                        c, 0, 0, 0);
    };

    // G_NS-stage pipeline over K-blocks of KSL 16-deep slices.  Block kb runs
    // its slices with a one-slice fragment lookahead (slice s+1 is read while
    // slice s is multiplied, two register buffers).  Before the last slice's
    // MFMAs: wait for this wave's loads of block kb+1 and one barrier, which
    // publishes kb+1 and proves every wave has consumed block kb-1 (its last
    // slice was multiplied); then slice 0 of kb+1 is read and the last slice
    // is multiplied with the global->LDS loads of block kb+G_NS-1 (into the
    // stage of kb-1) issued between MFMAs.  LDS read latency is covered by the
    // previous slice's MFMAs and no barrier sits between a fragment read and
    // its use.
    auto wait_loads = [&](int later) {  // at most `later` blocks of loads may stay in flight
        if (later >= 2) __builtin_amdgcn_s_waitcnt(vm_wait(2 * UPW));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(vm_wait(UPW));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
    };
#pragma unroll
    for (int s0 = 0; s0 < G_NS - 1; ++s0)
        if (s0 < nkb) {
#pragma unroll
            for (int q = 0; q < UPW; ++q) dma(s0, q);
        }
    wait_loads(min(G_NS - 2, nkb - 1));
    __syncthreads();
    read_frags(lds, 0, A[0], B[0]);
    // The final block is peeled off so the loop body has a single path: at a
    // control-flow join the compiler's wait counting would make the last
    // slice's MFMAs wait for the next block's fragment reads.
    auto kblock = [&](int kb, auto last) {
        constexpr bool LAST = decltype(last)::value;
        const uint8_t* st = lds + (kb % G_NS) * G_STAGE;
#pragma unroll
        for (int sl = 0; sl < KSL - 1; ++sl) {
            read_frags(st, sl + 1, A[(sl + 1) & 1], B[(sl + 1) & 1]);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < NBW * MB; ++i) mfma(A[sl & 1][i / MB], B[sl & 1][i % MB], acc[i / MB][i % MB]);
            __builtin_amdgcn_s_setprio(0);
        }
        constexpr int LB = (KSL - 1) & 1;  // register buffer of the last slice
        if constexpr (!LAST) {
            wait_loads(min(G_NS - 3, nkb - kb - 2));
            __syncthreads();
            read_frags(lds + ((kb + 1) % G_NS) * G_STAGE, 0, A[LB ^ 1], B[LB ^ 1]);
        }
        const bool more = kb + G_NS - 1 < nkb;
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < NBW * MB; ++i) {
            mfma(A[LB][i / MB], B[LB][i % MB], acc[i / MB][i % MB]);
            constexpr int per = (NBW * MB) / UPW > 0 ? (NBW * MB) / UPW : 1;  // MFMAs per load issue
            if constexpr (!LAST) {
                if (i % per == per - 1 && i / per < UPW) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (more) dma(kb + G_NS - 1, i / per);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if constexpr (!LAST && (NBW * MB) / UPW == 0) {  // more units than MFMAs: the rest after them
#pragma unroll
            for (int q = NBW * MB; q < UPW; ++q)
                if (more) dma(kb + G_NS - 1, q);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    for (int kb = 0; kb < nkb - 1; ++kb) kblock(kb, std::false_type{});
    kblock(nkb - 1, std::true_type{});

    // ---- split-K hand-off: agent-scope stores of this split's tile, wait
    // for their completion, one arrival count per tile; the last split to
    // arrive sums all S partial tiles in split order (its own included) and
    // runs the epilogue, the others leave.  The counter returns to zero.
    if constexpr (SPLITK) {
        if (S > 1) {
            constexpr int PER = NBW * MB * 16;  // accumulator floats per lane
            constexpr int P16 = PER / 4;          // 16-byte pieces per lane
            // partial tiles [tile][split][thread][PER], written and read with
            // device-coherent (sc1) 16-byte accesses
            const uint64_t pbytes = (uint64_t)(a.nblk_n * a.nblk_m) * S * (NW * 64) * PER * 4;
            const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.partials, (uint32_t)min(pbytes, (uint64_t)0x7fffffff));
            const uint32_t tbase = (uint32_t)(((uint64_t)tile * S * (NW * 64) + threadIdx.x) * PER * 4);
            const uint32_t sstride = (uint32_t)((NW * 64) * PER * 4);
#pragma unroll
            for (int i = 0; i < NBW; ++i)
#pragma unroll
                for (int j = 0; j < MB; ++j)
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4) {
                        const f32x4 v = {acc[i][j][4 * e4], acc[i][j][4 * e4 + 1], acc[i][j][4 * e4 + 2], acc[i][j][4 * e4 + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                               tbase + sk * sstride + ((i * MB + j) * 4 + e4) * 16, 0,
                                                               AUX_SC1);
                    }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __shared__ unsigned last_s;
            __syncthreads();
            if (threadIdx.x == 0) {
                const unsigned old = __hip_atomic_fetch_add(&a.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_s = old == (unsigned)(S - 1) ? 1u : 0u;
                if (old == (unsigned)(S - 1)) __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (!last_s) return;  // uniform over the workgroup
#pragma unroll
            for (int i = 0; i < NBW; ++i)
#pragma unroll
                for (int j = 0; j < MB; ++j) acc[i][j] = f32x16{};
            for (int s2 = 0; s2 < S; ++s2) {  // split order; all of a split's loads in flight at once
                f32x4 pv[P16];
#pragma unroll
                for (int p = 0; p < P16; ++p)
                    pv[p] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, tbase + s2 * sstride + p * 16, 0,
                                                                                           AUX_SC1));
#pragma unroll
                for (int i = 0; i < NBW; ++i)
#pragma unroll
                    for (int j = 0; j < MB; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e) acc[i][j][e] += pv[(i * MB + j) * 4 + e / 4][e % 4];
            }
        }
    }

    // ---- epilogue ----
    // accumulator item q of lane l: weight row i = 8*(q/4) + 4*(l/32) + q%4 of
    // the 32-row block, token j = l%32 of the 32-token block
    const int ihi = 4 * (lane >> 5);
    if constexpr (ARGMAX) {
        unsigned long long best[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) best[mb] = 0ull;
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const int pt0 = nt0 + wn * 2 * NBW + nb * 2;
#pragma unroll
            for (int qg = 0; qg < 4; ++qg) {
                const int row = pt0 * 16 + 8 * qg + ihi;
                f32x4 sc = {1.f, 1.f, 1.f, 1.f};
                if (a.scales) sc = *reinterpret_cast<const f32x4*>(a.scales + row);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const unsigned long long kk = argmax_key(acc[nb][mb][4 * qg + e] * sc[e], (uint32_t)(row + e));
                        best[mb] = (row + e < a.N && kk > best[mb]) ? kk : best[mb];
                    }
            }
        }
        // lanes l and l^32 hold the same token; then the two waves sharing a
        // token range (wn = 0, 1) meet in LDS; then the grid via atomic max
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const unsigned long long o = __shfl_xor(best[mb], 32);
            best[mb] = o > best[mb] ? o : best[mb];
            if (lane < 32) best_s[wn][wm * WT + mb * 32 + lane] = best[mb];
        }
        __syncthreads();
        if (threadIdx.x < BM) {
            const int j = threadIdx.x;
            unsigned long long kk = best_s[0][j];
#pragma unroll
            for (int r = 1; r < WR; ++r) kk = best_s[r][j] > kk ? best_s[r][j] : kk;
            if (m0 + j < a.M && kk != 0ull)
                __hip_atomic_fetch_max(&a.keys[m0 + j], kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // completion count (agent-scope read-modify-writes are performed at the
        // coherence point; waiting for them orders the key updates first)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            best_s[0][0] = (old == gridDim.x - 1) ? 1ull : 0ull;
        }
        __syncthreads();
        if (best_s[0][0] == 1ull) {
            for (int m = threadIdx.x; m < a.M; m += NW * 64) {
                const unsigned long long kk =
                    __hip_atomic_exchange(&a.keys[m], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                a.ids[m] = (int32_t)key_index(kk);
                if (a.maxv) a.maxv[m] = key_value(kk);
            }
            if (threadIdx.x == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        // Results pass through LDS as [token][row] (row pitch G_EPI_PITCH
        // floats) so that each token's output rows leave as one contiguous,
        // coalesced store, and so that the accumulators are only ever indexed
        // with constants.  GLU: the wave's 16*NBW output rows in one pass;
        // plain: its 32*NBW rows in passes of 64.
        float* ep = reinterpret_cast<float*>(lds) + wave * (WT * G_EPI_PITCH);
        const int row_base = GLU ? ((nt0 + wn * 2 * NBW) >> 1) * 16 : (nt0 + wn * 2 * NBW) * 16;
        constexpr int PASSES = GLU ? 1 : NBW / 2;   // passes of (up to) 64 rows
        constexpr int NBP = GLU ? NBW : 2;          // 32-row blocks per pass
        constexpr int PROWS = GLU ? 16 * NBW : 64;  // output rows per pass
        const int tok_base = m0 + wm * WT;
        const bool has_res = (a.flags & EP_RESIDUAL) != 0;
        const bool has_split = (a.flags & EP_SPLIT) != 0;
        const int sp_log = a.split_period > 0 ? 31 - __builtin_clz((unsigned)a.split_period) : 0;
        __syncthreads();  // every wave is done reading the K-loop stages
#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass) {
#pragma unroll
            for (int nbl = 0; nbl < NBP; ++nbl) {
                const int nb = GLU ? nbl : pass * 2 + nbl;
                const int pt0 = nt0 + wn * 2 * NBW + nb * 2;
#pragma unroll
                for (int qg = 0; qg < (GLU ? 2 : 4); ++qg) {
                    const int r0 = 8 * qg + ihi;
                    f32x4 sg = {1.f, 1.f, 1.f, 1.f}, su = {1.f, 1.f, 1.f, 1.f};
                    if (a.scales) {
                        sg = *reinterpret_cast<const f32x4*>(a.scales + pt0 * 16 + r0);
                        if (GLU) su = *reinterpret_cast<const f32x4*>(a.scales + (pt0 + 1) * 16 + r0);
                    }
                    const int lrow = GLU ? nb * 16 + r0 : nbl * 32 + r0;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        f32x4 o4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if constexpr (GLU)
                                o4[e] = silu_f(acc[nb][mb][4 * qg + e] * sg[e]) * (acc[nb][mb][4 * qg + 8 + e] * su[e]);
                            else
                                o4[e] = acc[nb][mb][4 * qg + e] * sg[e];
                        }
                        *reinterpret_cast<f32x4*>(ep + (mb * 32 + (lane & 31)) * G_EPI_PITCH + lrow) = o4;
                    }
                }
            }
            // wave-local hand-off: each wave reads back only what it wrote
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            const int c = lane & 15;  // rows 4c .. 4c+3 (PROWS of them exist)
            const int row = row_base + pass * 64 + 4 * c;
            for (int it = 0; it < WT / 4; ++it) {
                const int jj = it * 4 + (lane >> 4);
                const int m = tok_base + jj;
                if (m < a.M && row < a.N && 4 * c < PROWS) {
                    f32x4 o4 = *reinterpret_cast<const f32x4*>(ep + jj * G_EPI_PITCH + 4 * c);
                    if (a.vec_store) {
                        if (has_res) o4 += load_act4(a.res, a.res_dt, (int64_t)m * a.ld_res + row);
                        void* dst = a.y;
                        int col = row;
                        if (has_split) {  // power-of-two period: shifts only
                            dst = ((row >> sp_log) & 1) ? a.y2 : a.y;
                            col = ((row >> (sp_log + 1)) << sp_log) + (row & (a.split_period - 1));
                        }
                        store_act4(dst, a.ydt, (int64_t)m * a.ldy + col, o4);
                    } else {
                        gemm_store_slow(a, m, row, o4);
                    }
                }
            }
            if (!GLU && pass + 1 < PASSES) {
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
}

template <typename Kern>
static hipError_t launch_gemm_k(Kern k, const GemmArgs& a, int grid, int threads, size_t lds, hipStream_t st) {
    {
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, st, a);
    return hipGetLastError();
}

template <int WF, int XDT, int BM, int NW, int RW>
static hipError_t launch_bm(const GemmArgs& a, bool glu, bool argmax, hipStream_t stream) {
    const int grid = a.nblk_n * a.nblk_m * ((RW == 64 && !argmax) ? std::max(1, a.splitk) : 1);
    const size_t lds = GTile<BM, NW, WF, RW>::lds_bytes();
    if (argmax) return launch_gemm_k(gemm_kernel<WF, XDT, false, true, BM, NW, RW>, a, grid, NW * 64, lds, stream);
    if (glu) return launch_gemm_k(gemm_kernel<WF, XDT, true, false, BM, NW, RW>, a, grid, NW * 64, lds, stream);
    return launch_gemm_k(gemm_kernel<WF, XDT, false, false, BM, NW, RW>, a, grid, NW * 64, lds, stream);
}

// Block shapes (rows x tokens, waves): BF16 weights 256 x 256 (8 or 4 waves),
// 256 x 128 (4 waves, two workgroups per CU); INT8 weights 256 x 256 and
// 256 x 128 (8 waves); both formats 64 x 128 (4 waves, each 64 x 32) for
// few tokens on few weight rows, where 256-row blocks leave CUs idle.
template <int WF, int XDT>
static hipError_t launch_wf(const GemmArgs& a, bool glu, bool argmax, hipStream_t stream) {
    if (a.rows == 64) {
        if (a.tile_m != 128 || a.nblk_m != (a.M + 127) / 128) return hipErrorInvalidValue;
        return launch_bm<WF, XDT, 128, 4, 64>(a, glu, argmax, stream);
    }
    if (a.rows != 256) return hipErrorInvalidValue;
    if (a.tile_m == 256 && a.nblk_m == (a.M + 255) / 256) {
        if (a.waves == 8) return launch_bm<WF, XDT, 256, 8, 256>(a, glu, argmax, stream);
        if constexpr (WF == WF_BF16) return launch_bm<WF, XDT, 256, 4, 256>(a, glu, argmax, stream);
        return hipErrorInvalidValue;
    }
    if (a.tile_m == 128 && a.nblk_m == (a.M + 127) / 128) {
        if constexpr (WF == WF_I8) return launch_bm<WF, XDT, 128, 8, 256>(a, glu, argmax, stream);
        else return launch_bm<WF, XDT, 128, 4, 256>(a, glu, argmax, stream);
    }
    return hipErrorInvalidValue;
}

int gemm_acc_floats_per_thread(int rows, int tile_m, int waves) {
    const int wr = rows == 256 ? 2 : 1;           // waves along the rows
    const int wt = tile_m / (waves / wr);         // tokens per wave
    return (rows / wr / 32) * (wt / 32) * 16;     // NBW * MB * 16
}

bool gemm_supported(int wf, int xdt) {
    return (wf == WF_BF16 && xdt == DT_BF16) || (wf == WF_I8 && (xdt == DT_BF16 || xdt == DT_F16));
}

hipError_t launch_gemm(const GemmArgs& a, int wf, int xdt, bool glu, bool argmax, hipStream_t stream) {
    if (!gemm_supported(wf, xdt)) return hipErrorInvalidValue;
    if (argmax && glu) return hipErrorInvalidValue;
    if (wf == WF_BF16) return launch_wf<WF_BF16, DT_BF16>(a, glu, argmax, stream);
    if (xdt == DT_F16) return launch_wf<WF_I8, DT_F16>(a, glu, argmax, stream);
    return launch_wf<WF_I8, DT_BF16>(a, glu, argmax, stream);
}

}  // namespace qwk
