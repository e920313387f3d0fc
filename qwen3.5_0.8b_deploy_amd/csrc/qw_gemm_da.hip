// qw_gemm_da.hip -- the prefill GEMM for BF16 weights and BF16 activations
// at many tokens ("direct-A"):  y[m][n] = sum_k W[n][k] * x[m][k] (+ epilogue).
//
// Shape.  A workgroup of 4 waves computes 256 weight rows x 128 tokens; wave
// w owns rows 64w..64w+63 for all 128 tokens (4 x 8 blocks of the 16x16x32
// bf16 MFMA, 128 accumulators), so two workgroups share a CU and each covers
// the other's prologue, barriers and epilogue.
//
// Operands.  A packed 1 KB weight unit (16 rows x one 32-deep k-step, lane
// l = r + 16g holding row r's k 8g..8g+7) is exactly the A operand of the
// 16x16x32 MFMA, and the four row tiles of a wave belong to it alone: the
// weights go straight from memory into a ring of VGPRs, D k-steps ahead,
// without LDS.  The activations are shared by the four waves: each k-step's
// 8 token units (16 tokens x 32 k, same lane order, i.e. the B operand)
// arrive through direct-to-LDS loads into one of NS stages, one barrier per
// k-step publishes them, and each wave reads its B fragments one k-step
// ahead, column by column as the previous ones retire.
//
// Per CU and k-step this moves 32 KB of weights (VGPRs) and 16 KB of
// activations (LDS), and reads 64 KB of B fragments from LDS, for 256 MFMAs.
//
// Epilogue.  Per 16-token column the wave stages its results as FP32
// [token][row] in a private LDS buffer (silu(gate)*up first for a GLU
// weight: the packer interleaves gate and up tiles, so a pair of row tiles
// becomes one output tile in registers), then reads them back as 4-row
// pieces and stores whole 128-byte (or 64-byte) token rows, adding the
// residual and applying the Q/gate de-interleave on the way.
//
// Persistent form (8 waves, 512-row blocks, the default where those blocks
// cover every CU): one workgroup per CU walks its XCD's share of the blocks.
// The weight ring and the activation stages run on from one block into the
// next, so the next block's operands load during this block's epilogue; for
// BF16 outputs without residual or split, half of a block's outputs (all of
// them for a GLU weight) wait in LDS and are stored during the next block's
// k-steps, so the output writes of all CUs do not come at once.
//
// Split-K (few blocks: the 1024-row projections at a few hundred to a few
// thousand tokens).  The S workgroups of a block take contiguous k-step
// ranges (multiples of the weight ring) and store their FP32 accumulators to
// a partial buffer [block][split][piece][thread] (coalesced, no epilogue);
// a second kernel (gemm_da_reduce), one workgroup per block and accumulator
// piece, sums the S partials in split order and runs the same epilogue
// per element.  One workgroup reducing a whole block would read S x 128 KB
// through one CU, which measured slower than not splitting.
//
// Buffers.  The weight and activation buffer descriptors start at the
// workgroup's first row / token and end at the operands' end, so rows past
// the end read zeros and per-lane offsets stay fixed; the k-step goes in the
// scalar offset.
//
// Reference operators replaced: the cuBLAS GemmEx / SGEMM projections of the
// batched paths (bf16_gemm.cuh:82-122, cublas_utils.cuh:48-93,
// full_attention_cuda.cu:708-714, linear_attention_cuda.cu:589-615).
#include "qw_stream.hpp"

#ifndef QW_DA_SCHED
#define QW_DA_SCHED 1
#endif

namespace qwk {

namespace {

constexpr int DA_D = 4;        // weight k-steps in flight per wave
constexpr int DA_NS = 4;       // activation stages (row-gather loads: one k-step each)
constexpr int DA_STG = 8192;   // one such stage: 8 token units of 1 KB
constexpr int DA_NS2 = 3;      // activation stages (line loads: two k-steps each)
constexpr int DA_U2 = 1024;    // one 8-token x 64-k unit
constexpr int DA_STG2 = 16 * DA_U2;
constexpr int DA_GROUP_M = 8;  // token blocks per raster group

// Deferred outputs of the persistent kernel: 64 KB of BF16 block outputs
// (GLU: all 128 tokens x 256 rows; plain: tokens 64..127 x 512 rows) kept in
// LDS after a block's K loop and stored during the next block's k-steps.
constexpr int DA_OB = 65536;

template <bool GLU> struct DaEpi {
    static constexpr int ROWS = GLU ? 32 : 64;   // output rows per wave
    static constexpr int PITCH = ROWS + 4;       // floats per staged token
    static constexpr int BYTES = 16 * PITCH * 4; // one 16-token column
    static constexpr int LPT = ROWS / 4;         // lanes per token when reading back
    static constexpr int TPR = 64 / LPT;         // tokens per read
};

// One 1 KB unit global -> LDS with a scalar offset (see lds_dma16).
__device__ __forceinline__ void lds_dma16_so(__amdgpu_buffer_rsrc_t rs, uint8_t* lds_unit, uint32_t voff, int soff) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds_unit;
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs), "s"(soff)
                 : "memory", "m0");
}

// Block `tile` of the grouped raster: DA_GROUP_M token blocks x all weight
// blocks per group, token block fastest -> first token m0, first 16-row tile nt0.
__device__ __forceinline__ void da_tile(const GemmArgs& a, int tile, int& m0, int& nt0, int tiles_per_blk = 16) {
    const int GM = a.group_m > 0 ? a.group_m : DA_GROUP_M;
    const int per_group = GM * a.nblk_n;
    const int group = tile / per_group;
    const int first_m = group * GM;
    const int gm = min(GM, a.nblk_m - first_m);
    const int in_group = tile - group * per_group;
    m0 = (first_m + in_group % gm) * 128;
    nt0 = (in_group / gm) * tiles_per_blk;
}

// Epilogue of one block: accumulator item e of lane l = row 4(l/16)+e of the
// row tile, token l%16 of the token tile.  Per 16-token column the wave stages
// FP32 [token][row] in its private LDS buffer `epw` (silu(gate)*up for a GLU
// weight), then reads 4-row pieces back and stores whole token rows, adding
// the residual and applying the Q/gate split.
template <bool GLU, int J0 = 0, int J1 = 8>
__device__ __forceinline__ void da_epilogue(const GemmArgs& a, const f32x4 (&acc)[4][8], float* epw, int m0, int nt0,
                                            int wave, int lane) {
    using E = DaEpi<GLU>;
    const int g = lane >> 4;
    const bool has_res = (a.flags & EP_RESIDUAL) != 0;
    const bool has_split = (a.flags & EP_SPLIT) != 0;
    const int sp_log = a.split_period > 0 ? 31 - __builtin_clz((unsigned)a.split_period) : 0;
    const int row_w = (GLU ? (nt0 >> 1) : nt0) * 16 + wave * E::ROWS;  // first output row of the wave
    const int rsub = (lane % E::LPT) * 4;
#pragma unroll
    for (int j = J0; j < J1; ++j) {
        float* eb = epw;
#pragma unroll
        for (int i = 0; i < (GLU ? 2 : 4); ++i) {
            f32x4 o;
            if constexpr (GLU) {
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = silu_f(acc[2 * i][j][e]) * acc[2 * i + 1][j][e];
            } else {
                o = acc[i][j];
            }
            *reinterpret_cast<f32x4*>(eb + (lane & 15) * E::PITCH + 16 * i + 4 * g) = o;
        }
#pragma unroll
        for (int c = 0; c < 16 / E::TPR; ++c) {
            const int tok = c * E::TPR + lane / E::LPT;
            f32x4 o = *reinterpret_cast<const f32x4*>(eb + tok * E::PITCH + rsub);
            const int m = m0 + 16 * j + tok;
            const int row = row_w + rsub;
            if (m < a.M && row < a.N) {
                if (has_res) o += load_act4(a.res, a.res_dt, (int64_t)m * a.ld_res + row);
                void* dst = a.y;
                int col = row;
                if (has_split) {  // power-of-two period: shifts only
                    dst = ((row >> sp_log) & 1) ? a.y2 : a.y;
                    col = ((row >> (sp_log + 1)) << sp_log) + (row & (a.split_period - 1));
                }
                store_act4(dst, a.ydt, (int64_t)m * a.ldy + col, o);
            }
        }
    }
}

}  // namespace

// PART: one K split of a block (blockIdx = block * splitk + split after the
// XCD order), partial accumulators out, no epilogue.
// NWV waves (4, or 8 with line loads): 64 * NWV weight rows per block, the
// activation stages shared by all of them.
template <bool GLU, bool LINE, bool PART, int NWV = 4>
__global__ __launch_bounds__(64 * NWV, NWV == 4 ? 2 : 1) void gemm_da_kernel(GemmArgs a) {
    static_assert(NWV == 4 || (NWV == 8 && LINE && !PART), "8 waves: line loads, no split");
    constexpr int QN = 16 / NWV;  // activation units per wave and stage (line loads)
    using E = DaEpi<GLU>;
    constexpr int D = DA_D, NS = LINE ? DA_NS2 : DA_NS;
    constexpr int STG = LINE ? DA_STG2 : DA_STG;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* const epw = reinterpret_cast<float*>(lds + NS * STG + wave * E::BYTES);

    // XCD-aware order (consecutive ids go to different XCDs: give each XCD a
    // contiguous range; the splits of a block are consecutive in it), then
    // the grouped raster
    const int nwg = gridDim.x;
    int b = blockIdx.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    const int S = PART ? a.splitk : 1;
    const int sk = PART ? b % S : 0;
    if constexpr (PART) b /= S;
    int m0, nt0;
    da_tile(a, b, m0, nt0, 4 * NWV);
    const int ks_n = a.ksteps / S;  // k-steps of this split (a multiple of D)
    const int kbase = sk * ks_n;

    const __amdgpu_buffer_rsrc_t wrs =
        make_rsrc(a.w + (size_t)nt0 * a.ksteps * 1024, (uint32_t)((a.n_tiles - nt0) * a.ksteps * 1024));
    const __amdgpu_buffer_rsrc_t xrs =
        make_rsrc(static_cast<const uint16_t*>(a.x) + (size_t)m0 * a.ldx, (uint32_t)((a.M - m0) * a.ldx * 2));
    uint32_t va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = (uint32_t)(((wave * 4 + i) * a.ksteps * 64 + lane) * 16);
    // k-steps past the end reload the last one (never used)
    auto kc = [&](int ks) { return __builtin_amdgcn_readfirstlane(min(ks, ks_n - 1)); };
    u32x4 A[D][4], B[8];
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto loadA = [&](u32x4 (&dst)[4], int ks) {
        const int so = (kbase + kc(ks)) * 1024;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, va[i], so, 0);
    };
    auto mfma_step = [&](int u, const uint8_t* stn, int noff0, int noff1) {
        // column j's B is refilled (k-step ks+1) as soon as its MFMAs are issued
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A[u][i]),
                                                                   __builtin_bit_cast(bf16x8, B[j]), acc[i][j], 0, 0, 0);
            B[j] = *reinterpret_cast<const u32x4*>(stn + j * (LINE ? 2 * DA_U2 : 1024) + (LINE ? noff0 : 0));
        }
#if QW_DA_SCHED
        // keep column j's fragment read right behind its four MFMAs (the
        // scheduler otherwise gathers the eight reads near the end of the
        // step, and the next step's first MFMAs wait for them)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#endif
        __builtin_amdgcn_s_setprio(0);
        (void)noff1;
    };

    if constexpr (!LINE) {
        // one k-step per stage: lane l = r + 16g of unit q loads token r's
        // k 8g..8g+7 (16 rows x 64 B per load)
        uint32_t vb[2];
#pragma unroll
        for (int q = 0; q < 2; ++q)
            vb[q] = (uint32_t)((((wave * 2 + q) * 16 + (lane & 15)) * a.ldx + (lane >> 4) * 8) * 2);
        auto dma = [&](int ks) {
            uint8_t* st = lds + (ks % NS) * STG + wave * 2048;
            const int so = (kbase + kc(ks)) * 64;
#pragma unroll
            for (int q = 0; q < 2; ++q) lds_dma16_so(xrs, st + q * 1024, vb[q], so);
        };
#pragma unroll
        for (int s0 = 0; s0 < NS - 1; ++s0) dma(s0);
#pragma unroll
        for (int d = 0; d < D; ++d) loadA(A[d], d);
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) B[j] = *reinterpret_cast<const u32x4*>(lds + j * 1024 + lane * 16);
        for (int ks0 = 0; ks0 < ks_n; ks0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int ks = ks0 + u;
                // this wave's activation loads of k-step ks+1 have landed
                // (after them came the 4 weight loads of their k-step and 6
                // loads per later one), then the barrier publishes everyone's
                // and frees the stage of ks-1 for k-step ks+NS-1
                __builtin_amdgcn_s_waitcnt(vm_wait(4 + 6 * (NS - 3)));
                __syncthreads();
                dma(ks + NS - 1);
                mfma_step(u, lds + ((ks + 1) % NS) * STG + lane * 16, 0, 0);
                loadA(A[u], ks + D);
            }
        }
    } else {
        // two k-steps (one 128-byte line of each token row) per stage: the
        // two loads (h = 0, 1) of a 16-token tile each take 8 tokens x 8
        // 16-byte chunks; chunk c of token t lands in slot (8c + (t ^ c)) ^ 8h
        // of its unit (lane l of the load takes the chunk of slot l).  A B
        // fragment read (lane = token t + 16 g of k-step s, chunk c = 4s + g)
        // then hits 16 different 16-byte bank groups per 16 lanes: whole-line
        // loads, conflict-free reads
        uint32_t vb[QN];
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            const int unit = wave * QN + q;  // = 2 * token tile + h
            const int sl = lane ^ (8 * (unit & 1));
            const int c_ld = sl >> 3, t_ld = (sl & 7) ^ c_ld;
            vb[q] = (uint32_t)(((unit * 8 + t_ld) * a.ldx + c_ld * 8) * 2);
        }
        auto dma = [&](int p) {  // k-steps 2p, 2p+1
            uint8_t* st = lds + (p % NS) * STG + wave * QN * DA_U2;
            const int so = kbase * 64 + __builtin_amdgcn_readfirstlane(min(p, (ks_n >> 1) - 1)) * 128;
#pragma unroll
            for (int q = 0; q < QN; ++q) lds_dma16_so(xrs, st + q * DA_U2, vb[q], so);
        };
        const int t_rd = lane & 15, g_rd = lane >> 4;
        auto roff = [&](int s) {  // read offset of k-step parity s within a tile's pair of units
            const int c = 4 * s + g_rd;
            return (t_rd >> 3) * DA_U2 + 16 * ((8 * c + ((t_rd & 7) ^ c)) ^ (8 * (t_rd >> 3)));
        };
        const int ro0 = roff(0), ro1 = roff(1);
#pragma unroll
        for (int s0 = 0; s0 < NS; ++s0) dma(s0);
#pragma unroll
        for (int d = 0; d < D; ++d) loadA(A[d], d);
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) B[j] = *reinterpret_cast<const u32x4*>(lds + j * 2 * DA_U2 + ro0);
        for (int ks0 = 0; ks0 < ks_n; ks0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int ks = ks0 + u;
                const int p = ks >> 1;
                if (u & 1) {
                    // second k-step of pair p: our loads of pair p+1 have
                    // landed (after them: 4 weight loads, QN + 8 loads per
                    // later pair, 4 of this pair's first k-step), publish;
                    // pair p's stage is free for pair p+NS
                    __builtin_amdgcn_s_waitcnt(vm_wait(8 + (QN + 8) * (NS - 2)));
                    __syncthreads();
                    dma(p + NS);
                    mfma_step(u, lds + ((p + 1) % NS) * STG, ro0, 0);
                } else {
                    mfma_step(u, lds + (p % NS) * STG, ro1, 0);
                }
                loadA(A[u], ks + D);
            }
        }
    }

    if constexpr (PART) {
        // partial pieces [block][split][piece i*8+j][thread]
        f32x4* pp = reinterpret_cast<f32x4*>(a.partials) + ((size_t)b * S + sk) * 32 * 256 + threadIdx.x;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) pp[(i * 8 + j) * 256] = acc[i][j];
        return;
    }

    da_epilogue<GLU>(a, acc, epw, m0, nt0, wave, lane);
}

// Persistent form of the 8-wave line-load kernel: one workgroup per CU walks
// its XCD's share of the blocks (XCD x = blockIdx % 8 takes blocks
// [x T / 8, (x+1) T / 8) of the grouped raster, slot blockIdx / 8 every
// (gridDim / 8)-th of them).  The weight ring and the activation stages run on
// across blocks: the last k-steps of a block already load the next block's
// first weight k-steps and activation pairs (stage = running pair count mod
// NS), so the next block's operands are in flight while this block's
// epilogue runs, and no block starts from an empty pipeline.
template <bool GLU>
__global__ __launch_bounds__(512, 1) void gemm_da_persist_kernel(GemmArgs a) {
    constexpr int NWV = 8, QN = 2, D = DA_D, NS = DA_NS2, STG = DA_STG2;
    using E = DaEpi<GLU>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* const epw = reinterpret_cast<float*>(lds + NS * STG + wave * E::BYTES);
    uint8_t* const ob = lds + NS * STG + NWV * E::BYTES;  // DA_OB bytes (deferred outputs)

    const int T = a.nblk_n * a.nblk_m;
    const int xcd = blockIdx.x & 7, nslot = gridDim.x >> 3;
    const int hi = (int)(((long long)(xcd + 1) * T) >> 3);
    int t = (int)(((long long)xcd * T) >> 3) + (int)(blockIdx.x >> 3);
    if (t >= hi) return;
    const int ks_n = a.ksteps, P = ks_n >> 1;  // k-steps and activation pairs per block

    auto rsrcs = [&](int tile, __amdgpu_buffer_rsrc_t& wr, __amdgpu_buffer_rsrc_t& xr, int& m0, int& nt0) {
        da_tile(a, tile, m0, nt0, 4 * NWV);
        wr = make_rsrc(a.w + (size_t)nt0 * a.ksteps * 1024, (uint32_t)((a.n_tiles - nt0) * a.ksteps * 1024));
        xr = make_rsrc(static_cast<const uint16_t*>(a.x) + (size_t)m0 * a.ldx, (uint32_t)((a.M - m0) * a.ldx * 2));
    };
    int m0, nt0, m0n, nt0n;
    __amdgpu_buffer_rsrc_t wrs, xrs, wrn, xrn;
    rsrcs(t, wrs, xrs, m0, nt0);
    int tn = t + nslot;
    if (tn < hi) rsrcs(tn, wrn, xrn, m0n, nt0n);
    else { wrn = wrs; xrn = xrs; m0n = m0; nt0n = nt0; }

    uint32_t va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = (uint32_t)(((wave * 4 + i) * a.ksteps * 64 + lane) * 16);
    uint32_t vb[QN];
#pragma unroll
    for (int q = 0; q < QN; ++q) {
        const int unit = wave * QN + q;
        const int sl = lane ^ (8 * (unit & 1));
        const int c_ld = sl >> 3, t_ld = (sl & 7) ^ c_ld;
        vb[q] = (uint32_t)(((unit * 8 + t_ld) * a.ldx + c_ld * 8) * 2);
    }
    const int t_rd = lane & 15, g_rd = lane >> 4;
    auto roff = [&](int s) {
        const int c = 4 * s + g_rd;
        return (t_rd >> 3) * DA_U2 + 16 * ((8 * c + ((t_rd & 7) ^ c)) ^ (8 * (t_rd >> 3)));
    };
    const int ro0 = roff(0), ro1 = roff(1);

    u32x4 A[D][4], B[8];
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // k-step ks of the current block; ks >= ks_n: k-step ks - ks_n of the next
    auto loadA = [&](u32x4 (&dst)[4], int ks) {
        const bool nx = ks >= ks_n;
        const __amdgpu_buffer_rsrc_t r = nx ? wrn : wrs;
        const int so = __builtin_amdgcn_readfirstlane((nx ? ks - ks_n : ks) * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = __builtin_amdgcn_raw_buffer_load_b128(r, va[i], so, 0);
    };
    // activation pair p of the current block (p >= P: pair p - P of the next)
    // into stage (gp + p) % NS, gp = pairs of the earlier blocks
    int gp = 0;
    auto dma = [&](int p) {
        const bool nx = p >= P;
        const __amdgpu_buffer_rsrc_t r = nx ? xrn : xrs;
        uint8_t* st = lds + ((gp + p) % NS) * STG + wave * QN * DA_U2;
        const int so = __builtin_amdgcn_readfirstlane((nx ? p - P : p) * 128);
#pragma unroll
        for (int q = 0; q < QN; ++q) lds_dma16_so(r, st + q * DA_U2, vb[q], so);
    };
    auto mfma_step = [&](int u, const uint8_t* stn, int noff) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A[u][i]),
                                                                   __builtin_bit_cast(bf16x8, B[j]), acc[i][j], 0, 0, 0);
            B[j] = *reinterpret_cast<const u32x4*>(stn + j * 2 * DA_U2 + noff);
        }
#if QW_DA_SCHED
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#endif
        __builtin_amdgcn_s_setprio(0);
    };

    // Deferred outputs (BF16 output rows, no residual or split, K >= 1024):
    // token tk of the deferred range keeps its RB-byte output row at
    // ob + tk * RB, 16-byte chunk c stored at chunk c ^ (tk & 15), so the
    // epilogue's 8-byte writes (16 tokens per 16 lanes) and the row reads
    // (64 chunks of one or two rows) hit distinct banks.  Wave w stores its
    // 8 pieces (one 1 KB store each) at k-steps 2, 6, .., 30 of the next
    // block, after that block's first barrier, and all before its epilogue.
    constexpr int RB = GLU ? 512 : 1024;  // bytes of one token's output row in a block
    constexpr int DT0 = GLU ? 0 : 64;     // first deferred token of a block
    const bool defer = (a.flags & (EP_RESIDUAL | EP_SPLIT)) == 0 && a.ydt == DT_BF16 && ks_n >= 32 &&
                       (a.N & 7) == 0 && (a.ldy & 7) == 0 && a.vec_store &&  // 16-byte aligned row pieces
                       (long long)a.M * a.ldy * 2 < 0x7ffffff0ll;  // the dropped-store offset lies past every row
    bool pending = false;
    int pm0 = 0, prow0 = 0;  // first token / output row of the block in ob
    auto ob_put = [&]() {
        const int g = lane >> 4;
#pragma unroll
        for (int j = DT0 / 16; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < (GLU ? 2 : 4); ++i) {
                f32x4 o;
                if constexpr (GLU) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = silu_f(acc[2 * i][j][e]) * acc[2 * i + 1][j][e];
                } else {
                    o = acc[i][j];
                }
                const int tk = 16 * j + (lane & 15) - DT0;
                const int row = wave * E::ROWS + 16 * i + 4 * g;
                u32x2 w;
                w[0] = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
                w[1] = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
                *reinterpret_cast<u32x2*>(ob + tk * RB + ((((row >> 3) ^ (tk & 15))) << 4) + (row & 7) * 2) = w;
            }
    };
    // Piece k (0..7) of this wave, without branches: the store goes through a
    // buffer descriptor over the block's output rows, 0 bytes long when
    // nothing is pending (or the piece is past the eighth), and rows past N
    // take an offset past the end, so the hardware drops those stores.
    auto ob_store = [&](int k, bool act) {
        const int tk = GLU ? wave * 16 + 2 * k + (lane >> 5) : wave * 8 + k;
        const int c = GLU ? (lane & 31) : lane;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ob + tk * RB + ((c ^ (tk & 15)) << 4));
        const int mb = pm0 + DT0;  // first token of the deferred range
        const int nrec = act ? (a.M - mb) * a.ldy * 2 : 0;
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(static_cast<uint16_t*>(a.y) + (size_t)mb * a.ldy, (uint32_t)max(nrec, 0));
        const int row = prow0 + 8 * c;
        const uint32_t off = row < a.N ? (uint32_t)((tk * a.ldy + row) * 2) : 0x7ffffff0u;
        __builtin_amdgcn_raw_buffer_store_b128(v, yr, off, 0, 0);
    };

    // pipeline fill for the first block
#pragma unroll
    for (int s0 = 0; s0 < NS; ++s0) dma(s0);
#pragma unroll
    for (int d = 0; d < D; ++d) loadA(A[d], d);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) B[j] = *reinterpret_cast<const u32x4*>(lds + j * 2 * DA_U2 + ro0);

    for (;;) {
        for (int ks0 = 0; ks0 < ks_n; ks0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int ks = ks0 + u;
                const int p = ks >> 1;
                if (u & 1) {
                    // second k-step of pair p: our loads of pair p+1 have landed
                    // (after them: 4 weight loads, QN + 8 loads per later pair, 4 of
                    // this pair's first k-step), publish; pair p's stage is free
                    __builtin_amdgcn_s_waitcnt(vm_wait(8 + (QN + 8) * (NS - 2)));
                    __syncthreads();
                    dma(p + NS);
                    mfma_step(u, lds + ((gp + p + 1) % NS) * STG, ro0);
                } else {
                    mfma_step(u, lds + ((gp + p) % NS) * STG, ro1);
                }
                loadA(A[u], ks + D);
                if (u == 2) ob_store((ks0 >> 2) & 7, pending && ks0 < 32);
            }
        }
        // the next block's first D weight k-steps, NS activation pairs and its
        // first B fragments are in flight or loaded; this block's epilogue
        // overlaps them
        if (defer) {
            if constexpr (!GLU) da_epilogue<GLU, 0, DT0 / 16>(a, acc, epw, m0, nt0, wave, lane);
            ob_put();
            pending = true;
            pm0 = m0;
            prow0 = (GLU ? (nt0 >> 1) : nt0) * 16;
        } else {
            da_epilogue<GLU>(a, acc, epw, m0, nt0, wave, lane);
        }
        if (tn >= hi) {
            if (pending) {
                __syncthreads();
#pragma unroll
                for (int k = 0; k < 8; ++k) ob_store(k, true);
            }
            // no direct-to-LDS load may land after the workgroup has exited
            __builtin_amdgcn_s_waitcnt(vm_wait(0));
            break;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        gp += P;
        t = tn;
        wrs = wrn; xrs = xrn; m0 = m0n; nt0 = nt0n;
        tn = t + nslot;
        if (tn < hi) rsrcs(tn, wrn, xrn, m0n, nt0n);
    }
}

// The split-K epilogue: workgroup (block, piece) sums the S partial pieces of
// its 256 threads in split order and stores them as gemm_da_kernel's epilogue
// would (the GLU pairs gate piece 2i with up piece 2i+1 of the same column).
template <bool GLU>
__global__ __launch_bounds__(256) void gemm_da_reduce(GemmArgs a) {
    constexpr int PP = GLU ? 16 : 32;  // output pieces per block
    const int blk = blockIdx.x / PP, q = blockIdx.x % PP;
    const int i = q / 8, j = q % 8;    // row tile (pair for GLU) and token column
    const int S = a.splitk;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const f32x4* pp = reinterpret_cast<const f32x4*>(a.partials) + (size_t)blk * S * 32 * 256 + tid;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    const int p0 = GLU ? (2 * i) * 8 + j : i * 8 + j, p1 = (2 * i + 1) * 8 + j;
    for (int sp = 0; sp < S; ++sp) {
        s0 += pp[((size_t)sp * 32 + p0) * 256];
        if (GLU) s1 += pp[((size_t)sp * 32 + p1) * 256];
    }
    f32x4 o;
    if constexpr (GLU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = silu_f(s0[e]) * s1[e];
    } else {
        o = s0;
    }
    int m0, nt0;
    da_tile(a, blk, m0, nt0);
    const int rows_w = GLU ? 32 : 64;
    const int row = (GLU ? (nt0 >> 1) : nt0) * 16 + wave * rows_w + i * 16 + 4 * g;
    const int m = m0 + 16 * j + (lane & 15);
    if (m < a.M && row < a.N) {
        if (a.flags & EP_RESIDUAL) o += load_act4(a.res, a.res_dt, (int64_t)m * a.ld_res + row);
        void* dst = a.y;
        int col = row;
        if (a.flags & EP_SPLIT) {
            const int sp_log = 31 - __builtin_clz((unsigned)a.split_period);
            dst = ((row >> sp_log) & 1) ? a.y2 : a.y;
            col = ((row >> (sp_log + 1)) << sp_log) + (row & (a.split_period - 1));
        }
        store_act4(dst, a.ydt, (int64_t)m * a.ldy + col, o);
    }
}

bool gemm_da_fits(const GemmArgs& a, int wf, int xdt, bool argmax) {
    if (a.ldx % 8 != 0) return false;  // 16-byte activation chunks
    if (wf != WF_BF16 || xdt != DT_BF16 || argmax || a.splitk > 1) return false;
    if (a.N % 4 != 0 || !a.vec_store) return false;
    if ((a.flags & EP_SPLIT) && (a.split_period < 4 || (a.split_period & (a.split_period - 1)) != 0)) return false;
    if ((uint64_t)a.M * a.ldx * 2 >= (1ull << 31) || (uint64_t)a.n_tiles * a.ksteps * 1024 >= (1ull << 31)) return false;
    return a.ksteps % DA_D == 0;
}

size_t gemm_da_lds_bytes(bool glu, bool line, int nwv) {
    return (size_t)(line ? DA_NS2 * DA_STG2 : DA_NS * DA_STG) + nwv * (glu ? DaEpi<true>::BYTES : DaEpi<false>::BYTES);
}

hipError_t launch_gemm_da(const GemmArgs& a, bool glu, bool line, hipStream_t stream, int nwv, int persist_wgs) {
    if (nwv == 8 && !line) nwv = 4;
    GemmArgs b = a;
    const int rows = 64 * nwv;
    b.nblk_n = (a.n_tiles * 16 + rows - 1) / rows;
    b.nblk_m = (a.M + 127) / 128;
    int grid = b.nblk_n * b.nblk_m;
    const size_t lds = gemm_da_lds_bytes(glu, line, nwv);
    if (nwv == 8 && persist_wgs >= 8) {
        // one workgroup per CU, a multiple of 8 (each XCD's share of the blocks)
        const int slots = std::min((grid + 7) / 8, persist_wgs / 8);
        auto kp = glu ? gemm_da_persist_kernel<true> : gemm_da_persist_kernel<false>;
        const size_t lds_p = lds + DA_OB;
        hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(kp), (int)lds_p);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kp, dim3(8 * slots), dim3(512), lds_p, stream, b);
        return hipGetLastError();
    }
    auto go = [&](auto k) {
        {
            hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k, dim3(grid), dim3(64 * nwv), lds, stream, b);
        return hipGetLastError();
    };
    if (nwv == 8) return glu ? go(gemm_da_kernel<true, true, false, 8>) : go(gemm_da_kernel<false, true, false, 8>);
    if (line) return glu ? go(gemm_da_kernel<true, true, false>) : go(gemm_da_kernel<false, true, false>);
    return glu ? go(gemm_da_kernel<true, false, false>) : go(gemm_da_kernel<false, false, false>);
}

size_t gemm_da_split_bytes(const GemmArgs& a, int S) {
    return (size_t)((a.n_tiles * 16 + 255) / 256) * ((a.M + 127) / 128) * S * 32 * 256 * 16;
}

hipError_t launch_gemm_da_split(const GemmArgs& a, bool glu, bool line, int S, hipStream_t stream) {
    if (S < 2 || a.ksteps % (DA_D * S) != 0 || !a.partials) return hipErrorInvalidValue;
    GemmArgs b = a;
    b.nblk_n = (a.n_tiles * 16 + 255) / 256;
    b.nblk_m = (a.M + 127) / 128;
    b.splitk = S;
    const int blocks = b.nblk_n * b.nblk_m;
    const size_t lds = gemm_da_lds_bytes(glu, line, 4);
    auto go = [&](auto k) {
        {
            hipError_t e = ensure_max_lds(reinterpret_cast<const void*>(k), (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k, dim3(blocks * S), dim3(256), lds, stream, b);
        return hipGetLastError();
    };
    hipError_t e = line ? (glu ? go(gemm_da_kernel<true, true, true>) : go(gemm_da_kernel<false, true, true>))
                        : (glu ? go(gemm_da_kernel<true, false, true>) : go(gemm_da_kernel<false, false, true>));
    if (e != hipSuccess) return e;
    if (glu) hipLaunchKernelGGL(gemm_da_reduce<true>, dim3(blocks * 16), dim3(256), 0, stream, b);
    else hipLaunchKernelGGL(gemm_da_reduce<false>, dim3(blocks * 32), dim3(256), 0, stream, b);
    return hipGetLastError();
}

}  // namespace qwk
