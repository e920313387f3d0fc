// qw_gemm.hip -- LDS double-buffered MFMA GEMM for gfx950 (prefill and
// large-batch decode):  y[m][n] = sum_k W[n][k] * x[m][k]  (+ epilogue).
//
// Tiling.  A workgroup (4 waves) computes 256 weight rows x 256 tokens; each
// wave a 128 x 128 quadrant as 4 x 4 blocks of v_mfma_f32_32x32x16_bf16
// (weights are the A operand, tokens the B operand; FP32 accumulators).  K
// advances in blocks of 64.
//
// Loads.  Both operands reach LDS through direct buffer->LDS loads
// (buffer_load_dwordx4 ... lds): one wave instruction moves one 1 KB unit.
// The weights are already stored in the packed tile order (qw_device.hpp),
// and the activations are fetched so that they land in the same order: lane
// (r, g) of a unit carries x[token r][8 k starting at group g].  A 32 x 32 x 16
// fragment of either operand is then one conflict-free ds_read_b128 per lane.
// Two LDS stages (2 x 64 KB) let the loads of K-block i+1 fly while K-block i
// is multiplied.
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

constexpr int GB_N = 256, GB_M = 256;      // block tile: weight rows x tokens
constexpr int G_STAGE = 64 * 1024;         // bytes per LDS stage
constexpr int G_XOFF = 32 * 1024;          // activation region within a stage
constexpr int G_EPI_PITCH = 68;            // epilogue LDS row pitch (floats): 64 rows + pad

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds_unit, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds_unit, 16, voff, 0, 0, 0);
}

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

template <bool GLU, bool ARGMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_bf16_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ unsigned long long best_s[2][GB_M];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wn = wave >> 1, wm = wave & 1;   // quadrant of this wave

    // XCD-aware order: consecutive workgroup ids go to different XCDs; give
    // each XCD a contiguous range of tiles (M fastest) so the tiles that
    // share a weight block run on the same L2.
    const int nwg = gridDim.x;
    int b = blockIdx.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    const int bm = b % a.nblk_m, bn = b / a.nblk_m;
    const int nt0 = bn * (GB_N / 16);          // first physical 16-row tile
    const int m0 = bm * GB_M;

    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)((uint64_t)a.n_tiles * a.ksteps * 1024u));
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * a.ldx * 2u));
    const int nkb = a.ksteps / 2;

    // The 16 units this wave moves per K-block: waves 0,1 the 32 weight units
    // (16 tiles x 2 k-steps), waves 2,3 the 32 activation units (16 token
    // groups x 2 k-steps); unit u lands at byte u*1024 of the stage either
    // way.  Offsets for K-block 0 are computed once; K-block kb adds kb*kstep.
    const bool wrole = wave < 2;
    const __amdgpu_buffer_rsrc_t rs = wrole ? wrs : xrs;
    const uint32_t kstep = wrole ? 2048u : 128u;
    uint32_t vbase[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int v = (wave & 1) * 16 + q;  // unit within the role
        const int t = v >> 1, ks = v & 1;
        if (wrole) {
            const int pt = nt0 + t;
            vbase[q] = pt < a.n_tiles ? (uint32_t)((pt * a.ksteps + ks) * 1024 + lane * 16) : OOB;
        } else {
            const int row = m0 + t * 16 + (lane & 15);
            vbase[q] = row < a.M ? (uint32_t)((row * a.ldx + ks * 32 + (lane >> 4) * 8) * 2) : OOB;
        }
    }
    auto issue = [&](int kb, int stage) {
        uint8_t* st = lds + stage * G_STAGE + wave * 16 * 1024;
        const uint32_t add = (uint32_t)kb * kstep;
#pragma unroll
        for (int q = 0; q < 16; ++q) lds_dma16(rs, st + q * 1024, vbase[q] + add);
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    // lane -> fragment address within a (tile pair, k-step) unit: row l%32 of
    // a 32-row block = tile (l%32)/16, row l%16; k-group 2h + l/32
    const int frag_tile = (lane & 31) >> 4;
    const int frag_off = ((lane & 15) + 16 * (lane >> 5)) * 16;  // + 32*16*h

    // fragments of sub-step s = 2*ks + h of a K-block
    bf16x8 A[2][4], B[2][4];
    auto read_frags = [&](const uint8_t* st, int sub, bf16x8 (&Ad)[4], bf16x8 (&Bd)[4]) {
        const int ks = sub >> 1, h = sub & 1;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const int t = wn * 8 + nb * 2 + frag_tile;
            Ad[nb] = *reinterpret_cast<const bf16x8*>(st + (t * 2 + ks) * 1024 + frag_off + h * 512);
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int t = wm * 8 + mb * 2 + frag_tile;
            Bd[mb] = *reinterpret_cast<const bf16x8*>(st + G_XOFF + (t * 2 + ks) * 1024 + frag_off + h * 512);
        }
    };

    // Software pipeline: the fragments of the next sub-step are read from LDS
    // while the 16 MFMAs of the current one run; the global->LDS loads of
    // K-block kb+1 are in flight during all of K-block kb.
    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    read_frags(lds, 0, A[0], B[0]);
    for (int kb = 0; kb < nkb; ++kb) {
        const uint8_t* st = lds + (kb & 1) * G_STAGE;
        if (kb + 1 < nkb) issue(kb + 1, (kb + 1) & 1);
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            const int cur = sub & 1;
            if (sub < 3) {
                read_frags(st, sub + 1, A[cur ^ 1], B[cur ^ 1]);
            } else {
                // stage kb+1 complete and every wave done with stage kb
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                if (kb + 1 < nkb) read_frags(lds + ((kb + 1) & 1) * G_STAGE, 0, A[cur ^ 1], B[cur ^ 1]);
            }
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[cur][nb], B[cur][mb], acc[nb][mb], 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);
        }
    }

    // ---- epilogue ----
    // accumulator item q of lane l: weight row i = 8*(q/4) + 4*(l/32) + q%4 of
    // the 32-row block, token j = l%32 of the 32-token block
    const int ihi = 4 * (lane >> 5);
    if constexpr (ARGMAX) {
        unsigned long long best[4] = {0ull, 0ull, 0ull, 0ull};
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const int pt0 = nt0 + wn * 8 + nb * 2;
#pragma unroll
            for (int qg = 0; qg < 4; ++qg) {
                const int row = pt0 * 16 + 8 * qg + ihi;
                f32x4 sc = {1.f, 1.f, 1.f, 1.f};
                if (a.scales) sc = *reinterpret_cast<const f32x4*>(a.scales + row);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
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
        for (int mb = 0; mb < 4; ++mb) {
            const unsigned long long o = __shfl_xor(best[mb], 32);
            best[mb] = o > best[mb] ? o : best[mb];
            if (lane < 32) best_s[wn][wm * 128 + mb * 32 + lane] = best[mb];
        }
        __syncthreads();
        if (threadIdx.x < GB_M) {
            const int j = threadIdx.x;
            unsigned long long k0 = best_s[0][j], k1 = best_s[1][j];
            const unsigned long long kk = k0 > k1 ? k0 : k1;
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
            for (int m = threadIdx.x; m < a.M; m += 256) {
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
        // with constants.  GLU: the wave's 64 output rows in one pass; plain:
        // its 128 rows in two passes of 64.
        float* ep = reinterpret_cast<float*>(lds) + wave * (128 * G_EPI_PITCH);
        const int row_base = GLU ? ((nt0 + wn * 8) >> 1) * 16 : (nt0 + wn * 8) * 16;
        const int tok_base = m0 + wm * 128;
        const bool has_res = (a.flags & EP_RESIDUAL) != 0;
        const bool has_split = (a.flags & EP_SPLIT) != 0;
        const int sp_log = a.split_period > 0 ? 31 - __builtin_clz((unsigned)a.split_period) : 0;
        __syncthreads();  // every wave is done reading the K-loop stages
#pragma unroll
        for (int pass = 0; pass < (GLU ? 1 : 2); ++pass) {
#pragma unroll
            for (int nbl = 0; nbl < (GLU ? 4 : 2); ++nbl) {
                const int nb = GLU ? nbl : pass * 2 + nbl;
                const int pt0 = nt0 + wn * 8 + nb * 2;
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
                    for (int mb = 0; mb < 4; ++mb) {
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
            const int c = lane & 15;  // rows 4c .. 4c+3
            const int row = row_base + pass * 64 + 4 * c;
            for (int it = 0; it < 32; ++it) {
                const int jj = it * 4 + (lane >> 4);
                const int m = tok_base + jj;
                if (m < a.M && row < a.N) {
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
            if (!GLU && pass == 0) {
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
}

size_t gemm_lds_bytes() {
    const size_t epi = 4 * 128 * G_EPI_PITCH * sizeof(float);
    return epi > 2 * (size_t)G_STAGE ? epi : 2 * (size_t)G_STAGE;
}

template <typename Kern>
static hipError_t launch_gemm_k(Kern k, const GemmArgs& a, int grid, hipStream_t st) {
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_lds_bytes());
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(256), gemm_lds_bytes(), st, a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& a, int wf, int xdt, bool glu, bool argmax, hipStream_t stream) {
    if (wf != WF_BF16 || xdt != DT_BF16) return hipErrorInvalidValue;
    if (a.ksteps % 2 != 0) return hipErrorInvalidValue;
    if (argmax && glu) return hipErrorInvalidValue;
    const int grid = a.nblk_n * a.nblk_m;
    if (argmax) return launch_gemm_k(gemm_bf16_kernel<false, true>, a, grid, stream);
    if (glu) return launch_gemm_k(gemm_bf16_kernel<true, false>, a, grid, stream);
    return launch_gemm_k(gemm_bf16_kernel<false, false>, a, grid, stream);
}

}  // namespace qwk
