// qw_kernels.hpp -- host-visible launch descriptors of the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qwk {

// Maximum dynamic LDS of a kernel.  The attribute is not a stream operation,
// so it is set in the relaxed capture mode: a first launch of a kernel inside
// a thread's stream capture (qw_graph_begin) must not invalidate the capture.
inline hipError_t set_max_lds(const void* kernel, int bytes) {
    hipStreamCaptureMode m = hipStreamCaptureModeRelaxed;
    const hipError_t e0 = hipThreadExchangeStreamCaptureMode(&m);
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e0 == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&m);
    return e;
}

// set_max_lds once per (kernel, size): a thread-safe table keyed on the
// kernel's address remembers the largest size set, so each instantiation is
// configured before its first launch and again when a launch asks for more.
hipError_t ensure_max_lds(const void* kernel, int bytes);


// One skinny (small-M) projection launch.  See qw_skinny.hip.
struct SkinnyArgs {
    const uint8_t* w;        // packed weight (tile order)
    const float* scales;     // per physical row (INT8) or nullptr
    const void* x;           // activations [M][ldx]
    int ldx;
    int M;                   // tokens
    int K;                   // inputs (multiple of 64)
    int N;                   // logical output rows (GLU: rows of the pair)
    int n_groups;            // logical 16-row output tiles
    int S;                   // k splits per tile
    int ksteps;              // K / (4*KE)
    int n_items;             // n_groups * S
    unsigned flags;          // QW_EP_* bits
    const void* res;         // residual [M][ld_res]
    int res_dt;
    int ld_res;
    const float* gamma;      // RMSNorm weight [K]
    float eps;
    void* y;                 // output [M][ldy]
    int ydt;
    int ldy;
    void* y2;                // split output
    int split_period;
    int vec_store;           // 1: 4-wide stores are aligned
    float4* partials;        // split-K partial tiles
    unsigned* counters;      // split-K arrival counters, one per tile (self-resetting)
    unsigned long long* keys;  // argmax keys [M] (self-resetting)
    unsigned* done;          // argmax completion counter (self-resetting)
    int32_t* ids;            // argmax ids [M]
    float* maxv;             // argmax values [M] or nullptr
    int tg_size;             // token-group height (tokens per group); 0: one group
    int tg_grid;             // workgroups per token group; 0: one group
};

// LDS the skinny kernel stages its activations in: (M+1) rows of the split's
// K range in the MFMA input type (two planes when an FP32 activation feeds a
// 16-bit MFMA), each row padded by 16 bytes.
constexpr size_t kSkinnyMaxLds = 136 * 1024;
size_t skinny_lds_bytes(int wf, int xdt, int M, int ksteps_per_split);

// Register-direct decode GEMV (qw_gemv.hip): M <= 32; BF16 weights with BF16
// activations, INT8 weights with F16 or BF16 activations.
bool gemv_supported(int wf, int xdt, int M, bool norm);
// consecutive 16-row tiles per argmax item of the GEMV
int gemv_argmax_tiles(int wf);
// workgroup size (waves) the GEMV instantiates closest to the one wanted
int gemv_waves(int wf, int M, bool glu, bool argmax, bool norm, int nw_wanted);
hipError_t launch_gemv(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int nw, int grid,
                       hipStream_t stream);

// nw: waves per workgroup (4 or 16)
hipError_t launch_skinny(const SkinnyArgs& a, int wf, int xdt, bool glu, bool argmax, int nw, int grid,
                         hipStream_t stream);

// Weight-stationary projection for 17..512 tokens (qw_wide.hip): BF16
// weights with BF16 activations, INT8 weights with F16 activations; no
// argmax.  The host plans the K splits and the workgroup shape (wide_plan).
constexpr size_t kWideMaxLds = 144 * 1024;
constexpr int kWideMaxM = 512;
struct WideArgs {
    SkinnyArgs s;      // operands, epilogue, split count (s.S), counters and partials
    int nblocks;       // blocks of two physical 16-row tiles (GLU: one gate/up pair)
    int n_ptiles;      // physical tiles of the packed weight
    int off_gamma;     // LDS offsets of the norm-weight slice, residual tiles, scales
    int off_res;
    int off_scales;
    int res_lds;       // 1: the residual is staged in LDS (4-wide aligned path)
    int T;             // token groups (each Mg tokens, its own workgroups)
    int Mg;
    int ngrp;          // block groups (NB blocks each; a multiple of 8 when T > 1)
    int dbg;           // timing probes only (wrong results): 1 no MFMAs, 2 no split-K hand-off, 4 no staging
    float4* wpart;     // split-K partials of this kernel, every word kWideSentinel between launches
    unsigned* err;     // device error flag (a split's partial never arrived)
};
// The bit pattern of an empty partials word.  No partial sum of products of
// 16-bit operands has it (their NaN payloads leave the low 13 bits zero), and
// the producers map it to the canonical NaN anyway.
constexpr uint32_t kWideSentinel = 0xffffffffu;
struct WidePlan {
    int S, T, Mg, ngrp, NB, KW, CT, grid;
    size_t smem;
    int off_gamma, off_res, off_scales, nblocks, n_ptiles, res_lds;
};
bool wide_supported(int wf, int xdt, int M);
// false when no configuration fits (LDS, workspace); force_s / force_cfg
// (1..3: 4x1, 2x2, 1x4 blocks x waves per block) pin the choice when nonzero
bool wide_plan(const SkinnyArgs& s, int wf, bool glu, int num_cus, size_t partials_cap, int max_counters, int force_s,
               int force_cfg, WidePlan& p);
hipError_t launch_wide(const WideArgs& a, const WidePlan& p, int wf, int xdt, bool glu, hipStream_t stream);

// Tied lm_head + greedy argmax, weight-stationary (qw_wide.hip), 1..256 tokens.
struct WideArgmaxArgs {
    const uint8_t* w;          // packed E (non-GLU)
    const float* scales;       // INT8 per-row scales or nullptr
    const void* x;             // [M][ldx] hidden states
    int ldx, M, K, V;
    int n_tiles, n_blk;        // 16-row tiles, 32-row blocks
    int ksteps;
    int T, Mg, CT;             // token groups of Mg tokens, CT 16-token tiles each
    int nw;                    // waves per workgroup (4 or 8; 0: the plan chooses)
    int wcache;                // weight loads: 1 default cache policy, 0 non-temporal, -1 the plan chooses
    unsigned long long* keys;  // [M] (self-resetting)
    unsigned* done;            // completion counter (self-resetting)
    int32_t* ids;
    float* maxv;
    int dbg;                   // timing probes only (wrong results): 1 no MFMAs
};
bool wide_argmax_plan(int wf, int xdt, int M, int K, int num_cus, WideArgmaxArgs& a, int& grid, size_t& smem);
hipError_t launch_wide_argmax(const WideArgmaxArgs& a, int wf, int xdt, int grid, size_t smem, hipStream_t stream);
// The activation-stationary form (BF16 E, 65..128 tokens, K = 1024): E
// streamed once through an LDS ring, each wave holding one token tile's
// activations; false where it does not apply.
bool as_argmax_plan(int wf, int xdt, int M, int K, int num_cus, int& grid, size_t& smem);
hipError_t launch_as_argmax(const WideArgmaxArgs& a, int wf, int xdt, int grid, size_t smem, hipStream_t stream);

// LDS double-buffered MFMA GEMM for many tokens (qw_gemm.hip).
struct GemmArgs {
    const uint8_t* w;        // packed weight
    const float* scales;     // per physical row (INT8) or nullptr
    int n_tiles;             // physical 16-row tiles
    int ksteps;              // k-steps of the packed weight
    const void* x;           // activations [M][ldx]
    int ldx;
    int M, K, N;             // N: logical output rows
    int nblk_n, nblk_m;      // block grid: `rows` weight rows x tile_m tokens
    int rows;                // weight rows per block: 256, or 64 (tile_m 128)
    int tile_m;              // tokens per block: 256 or 128
    int waves;               // waves per workgroup: 4, or 8 (tile_m 256 only)
    unsigned flags;
    const void* res;
    int res_dt, ld_res;
    void* y;
    int ydt, ldy;
    void* y2;
    int split_period;
    int vec_store;
    unsigned long long* keys;
    unsigned* done;
    int32_t* ids;
    float* maxv;
    int splitk;              // K splits per tile (1: none; not with argmax)
    float* partials;         // split-K partial tiles [tiles][splitk][threads][acc floats]
    unsigned* counters;      // split-K arrival counters per tile (self-resetting)
    int group_m;             // direct-A kernel: token blocks per raster group (0: 8)
};
int gemm_acc_floats_per_thread(int rows, int tile_m, int waves);
bool gemm_supported(int wf, int xdt);
hipError_t launch_gemm(const GemmArgs& a, int wf, int xdt, bool glu, bool argmax, hipStream_t stream);
// Direct-A GEMM (qw_gemm_da.hip): BF16 x BF16, 256-row x 128-token blocks,
// two workgroups per CU; plain, GLU, residual and split epilogues.
bool gemm_da_fits(const GemmArgs& a, int wf, int xdt, bool argmax);
size_t gemm_da_lds_bytes(bool glu, bool line, int nwv);
// line: activation loads of whole 128-byte row lines (two k-steps, swizzled
// into LDS) instead of 64-byte row pieces
// persist_wgs >= 8 with nwv 8: the persistent form, at most persist_wgs
// workgroups (one per CU)
hipError_t launch_gemm_da(const GemmArgs& a, bool glu, bool line, hipStream_t stream, int nwv = 4, int persist_wgs = 0);
// split-K form: S K splits (a.ksteps a multiple of 4 S) into a.partials
// (gemm_da_split_bytes), then the reduce + epilogue kernel
size_t gemm_da_split_bytes(const GemmArgs& a, int S);
hipError_t launch_gemm_da_split(const GemmArgs& a, bool glu, bool line, int S, hipStream_t stream);

// Fused MLP block in one launch (qw_mlp.hip): `up` is the gate/up GLU pass
// (x -> h, y = the h buffer), `down` the down pass (h -> y).
struct MlpArgs {
    SkinnyArgs up;
    SkinnyArgs down;
    unsigned* ctl;   // [3]: error flag (a wait that expired)
    unsigned* cnt;   // completion / exit counter slots, zero between launches (mlp_counter_words())
    int n_up;
    int n_down;
    // optional out-projection ahead of the block (qw_layer_tail): pre.w != null
    // -> x_mid = x + pre.w . pre.x (FP32 x only) written to xmid [M][H], and the
    // block runs on x_mid with x_mid as its residual
    SkinnyArgs pre;
    float* xmid;
};
// largest k-step count per projection the one-launch MLP holds in registers
// (0: weight format not supported)
int mlp_fused_max_ksteps(int wf, bool down);
int mlp_counter_words();
int mlp_pre_max_ksteps(int wf);  // k-steps of the out-projection stage (qw_layer_tail)
int mlp_fused_max_m(int xdt);  // tokens the one-launch MLP takes for activations of this dtype
hipError_t launch_mlp_fused(const MlpArgs& p, int wf, int xdt, hipStream_t stream);

// L consecutive MLP blocks in one persistent launch (qw_mlpstack.hip), decode
// (M <= mlp_stack_max_m() tokens) at H = 1024, I = 3584, on 256 resident
// workgroups; x and y [M][1024] in the activation dtype (y may alias x).
constexpr int kMlpStackMaxLayers = 48;
struct MlpStackArgs {
    const uint8_t* gu[kMlpStackMaxLayers];        // packed GLU gate/up weights
    const uint8_t* dn[kMlpStackMaxLayers];        // packed down weights
    const float* gu_scales[kMlpStackMaxLayers];   // INT8 per-row scales (physical rows)
    const float* dn_scales[kMlpStackMaxLayers];
    const float* gamma[kMlpStackMaxLayers];       // RMSNorm weights (all NULL: folded into gate/up)
    const void* x;
    void* y;
    int M, L;
    float eps;
    uint64_t* hbuf;     // hand-off words, mlp_stack_ws_bytes() zeroed once (h words, then the x words)
    uint64_t* xbuf;     // set by launch_mlp_stack
    unsigned* epoch;    // [3]: launch epoch (advanced by every launch), abort word, wrap barrier counter
    unsigned* err;      // device error flag
    int dbg;            // timing probes (wrong results): 1 no gate/up weight loads, 2 no down weight loads
    int gap;            // 100 MHz ticks between the k-steps of a gate/up group's weight requests
    uint64_t* trace;    // timing probe [layer][workgroup][16] real-time stamps of the last launch, or nullptr
};
size_t mlp_stack_ws_bytes();
int mlp_stack_max_m();
int mlp_stack_grid();
hipError_t launch_mlp_stack(const MlpStackArgs& a, int wf, int xdt, hipStream_t stream);

// A chain of dependent projections in one persistent launch (qw_chain.hip),
// decode (M <= chain_max_m() tokens); the op table lives in device memory.
constexpr int kChainMaxK = 3584;     // inputs per op (the largest Qwen3.5-0.8B K)
constexpr int kChainMaxImports = 8;  // slots fed from buffers at launch start
constexpr int kChainMaxOps = 128;    // ops per chain (the op table is held in LDS)
struct ChainOp {
    const uint8_t* w;          // packed weight
    const float* scales;       // INT8 per physical row, or nullptr
    int glu;                   // 1: blocks are gate/up tile pairs (SiLU*mul)
    int n_blk;                 // output blocks (16 rows each)
    int ksteps;                // k-steps of the packed weight
    int K, N;                  // inputs, outputs (N = 16 * n_blk)
    const uint64_t* in_words;  // input slot words [M][in_ld]
    int in_ld, in_off;         // words per token row; first input element (even)
    int in_tag;                // tag of the input's writer: op index + 1, 0 = imported
    const float* gamma;        // RMSNorm weight of the prologue, or nullptr
    int norm;                  // 1: RMSNorm prologue (gamma, or folded into the weight)
    float eps;
    uint64_t* out_words;       // output slot words [M][out_ld]
    int out_ld;
    uint16_t* exp;             // plain copy of the output [M][exp_ld], or nullptr
    int exp_ld;
    int residual;              // 1: add the slot's previous values of the output rows
    int res_tag;               // tag of their writer
    int base;                  // first workgroup of the round robin over the blocks
};
struct ChainImport {
    uint64_t* words_ptr;       // slot words [M][words]
    int words;                 // words per token row
    const void* src;           // [M][ld] 16-bit values
    int ld;
};
struct ChainArgs {
    const ChainOp* ops;
    int n_ops, M;
    ChainImport imports[kChainMaxImports];
    int n_imports;
    unsigned* epoch;           // [3]: launch epoch (advanced by every launch), abort word, wrap barrier counter
    uint64_t* words;           // every slot word of the chain (cleared when the epoch field wraps)
    uint32_t n_words;
    unsigned* err;             // device error flag
    uint64_t* trace;           // timing probe [op][4][256] real-time stamps, or nullptr (QW_CHAIN_TRACE)
};
int chain_grid();
int chain_max_m();
int chain_max_blocks();        // output blocks per op
int chain_max_loads(int wf);   // weight loads per compute wave and op
int chain_compute_waves();
hipError_t launch_chain(const ChainArgs& a, int wf, int xdt, hipStream_t stream);

// Gated-DeltaNet decode step (qw_gdn.hip): one token of each of B sequences.
struct GdnArgs {
    int B, T, nh, kd, vd, K;  // B sequences of T consecutive tokens; row = b*T + t
    const void* mixed;     // [B*T][ld_in] rows: q | k | v channels
    const void* z;         // [B*T][ld_in]: nh*vd
    const void* a;         // [B*T][ld_in]: nh
    const void* b;         // [B*T][ld_in]: nh
    int in_dt, ld_in;
    const float* conv_w;   // [conv_dim][K]
    const float* A_log;    // [nh]
    const float* dt_bias;  // [nh]
    const float* norm_w;   // [vd]
    float* conv_state;     // [B][conv_dim][K-1]
    float* rec_state;      // [B][nh][kd][vd]
    void* out;             // [B*T][ld_out]: nh*vd
    int out_dt, ld_out;
};
hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream);
// chunked form for long token runs: workspace bytes per token of each sequence
size_t gdn_chunked_bytes_per_token(int nh);
// hipErrorInvalidValue when the workspace does not hold one 64-token chunk per sequence
hipError_t launch_gdn_chunked(const GdnArgs& a, void* ws, size_t ws_bytes, hipStream_t stream);

// Gated full attention between the projections (qw_attn.hip): B sequences of
// T new tokens each; row r = b*T + t is at cache position pos[b] + t.
struct AttnArgs {
    int B, T, nh, nkv, hd, rot;
    float theta;
    const float* qn_w;     // [hd] RMSNorm (1 + w) of q
    const float* kn_w;     // [hd] of k
    const void* q;         // row r, head h, dim d at r*ld_in + h*q_hs + d
    const void* gate;      // same indexing as q
    const void* k;         // r*ld_in + g*hd + d
    const void* v;
    int q_hs, in_dt, ld_in;
    int kv_dt;             // DT_F32 or DT_I8 (per-(token, head) scales)
    void* kc;              // [B][cap][nkv][hd]
    void* vc;
    float* ks;             // [B][cap][nkv] (INT8)
    float* vs;
    int cap;
    const int* pos;        // device [B]
    void* out;             // r*ld_out + h*hd + d
    int out_dt, ld_out;
    unsigned* err;         // device error flag (position out of the cache)
    int row0, rows;        // the segment of rows of this launch
    float* qn;             // workspace [rows][nh][hd]: normalized, rotated q
    float* part;           // workspace [rows][nh][nsplit][hd + 2]: split partials
    int split, nsplit;     // keys per split, splits per row (upper bound)
    int prefill;           // query-block kernel: tokens [tb, tb + ntok) of sequences [b0, b0 + nb)
    int b0, nb, tb, ntok;  // (the rows of the segment are then contiguous: row0 = b0*T + tb)
    unsigned* cnt;         // one-launch decode (T == 1, INT8): arrival counters [rows][nkv], zero between launches
    int vcoal;             // INT8 decode: coalesced V row loads (launches that fill the chip)
};
// workspace bytes per row for a given split count
size_t attn_bytes_per_row(int nh, int hd, int nsplit);
hipError_t launch_attn(const AttnArgs& a, hipStream_t stream);

// Token-embedding gather and the decode-step position advance (qw_embed.hip).
hipError_t launch_embed_gather(const void* table, int tdt, int vocab, int K, const int32_t* ids, int M, void* out,
                               int odt, int ld_out, unsigned* err, hipStream_t stream);
hipError_t launch_positions_add(int32_t* pos, int n, int delta, hipStream_t stream);

// Weight packing (qw_pack.hip).  src is a device buffer W[N][K] in src_dt.
// Output rows are written to physical tile `tile_of_row(o)` (GLU interleave
// handled by the caller through tile_mul/tile_add: pt = t*tile_mul+tile_add).
hipError_t launch_fold_norm(uint8_t* w, int wf, int phys_tiles, int ksteps, const float* gamma, hipStream_t stream);
hipError_t launch_pack(const void* src, int src_dt, int wf, const float* src_scales, int N, int K,
                       uint8_t* dst, float* dst_scales, int tile_mul, int tile_add,
                       hipStream_t stream);
hipError_t launch_unpack(const uint8_t* src, int wf, int n_rows, int K, void* dst,
                         int tile_mul, int tile_add, hipStream_t stream);

// RMSNorm family (qw_norm.hip)
hipError_t launch_rmsnorm(const void* x, int xdt, const void* add, void* sum_out,
                          const float* gamma, float eps, void* y, int ydt, int M, int K,
                          hipStream_t stream);
hipError_t launch_rmsnorm_ld(const void* x, int xdt, int ldx, const float* gamma, float eps, void* y, int ydt,
                             int ldy, int M, int K, hipStream_t stream);
hipError_t launch_argmax_rows(const void* logits, int dt, int M, int V, int64_t ld, unsigned long long* keys,
                              unsigned* done, int32_t* ids, float* maxv, hipStream_t stream);
hipError_t launch_silu_mul(const void* g, const void* u, void* h, int dt, int64_t n,
                           hipStream_t stream);

}  // namespace qwk
