// qw_api.cpp -- C ABI of the projection library (declared in include/qw_linear.h).
//
// Host side only: argument validation, workspace carving, kernel choice and
// launch.  Nothing here synchronizes the stream or allocates on the hot path;
// device memory is reserved by qw_init (workspace) and qw_weight_pack
// (weights) only.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qw_linear.h"
#include "qw_internal.hpp"
#include "qw_kernels.hpp"

hipError_t qwk::ensure_max_lds(const void* kernel, int bytes) {
    // a fixed table (no heap allocation, so the no-allocation entry point may
    // take this path); when it is full the attribute is simply set again
    struct Entry {
        int dev;
        const void* kernel;
        int bytes;
    };
    static std::mutex mu;
    static Entry table[1024];
    static int used = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(mu);
    Entry* hit = nullptr;
    for (int i = 0; i < used; ++i)
        if (table[i].dev == dev && table[i].kernel == kernel) hit = &table[i];
    if (hit && hit->bytes >= bytes) return hipSuccess;
    e = set_max_lds(kernel, bytes);
    if (e != hipSuccess) return e;
    if (hit) hit->bytes = bytes;
    else if (used < 1024) table[used++] = Entry{dev, kernel, bytes};
    return hipSuccess;
}

constexpr int kGemmMinM = 33;
constexpr int kWideMinM = 17;  // default token count from which the weight-stationary kernel is used  // default token count from which the MFMA GEMM is used
constexpr int kGdnChunkMin = 24;  // tokens per sequence from which the chunked Gated-DeltaNet form runs (measured crossover 20-26)

struct qw_ctx {
    int device = 0;
    int num_cus = 256;
    int wg_per_cu = 2;       // resident skinny workgroups per CU (grid cap)
    int min_items = 0;       // split K until a launch has this many items (0: never)
    int force_nw = 0;        // waves per skinny workgroup (0: automatic)
    int force_nw_glu = 0;    // same, GLU weights only
    int mlp_fused = -1;      // one-launch MLP block at decode sizes: -1 auto (BF16 weights, where it
                             // measured faster), 1 also INT8 (QW_MLP_FUSED=1), 0 never (QW_MLP_FUSED=0)
    bool gemv = true;        // register-direct GEMV for M <= 32 (QW_GEMV=0: skinny kernel)
    int gemm_min_m = kGemmMinM;  // tokens from which BF16 calls may use the MFMA GEMM
    bool gemm_forced = false;    // QW_GEMM_MIN_M given: GEMM from gemm_min_m tokens on, always
    int gemm_tile_m = 0;         // tokens per GEMM block (QW_GEMM_TILE_M: 128 or 256; 0 = by shape)
    int gemm_waves = 8;          // waves per 256-token GEMM block (QW_GEMM_WAVES: 4 or 8)
    int gemm_da = 1;             // direct-A GEMM for BF16 x BF16 256-row blocks (QW_GEMM_DA: 0 off,
                                 // 1 where its blocks fill the chip, 2 wherever it applies)
    bool gemm_da_line = true;    // its activation loads as whole row lines (QW_GEMM_DA_LINE=0: row pieces)
    int gemm_da_group = 0;       // its token blocks per raster group (QW_GEMM_DA_GROUP; 0: 8)
    int gemm_da_persist = 1;     // its 8-wave form as one persistent workgroup per CU (QW_GEMM_DA_PERSIST=0: off)
    int gemm_da_waves = 0;       // its waves per block: 4 (256 rows, two blocks per CU) or 8 (512 rows, one);
                                 // 0: 8 where the 512-row blocks cover every CU (QW_GEMM_DA_W8=0/1 forces 4/8)
    int gemm_rows = 0;           // weight rows per GEMM block (QW_GEMM_ROWS: 64 or 256; 0 = by shape)
    int gemm_splitk = 0;         // K splits per GEMM tile (QW_GEMM_SPLITK; 0 = by shape)
    int gdn_chunk_min = kGdnChunkMin;
    bool wide = true;            // weight-stationary kernel for wide_min..wide_max tokens (QW_WIDE=0: off)
    int wide_min = kWideMinM;    // QW_WIDE_MIN
    int wide_max = qwk::kWideMaxM;  // QW_WIDE_MAX
    int wide_s = 0;              // K splits (QW_WIDE_S; 0 = planned)
    bool wide_norm_sep = false;  // RMSNorm prologue as a separate launch (QW_WIDE_NORM_SEP=1) instead of in the kernel
    int wide_dbg = 0;            // QW_WIDE_DBG: timing probes (wrong results)
    int stack_dbg = 0;           // QW_MLP_STACK_DBG: timing probes of the MLP stack (wrong results)
    uint64_t* stack_trace = nullptr;       // QW_MLP_STACK_TRACE=<file>: per-block timestamps of the last stack launch
    std::string stack_trace_path;
    int stack_gap = -1;          // QW_MLP_STACK_GAP: 10 ns ticks between a gate/up group's weight k-steps
                                 // (-1: 20 for BF16 weights, 120 for INT8, the measured best of each)
    int wide_cfg = 0;            // blocks x waves per block (QW_WIDE_CFG 1: 4x1, 2: 2x2, 3: 1x4; 0 = planned)
    int attn_split = 0;          // keys per decode split, 0 = by size (QW_ATTN_SPLIT forces a multiple of 64)
    int attn_vcoal = -1;         // INT8 decode V loads: -1 by launch size, 0 scattered, 1 coalesced (QW_ATTN_VCOAL)
    bool attn_fused = true;      // one-launch INT8 decode attention (QW_ATTN_FUSED=0: prep / split / combine)
    int attn_prefill_min = 16;   // tokens per sequence from which the query-block attention kernel runs (QW_ATTN_PREFILL_MIN)  // tokens per sequence from which the chunked GDN form runs (QW_GDN_CHUNK_MIN)
    uint8_t* ws = nullptr;
    size_t ws_bytes = 0;
    // carved regions
    unsigned* counters = nullptr;          // split-K arrival counters
    unsigned long long* keys = nullptr;    // argmax keys
    unsigned* done = nullptr;              // argmax completion counter
    unsigned* mlp_ctl = nullptr;           // fused MLP: ticket, up done, exited, error flag
    unsigned* stack_epoch = nullptr;       // persistent MLP stack: launch epoch, abort word
    uint64_t* stack_words = nullptr;       // persistent MLP stack: hand-off words
    bool mlp_stack = true;                 // QW_MLP_STACK=0: per-layer launches in qw_mlp_stack
    int argmax_cache = -1;                 // QW_ARGMAX_CACHE: weight-load cache policy of that kernel (-1 auto, 0 NT, 1 default)
    int argmax_wide_min_i8 = 8;            // QW_ARGMAX_WIDE_MIN_I8: INT8 lm_head tokens from which the weight-stationary argmax runs
    bool argmax_as = true;                 // QW_ARGMAX_AS=0: no activation-stationary lm_head argmax
    int argmax_as_min = 65;                // QW_ARGMAX_AS_MIN: tokens from which it runs (to 128)
    int argmax_nw = 0;                     // QW_ARGMAX_NW: waves per weight-stationary argmax workgroup (0 auto, 4, 8)
    int gemm_da_split = -1;                // QW_GEMM_DA_SPLIT: split-K direct-A for few blocks (-1 auto, 0 off, S)
    bool layer_tail = false;               // QW_LAYER_TAIL=1: qw_layer_tail in one launch (measured slower)
    float4* partials = nullptr;
    size_t partials_bytes = 0;
    float4* wide_partials = nullptr;        // the weight-stationary kernel's, every word kWideSentinel
    uint8_t* scratch = nullptr;            // MLP intermediate h
    size_t scratch_bytes = 0;
    uint8_t* xnorm = nullptr;              // RMSNorm-ed activations for the GEMM path
    size_t xnorm_bytes = 0;
    // optional weight arena: packed weights are carved from one large
    // allocation (2 MiB aligned) instead of one hipMalloc each
    uint8_t* arena = nullptr;
    size_t arena_bytes = 0;
    size_t arena_used = 0;
    std::string err;
};

struct qw_weight {
    qw_ctx* ctx = nullptr;
    uint8_t* packed = nullptr;
    float* scales = nullptr;
    int N = 0;        // logical output rows
    int K = 0;
    int wf = 0;       // qw_wfmt
    int glu = 0;
    int phys_tiles = 0;
    int ksteps = 0;
    size_t bytes = 0;
    bool owns = true;
    bool in_arena = false;
    bool norm_folded = false;  // (1 + gamma) of an RMSNorm multiplied into the columns
};

struct qw_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

constexpr size_t kCountersBytes = 64 * 1024;     // 16384 tiles
constexpr size_t kKeysBytes = 64 * 1024;         // 8192 tokens
constexpr size_t kDoneBytes = 256;
constexpr size_t kPartialsBytes = 64u << 20;
// the weight-stationary kernel's split-K partials, kept at kWideSentinel (the
// most it can use: one workgroup per CU x 32 units x 64 lanes x 36 bytes)
constexpr size_t kWidePartialsBytes = 20u << 20;
constexpr size_t kStackBytes = 512 * 1024;  // hand-off words of the persistent MLP stack (zeroed at init)
constexpr size_t kFixedBytes =
    kCountersBytes + kKeysBytes + kDoneBytes + kStackBytes + kPartialsBytes + kWidePartialsBytes;
constexpr int kMlpCounterWords = 4096;  // tail of the counter region: the one-launch MLP's slots
constexpr int kMaxCounters = (int)(kCountersBytes / 4) - kMlpCounterWords;
constexpr int kMaxKeys = (int)(kKeysBytes / 8);
constexpr int kSkinnyMaxM = 32;

qw_status fail(qw_ctx* c, qw_status s, const char* fmt, ...) {
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return s;
}

qw_status hip_fail(qw_ctx* c, hipError_t e, const char* what) {
    return fail(c, QW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int ke_of(int wf) { return wf == QW_WFMT_F32 ? 4 : (wf == QW_WFMT_BF16 ? 8 : 16); }
int esize_of(int wf) { return wf == QW_WFMT_F32 ? 4 : (wf == QW_WFMT_BF16 ? 2 : 1); }
int dsize(qw_dtype d) { return d == QW_F32 ? 4 : (d == QW_I8 ? 1 : 2); }
bool valid_act(qw_dtype d) { return d == QW_F32 || d == QW_BF16 || d == QW_F16; }
bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

size_t scratch_need(int M, int I) { return (size_t)M * I * 4; }
size_t xnorm_need(int M, int K) { return (size_t)M * K * 2; }

}  // namespace

extern "C" {

int qw_abi_version(void) { return QW_ABI_VERSION; }

const char* qw_status_string(qw_status s) {
    switch (s) {
        case QW_OK: return "ok";
        case QW_ERR_INVALID: return "invalid argument";
        case QW_ERR_NULL: return "null pointer";
        case QW_ERR_SHAPE: return "unsupported shape";
        case QW_ERR_DTYPE: return "unsupported dtype";
        case QW_ERR_ALIGN: return "misaligned pointer or leading dimension";
        case QW_ERR_WORKSPACE: return "workspace too small";
        case QW_ERR_HIP: return "HIP runtime error";
        case QW_ERR_NOMEM: return "out of device memory";
        case QW_ERR_STATE: return "invalid state";
    }
    return "unknown status";
}

const char* qw_last_error(const qw_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

size_t qw_workspace_query(int max_M, int max_N, int max_K) {
    (void)max_K;
    if (max_M < 1) max_M = 1;
    if (max_N < 1) max_N = 1;
    if (max_K < 1) max_K = 1;
    size_t s = kFixedBytes + scratch_need(max_M, max_N) + xnorm_need(max_M, max_K) + 4096;
    return (s + 4095) & ~(size_t)4095;
}

qw_status qw_init(qw_ctx** out, int device, size_t workspace_bytes) {
    if (!out) return QW_ERR_NULL;
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return QW_ERR_HIP;
    if (device < 0 || device >= ndev) return QW_ERR_INVALID;
    if (hipSetDevice(device) != hipSuccess) return QW_ERR_HIP;
    qw_ctx* c = new qw_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        c->num_cus = prop.multiProcessorCount;
    if (const char* v = getenv("QW_WEIGHT_ARENA_MB")) {
        const size_t mb = (size_t)std::max(0, atoi(v));
        if (mb && hipMalloc(&c->arena, mb << 20) == hipSuccess) c->arena_bytes = mb << 20;
    }
    if (const char* v = getenv("QW_SKINNY_WG_PER_CU")) c->wg_per_cu = std::max(1, atoi(v));
    if (const char* v = getenv("QW_SKINNY_MIN_ITEMS")) c->min_items = std::max(0, atoi(v));
    auto nw_of = [](const char* v) { const int n = atoi(v); return (n == 4 || n == 8 || n == 16) ? n : 0; };
    if (const char* v = getenv("QW_SKINNY_NW")) c->force_nw = nw_of(v);
    if (const char* v = getenv("QW_SKINNY_NW_GLU")) c->force_nw_glu = nw_of(v);
    if (const char* v = getenv("QW_MLP_FUSED")) c->mlp_fused = atoi(v) != 0 ? 1 : 0;
    if (const char* v = getenv("QW_GEMV")) c->gemv = atoi(v) != 0;
    if (const char* v = getenv("QW_MLP_STACK")) c->mlp_stack = atoi(v) != 0;
    if (const char* v = getenv("QW_LAYER_TAIL")) c->layer_tail = atoi(v) != 0;
    if (const char* v = getenv("QW_GEMM_DA_SPLIT")) c->gemm_da_split = atoi(v);
    if (const char* v = getenv("QW_ARGMAX_CACHE")) c->argmax_cache = atoi(v) ? 1 : 0;
    if (const char* v = getenv("QW_ARGMAX_WIDE_MIN_I8")) c->argmax_wide_min_i8 = std::max(1, atoi(v));
    if (const char* v = getenv("QW_ARGMAX_AS")) c->argmax_as = atoi(v) != 0;
    if (const char* v = getenv("QW_ARGMAX_AS_MIN")) c->argmax_as_min = std::max(1, atoi(v));
    if (const char* v = getenv("QW_ARGMAX_NW")) c->argmax_nw = (atoi(v) == 4 || atoi(v) == 8) ? atoi(v) : 0;
    if (const char* v = getenv("QW_GEMM_TILE_M")) c->gemm_tile_m = atoi(v) == 256 ? 256 : 128;  // forced
    if (const char* v = getenv("QW_GEMM_WAVES")) c->gemm_waves = atoi(v) == 4 ? 4 : 8;
    if (const char* v = getenv("QW_GEMM_DA")) c->gemm_da = std::max(0, std::min(2, atoi(v)));
    if (const char* v = getenv("QW_GEMM_DA_LINE")) c->gemm_da_line = atoi(v) != 0;
    if (const char* v = getenv("QW_GEMM_DA_GROUP")) c->gemm_da_group = std::max(0, atoi(v));
    if (const char* v = getenv("QW_GEMM_DA_W8")) c->gemm_da_waves = atoi(v) != 0 ? 8 : 4;
    if (const char* v = getenv("QW_GEMM_DA_PERSIST")) c->gemm_da_persist = atoi(v) != 0;
    if (const char* v = getenv("QW_GEMM_SPLITK")) c->gemm_splitk = std::max(0, std::min(8, atoi(v)));
    if (const char* v = getenv("QW_GEMM_ROWS")) c->gemm_rows = atoi(v) == 64 ? 64 : 256;
    if (const char* v = getenv("QW_ATTN_FUSED")) c->attn_fused = atoi(v) != 0;
    if (const char* v = getenv("QW_ATTN_SPLIT")) c->attn_split = std::max(0, atoi(v)) / 64 * 64;
    if (const char* v = getenv("QW_ATTN_VCOAL")) c->attn_vcoal = atoi(v) != 0 ? 1 : 0;
    if (const char* v = getenv("QW_ATTN_PREFILL_MIN")) c->attn_prefill_min = std::max(1, atoi(v));
    if (const char* v = getenv("QW_GDN_CHUNK_MIN")) c->gdn_chunk_min = std::max(1, atoi(v));
    if (const char* v = getenv("QW_WIDE")) c->wide = atoi(v) != 0;
    if (const char* v = getenv("QW_WIDE_MIN")) c->wide_min = std::max(1, atoi(v));
    if (const char* v = getenv("QW_WIDE_MAX")) c->wide_max = std::min(qwk::kWideMaxM, atoi(v));
    if (const char* v = getenv("QW_WIDE_S")) c->wide_s = std::max(0, atoi(v));
    if (const char* v = getenv("QW_WIDE_NORM_SEP")) c->wide_norm_sep = atoi(v) != 0;
    if (const char* v = getenv("QW_WIDE_DBG")) c->wide_dbg = atoi(v);
    if (const char* v = getenv("QW_MLP_STACK_DBG")) c->stack_dbg = atoi(v);
    if (const char* v = getenv("QW_MLP_STACK_TRACE")) {
        // timing probe: [layer][workgroup][16] s_memrealtime stamps of the last
        // launch (x seen and h stored by gate/up, h seen and x stored by down;
        // 4..11: x seen by gate/up wave w, h seen by down poller w; 12: the
        // last arriver starts its epilogue),
        // written to the file at qw_destroy
        if (hipMalloc(&c->stack_trace, (size_t)qwk::kMlpStackMaxLayers * 256 * 16 * 8) == hipSuccess) {
            hipMemset(c->stack_trace, 0, (size_t)qwk::kMlpStackMaxLayers * 256 * 16 * 8);
            c->stack_trace_path = v;
        }
    }
    if (const char* v = getenv("QW_MLP_STACK_GAP")) c->stack_gap = std::max(0, std::min(1000, atoi(v)));
    if (const char* v = getenv("QW_WIDE_CFG")) c->wide_cfg = std::max(0, std::min(3, atoi(v)));
    if (const char* v = getenv("QW_WIDE_T")) c->wide_cfg |= std::max(0, std::min(8, atoi(v))) << 4;  // token groups
    if (const char* v = getenv("QW_GEMM_MIN_M")) {
        c->gemm_min_m = std::max(1, atoi(v));
        c->gemm_forced = true;
    }
    if (workspace_bytes == 0) workspace_bytes = qw_workspace_query(4096, 8224, 4096);
    workspace_bytes = std::max(workspace_bytes, kFixedBytes + (size_t)(3u << 20));
    workspace_bytes = (workspace_bytes + 4095) & ~(size_t)4095;
    if (hipMalloc(&c->ws, workspace_bytes) != hipSuccess) {
        delete c;
        return QW_ERR_NOMEM;
    }
    c->ws_bytes = workspace_bytes;
    uint8_t* p = c->ws;
    c->counters = reinterpret_cast<unsigned*>(p); p += kCountersBytes;
    c->keys = reinterpret_cast<unsigned long long*>(p); p += kKeysBytes;
    c->done = reinterpret_cast<unsigned*>(p);
    c->mlp_ctl = c->done + 16;
    c->stack_epoch = c->done + 32;
    p += kDoneBytes;
    c->stack_words = reinterpret_cast<uint64_t*>(p); p += kStackBytes;
    c->partials = reinterpret_cast<float4*>(p); p += kPartialsBytes;
    c->partials_bytes = kPartialsBytes;
    c->wide_partials = reinterpret_cast<float4*>(p); p += kWidePartialsBytes;
    {
        // the rest: normalized activations (about a third) and the MLP intermediate
        const size_t rest = workspace_bytes - kFixedBytes;
        c->xnorm_bytes = (rest / 3) & ~(size_t)4095;
        c->xnorm = p;
        p += c->xnorm_bytes;
        c->scratch = p;
        c->scratch_bytes = rest - c->xnorm_bytes;
    }
    // counters, keys and the completion counter start at zero; every kernel
    // that uses them returns them to zero before it exits.
    // The weight-stationary kernel's partials start empty (every word the
    // sentinel); its finishing workgroups empty what they consumed.
    if (hipMemset(c->ws, 0, kCountersBytes + kKeysBytes + kDoneBytes + kStackBytes) != hipSuccess ||
        hipMemset(c->wide_partials, 0xff, kWidePartialsBytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        hipFree(c->ws);
        delete c;
        return QW_ERR_HIP;
    }
    *out = c;
    return QW_OK;
}

qw_status qw_destroy(qw_ctx* ctx) {
    if (!ctx) return QW_ERR_NULL;
    hipSetDevice(ctx->device);
    if (ctx->stack_trace) {
        std::vector<uint64_t> h((size_t)qwk::kMlpStackMaxLayers * 256 * 16);
        hipDeviceSynchronize();
        if (hipMemcpy(h.data(), ctx->stack_trace, h.size() * 8, hipMemcpyDeviceToHost) == hipSuccess) {
            if (FILE* f = fopen(ctx->stack_trace_path.c_str(), "wb")) {
                fwrite(h.data(), 8, h.size(), f);
                fclose(f);
            }
        }
        hipFree(ctx->stack_trace);
    }
    if (ctx->ws) hipFree(ctx->ws);
    if (ctx->arena) hipFree(ctx->arena);
    delete ctx;
    return QW_OK;
}

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------

static qw_status alloc_weight(qw_ctx* ctx, qw_wfmt dst, int N, int K, int glu, qw_weight** out) {
    qw_weight* w = new qw_weight();
    w->ctx = ctx;
    w->N = N;
    w->K = K;
    w->wf = dst;
    w->glu = glu;
    const int tiles = (N + 15) / 16;
    w->phys_tiles = tiles * (glu ? 2 : 1);
    w->ksteps = K / (4 * ke_of(dst));
    w->bytes = (size_t)w->phys_tiles * w->ksteps * 1024;
    const size_t need = (w->bytes + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
    if (ctx->arena && ctx->arena_used + need <= ctx->arena_bytes) {
        w->packed = ctx->arena + ctx->arena_used;
        ctx->arena_used += need;
        w->in_arena = true;
    } else if (hipMalloc(&w->packed, w->bytes) != hipSuccess) {
        delete w;
        return fail(ctx, QW_ERR_NOMEM, "hipMalloc of %zu bytes for packed weight failed", w->bytes);
    }
    if (hipMemset(w->packed, 0, w->bytes) != hipSuccess) {
        hipFree(w->packed);
        delete w;
        return fail(ctx, QW_ERR_HIP, "hipMemset of packed weight failed");
    }
    if (dst == QW_WFMT_INT8_ROWSCALE) {
        const size_t sb = (size_t)w->phys_tiles * 16 * sizeof(float);
        if (hipMalloc(&w->scales, sb) != hipSuccess) {
            hipFree(w->packed);
            delete w;
            return fail(ctx, QW_ERR_NOMEM, "hipMalloc of scales failed");
        }
        hipMemset(w->scales, 0, sb);
    }
    *out = w;
    return QW_OK;
}

static qw_status check_pack_args(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N, int K,
                                 const float* scales) {
    if (!ctx) return QW_ERR_NULL;
    if (!w) return fail(ctx, QW_ERR_NULL, "weight pointer is NULL");
    if (N < 1 || K < 64 || K % 64 != 0)
        return fail(ctx, QW_ERR_SHAPE, "weight shape N=%d K=%d: need N>=1 and K a positive multiple of 64", N, K);
    if ((size_t)N * K > (size_t)1 << 34) return fail(ctx, QW_ERR_SHAPE, "weight too large");
    if (dst != QW_WFMT_F32 && dst != QW_WFMT_BF16 && dst != QW_WFMT_INT8_ROWSCALE)
        return fail(ctx, QW_ERR_DTYPE, "unknown weight format %d", (int)dst);
    if (src == QW_I8) {
        if (dst != QW_WFMT_INT8_ROWSCALE)
            return fail(ctx, QW_ERR_DTYPE, "INT8 source requires the INT8_ROWSCALE format");
        if (!scales) return fail(ctx, QW_ERR_NULL, "INT8 source requires per-row scales");
    } else if (!valid_act(src)) {
        return fail(ctx, QW_ERR_DTYPE, "unknown source dtype %d", (int)src);
    }
    return QW_OK;
}

// Pack one matrix of `rows` rows (host or device source) into physical tiles
// tile_off + t*tile_mul + tile_add (rows 0 = all of W).
static qw_status pack_one(qw_ctx* ctx, qw_weight* W, const void* src_ptr, qw_dtype src,
                          const float* src_scales, int tile_mul, int tile_add, bool on_device,
                          int rows = 0, int tile_off = 0) {
    if (rows == 0) rows = W->N;
    const size_t bytes = (size_t)rows * W->K * dsize(src);
    const void* dsrc = src_ptr;
    const float* dscales = src_scales;
    void* stage = nullptr;
    float* stage_s = nullptr;
    hipError_t e = hipSuccess;
    if (!on_device) {
        e = hipMalloc(&stage, bytes);
        if (e != hipSuccess) return fail(ctx, QW_ERR_NOMEM, "staging hipMalloc failed");
        e = hipMemcpy(stage, src_ptr, bytes, hipMemcpyHostToDevice);
        dsrc = stage;
        if (e == hipSuccess && src == QW_I8) {
            e = hipMalloc(&stage_s, (size_t)rows * sizeof(float));
            if (e == hipSuccess)
                e = hipMemcpy(stage_s, src_scales, (size_t)rows * sizeof(float), hipMemcpyHostToDevice);
            dscales = stage_s;
        }
    }
    if (e == hipSuccess)
        e = qwk::launch_pack(dsrc, (int)src, W->wf, dscales, rows, W->K,
                             W->packed + (size_t)tile_off * W->ksteps * 1024,
                             W->scales ? W->scales + (size_t)tile_off * 16 : nullptr, tile_mul, tile_add, 0);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (stage) hipFree(stage);
    if (stage_s) hipFree(stage_s);
    if (e != hipSuccess) return hip_fail(ctx, e, "weight packing");
    return QW_OK;
}

static qw_status pack_impl(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N, int K,
                           const float* scales, qw_weight** out, bool on_device) {
    if (!out) return fail(ctx, QW_ERR_NULL, "out is NULL");
    *out = nullptr;
    qw_status s = check_pack_args(ctx, w, src, dst, N, K, scales);
    if (s != QW_OK) return s;
    hipSetDevice(ctx->device);
    qw_weight* W = nullptr;
    if ((s = alloc_weight(ctx, dst, N, K, 0, &W)) != QW_OK) return s;
    if ((s = pack_one(ctx, W, w, src, scales, 1, 0, on_device)) != QW_OK) {
        qw_weight_free(W);
        return s;
    }
    *out = W;
    return QW_OK;
}

static qw_status pack_glu_impl(qw_ctx* ctx, const void* gate, const void* up, qw_dtype src,
                               qw_wfmt dst, int N, int K, const float* gate_scales,
                               const float* up_scales, qw_weight** out, bool on_device) {
    if (!out) return fail(ctx, QW_ERR_NULL, "out is NULL");
    *out = nullptr;
    qw_status s = check_pack_args(ctx, gate, src, dst, N, K, gate_scales);
    if (s != QW_OK) return s;
    if ((s = check_pack_args(ctx, up, src, dst, N, K, up_scales)) != QW_OK) return s;
    hipSetDevice(ctx->device);
    qw_weight* W = nullptr;
    if ((s = alloc_weight(ctx, dst, N, K, 1, &W)) != QW_OK) return s;
    if ((s = pack_one(ctx, W, gate, src, gate_scales, 2, 0, on_device)) != QW_OK ||
        (s = pack_one(ctx, W, up, src, up_scales, 2, 1, on_device)) != QW_OK) {
        qw_weight_free(W);
        return s;
    }
    *out = W;
    return QW_OK;
}

static qw_status pack_concat_impl(qw_ctx* ctx, int parts, const void* const* ws, const int* Ns, qw_dtype src,
                                  qw_wfmt dst, int K, const float* const* scales, qw_weight** out, bool on_device) {
    if (!ctx) return QW_ERR_NULL;
    if (!out) return fail(ctx, QW_ERR_NULL, "out is NULL");
    *out = nullptr;
    if (parts < 1 || !ws || !Ns) return fail(ctx, QW_ERR_NULL, "parts, ws and Ns are required");
    int64_t N = 0;
    for (int i = 0; i < parts; ++i) {
        qw_status s = check_pack_args(ctx, ws[i], src, dst, Ns[i], K, scales ? scales[i] : nullptr);
        if (s != QW_OK) return s;
        if (i + 1 < parts && Ns[i] % 16 != 0)
            return fail(ctx, QW_ERR_SHAPE, "part %d has %d rows: all parts but the last need a multiple of 16", i, Ns[i]);
        N += Ns[i];
    }
    if (N > (1 << 30)) return fail(ctx, QW_ERR_SHAPE, "too many rows");
    hipSetDevice(ctx->device);
    qw_weight* W = nullptr;
    qw_status s = alloc_weight(ctx, dst, (int)N, K, 0, &W);
    if (s != QW_OK) return s;
    int tile = 0;
    for (int i = 0; i < parts; ++i) {
        if ((s = pack_one(ctx, W, ws[i], src, scales ? scales[i] : nullptr, 1, 0, on_device, Ns[i], tile)) != QW_OK) {
            qw_weight_free(W);
            return s;
        }
        tile += (Ns[i] + 15) / 16;
    }
    *out = W;
    return QW_OK;
}

qw_status qw_weight_pack_concat(qw_ctx* ctx, int parts, const void* const* ws, const int* Ns, qw_dtype src,
                                qw_wfmt dst, int K, const float* const* scales, qw_weight** out) {
    return pack_concat_impl(ctx, parts, ws, Ns, src, dst, K, scales, out, false);
}

qw_status qw_weight_pack_concat_device(qw_ctx* ctx, int parts, const void* const* ws, const int* Ns, qw_dtype src,
                                       qw_wfmt dst, int K, const float* const* scales, qw_weight** out) {
    return pack_concat_impl(ctx, parts, ws, Ns, src, dst, K, scales, out, true);
}

qw_status qw_weight_pack(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N, int K,
                         const float* scales, qw_weight** out) {
    return pack_impl(ctx, w, src, dst, N, K, scales, out, false);
}

qw_status qw_weight_pack_device(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N, int K,
                                const float* scales, qw_weight** out) {
    return pack_impl(ctx, w, src, dst, N, K, scales, out, true);
}

qw_status qw_weight_pack_glu(qw_ctx* ctx, const void* gate, const void* up, qw_dtype src,
                             qw_wfmt dst, int N, int K, const float* gate_scales,
                             const float* up_scales, qw_weight** out) {
    return pack_glu_impl(ctx, gate, up, src, dst, N, K, gate_scales, up_scales, out, false);
}

qw_status qw_weight_pack_glu_device(qw_ctx* ctx, const void* gate, const void* up, qw_dtype src,
                                    qw_wfmt dst, int N, int K, const float* gate_scales,
                                    const float* up_scales, qw_weight** out) {
    return pack_glu_impl(ctx, gate, up, src, dst, N, K, gate_scales, up_scales, out, true);
}

qw_status qw_weight_wrap_packed(qw_ctx* ctx, void* packed, float* scales, qw_wfmt fmt, int N, int K,
                                qw_weight** out) {
    if (!ctx || !out) return QW_ERR_NULL;
    *out = nullptr;
    if (!packed) return fail(ctx, QW_ERR_NULL, "packed pointer is NULL");
    if (N < 1 || K < 64 || K % 64 != 0) return fail(ctx, QW_ERR_SHAPE, "bad shape N=%d K=%d", N, K);
    if (fmt == QW_WFMT_INT8_ROWSCALE && !scales) return fail(ctx, QW_ERR_NULL, "INT8 weight needs scales");
    if (!aligned(packed, 16) || (scales && !aligned(scales, 16)))
        return fail(ctx, QW_ERR_ALIGN, "packed data and scales must be 16-byte aligned");
    qw_weight* W = new qw_weight();
    W->ctx = ctx;
    W->N = N;
    W->K = K;
    W->wf = fmt;
    W->glu = 0;
    W->phys_tiles = (N + 15) / 16;
    W->ksteps = K / (4 * ke_of(fmt));
    W->bytes = (size_t)W->phys_tiles * W->ksteps * 1024;
    W->packed = static_cast<uint8_t*>(packed);
    W->scales = fmt == QW_WFMT_INT8_ROWSCALE ? scales : nullptr;
    W->owns = false;
    *out = W;
    return QW_OK;
}

qw_status qw_weight_free(qw_weight* w) {
    if (!w) return QW_ERR_NULL;
    if (w->owns) {
        if (w->packed && !w->in_arena) hipFree(w->packed);
        if (w->scales) hipFree(w->scales);
    }
    delete w;
    return QW_OK;
}

qw_status qw_weight_info(const qw_weight* w, int* N, int* K, qw_wfmt* fmt, int* is_glu,
                         size_t* packed_bytes) {
    if (!w) return QW_ERR_NULL;
    if (N) *N = w->N;
    if (K) *K = w->K;
    if (fmt) *fmt = (qw_wfmt)w->wf;
    if (is_glu) *is_glu = w->glu;
    if (packed_bytes) *packed_bytes = w->bytes;
    return QW_OK;
}

qw_status qw_weight_device_ptrs(const qw_weight* w, const void** packed, const float** scales) {
    if (!w) return QW_ERR_NULL;
    if (packed) *packed = w->packed;
    if (scales) *scales = w->scales;
    return QW_OK;
}

qw_status qw_weight_fold_norm(qw_ctx* ctx, qw_weight* w, const float* gamma, hipStream_t stream) {
    if (!ctx || !w) return QW_ERR_NULL;
    if (!gamma) return fail(ctx, QW_ERR_NULL, "gamma is NULL");
    if (w->wf == QW_WFMT_INT8_ROWSCALE)
        return fail(ctx, QW_ERR_DTYPE, "folding into INT8 weights would change their quantization");
    if (w->norm_folded) return fail(ctx, QW_ERR_STATE, "the weight already carries a norm weight");
    hipError_t e = qwk::launch_fold_norm(w->packed, w->wf, w->phys_tiles, w->ksteps, gamma, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "fold launch");
    w->norm_folded = true;
    return QW_OK;
}

qw_status qw_weight_unpack(qw_ctx* ctx, const qw_weight* w, void* dst, float* scales_dst) {
    if (!ctx || !w) return QW_ERR_NULL;
    if (!dst) return fail(ctx, QW_ERR_NULL, "dst is NULL");
    if (w->wf == QW_WFMT_INT8_ROWSCALE && !scales_dst) return fail(ctx, QW_ERR_NULL, "scales_dst is NULL");
    hipSetDevice(ctx->device);
    const int parts = w->glu ? 2 : 1;
    const size_t part_elems = (size_t)w->N * w->K;
    const int es = esize_of(w->wf);
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, part_elems * es);
    if (e != hipSuccess) return fail(ctx, QW_ERR_NOMEM, "staging hipMalloc failed");
    for (int p = 0; p < parts && e == hipSuccess; ++p) {
        e = qwk::launch_unpack(w->packed, w->wf, w->N, w->K, d, parts, p, 0);
        if (e == hipSuccess)
            e = hipMemcpy(static_cast<uint8_t*>(dst) + p * part_elems * es, d, part_elems * es,
                          hipMemcpyDeviceToHost);
        if (e == hipSuccess && w->wf == QW_WFMT_INT8_ROWSCALE) {
            // scales of logical tile t live at physical tile t*parts+p
            const int tiles = (w->N + 15) / 16;
            for (int t = 0; t < tiles && e == hipSuccess; ++t) {
                const int rows = std::min(16, w->N - t * 16);
                e = hipMemcpy(scales_dst + (size_t)p * w->N + t * 16,
                              w->scales + (size_t)(t * parts + p) * 16, rows * sizeof(float),
                              hipMemcpyDeviceToHost);
            }
        }
    }
    hipFree(d);
    if (e != hipSuccess) return hip_fail(ctx, e, "weight unpack");
    return QW_OK;
}

// ---------------------------------------------------------------------------
// projections
// ---------------------------------------------------------------------------

static qw_status check_xdt(qw_ctx* ctx, const qw_weight* W, qw_dtype xdt) {
    if (!valid_act(xdt)) return fail(ctx, QW_ERR_DTYPE, "activation dtype %d unsupported", (int)xdt);
    (void)W;
    return QW_OK;
}

// Skinny launch for M <= 32 tokens (argmax: ids/maxv set, y ignored).
// tg_size > 0 and M > tg_size: one launch over token groups of tg_size.
static qw_status run_skinny(qw_ctx* ctx, const qw_weight* W, const void* x, qw_dtype xdt, int ldx,
                            int M_total, void* y, qw_dtype ydt, int ldy, const qw_epilogue* ep,
                            int32_t* ids, float* maxv, hipStream_t stream, int tg_size = 0) {
    const bool argmax = ids != nullptr;
    const int groups = (tg_size > 0 && M_total > tg_size) ? (M_total + tg_size - 1) / tg_size : 1;
    const int M = groups > 1 ? tg_size : M_total;  // tokens one workgroup sees
    qwk::SkinnyArgs a{};
    a.w = W->packed;
    a.scales = W->scales;
    a.x = x;
    a.ldx = ldx;
    a.M = M_total;
    a.K = W->K;
    a.N = W->N;
    a.n_groups = (W->N + 15) / 16;
    a.ksteps = W->ksteps;
    const int CT = M <= 16 ? 1 : 2, RT = W->glu ? 2 : 1;
    // Workgroup shape: tiles plentiful -> 4 waves per tile; few tiles (the
    // 1024-row projections) -> 16 waves per tile so fewer CUs still keep
    // enough loads in flight.  K is split across workgroups only on request
    // (the split-K hand-off adds a device-coherent round trip).
    const bool wide_ok = !argmax && M <= 16;
    int nw = (wide_ok && !W->glu && a.n_groups * 4 < ctx->num_cus * 3) ? 16 : 4;
    // FP32 weights (64 KB tiles): 8 waves per tile keep more of each tile in
    // flight (config-1 GEMV 6.07 -> 5.65 us; 16 waves 6.82)
    if (wide_ok && !W->glu && W->wf == QW_WFMT_F32 && nw == 4) nw = 8;
    if (wide_ok && !W->glu && ctx->force_nw) nw = ctx->force_nw;
    if (W->glu && ctx->force_nw_glu && wide_ok) nw = ctx->force_nw_glu;
    int S = 1;
    if (!argmax && ctx->min_items > a.n_groups) {
        const int want = (ctx->min_items + a.n_groups - 1) / a.n_groups;
        S = std::max(1, std::min(want, W->ksteps / nw));
    }
    // Register-direct GEMV where it measured faster than LDS staging: it saves
    // the staging pass but reloads the activations for every tile, so it wins
    // while a workgroup sees few tiles (or the tokens are few); the lm_head
    // (thousands of tiles per launch) keeps the staged kernel from M = 5 on.
    // A single BF16 token with a per-call gamma also stays staged (the gamma
    // traffic of every lane outweighs the saved pass).
    const bool gamma_call = ep && (ep->flags & QW_EP_NORM_X) && ep->gamma;
    const int tiles_per_wg = a.n_groups / std::max(1, ctx->num_cus * ctx->wg_per_cu);
    const bool direct = ctx->gemv && qwk::gemv_supported(W->wf, (int)xdt, M, ep && (ep->flags & QW_EP_NORM_X)) &&
                        !(M == 1 && gamma_call && W->wf == QW_WFMT_BF16) && (M <= 4 || tiles_per_wg <= 4);
    if (direct)
        nw = qwk::gemv_waves(W->wf, M, W->glu != 0, argmax, ep && (ep->flags & QW_EP_NORM_X), nw);
    if (direct && argmax) {  // the GEMV's argmax items may be runs of consecutive tiles
        const int rows = 16 * qwk::gemv_argmax_tiles(W->wf);
        a.n_groups = (W->N + rows - 1) / rows;
    }
    // the activation slice of a split must fit the workgroup's LDS
    while (!direct && qwk::skinny_lds_bytes(W->wf, (int)xdt, M, (W->ksteps + S - 1) / S) > qwk::kSkinnyMaxLds) {
        if (argmax || S >= W->ksteps) return fail(ctx, QW_ERR_SHAPE, "K=%d too large for the skinny kernel", W->K);
        ++S;
    }
    if (S > 1) {
        if ((int64_t)a.n_groups * groups > kMaxCounters) return fail(ctx, QW_ERR_WORKSPACE, "too many split-K tiles");
        if ((size_t)a.n_groups * groups * S * 64 * (RT * CT * 4 + CT) * 4 > ctx->partials_bytes)
            return fail(ctx, QW_ERR_WORKSPACE, "split-K partials exceed the workspace");
    }
    a.S = S;
    a.n_items = a.n_groups * S;
    a.flags = ep ? ep->flags : 0u;
    if (ep && (ep->flags & QW_EP_RESIDUAL)) {
        a.res = ep->residual;
        a.res_dt = ep->residual_dtype;
        a.ld_res = ep->ld_residual ? ep->ld_residual : W->N;
    }
    if (ep && (ep->flags & QW_EP_NORM_X)) {
        a.gamma = ep->gamma;
        a.eps = ep->eps;
    }
    a.y = y;
    a.ydt = ydt;
    a.ldy = ldy;
    if (ep && (ep->flags & QW_EP_SPLIT)) {
        a.y2 = ep->y2;
        a.split_period = ep->split_period;
    }
    bool vec = (W->N % 4 == 0) && (ldy % 4 == 0) && aligned(y, 16);
    if (a.flags & QW_EP_SPLIT) vec = vec && aligned(a.y2, 16);
    if (a.flags & QW_EP_RESIDUAL) vec = vec && (a.ld_res % 4 == 0) && aligned(a.res, 16);
    a.vec_store = vec ? 1 : 0;
    a.partials = ctx->partials;
    a.counters = ctx->counters;
    a.keys = ctx->keys;
    a.done = ctx->done;
    a.ids = ids;
    a.maxv = maxv;
    // a workgroup keeps one K split for its life: grid is a multiple of S
    int grid = std::min(a.n_items, ctx->num_cus * ctx->wg_per_cu);
    grid = std::max(S, grid - grid % S);
    if (groups > 1) {
        // the groups share the device's workgroup slots; a multiple of 8 per
        // group puts the workgroups of one tile (one per group) on one XCD,
        // where the later ones find its weights in L2
        int per = (ctx->num_cus * ctx->wg_per_cu + groups - 1) / groups;
        per = std::min(per, a.n_items);
        per = (per + 7) / 8 * 8;
        per = (per + S - 1) / S * S;
        a.tg_size = tg_size;
        a.tg_grid = per;
        grid = per * groups;
    }
    if ((uint64_t)W->bytes >= (1ull << 32) || (uint64_t)M_total * ldx * dsize(xdt) >= (1ull << 32))
        return fail(ctx, QW_ERR_SHAPE, "operands above 4 GiB are not supported");
    hipError_t e = direct ? qwk::launch_gemv(a, W->wf, (int)xdt, W->glu != 0, argmax, nw, grid, stream)
                          : qwk::launch_skinny(a, W->wf, (int)xdt, W->glu != 0, argmax, nw, grid, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "skinny kernel launch");
    return QW_OK;
}

// Weight-stationary launch (qw_wide.hip) for wide_min..wide_max tokens.
// Returns QW_ERR_SHAPE without launching when no configuration fits, so the
// caller can take the small-M kernels instead.
static qw_status run_wide(qw_ctx* ctx, const qw_weight* W, const void* x, qw_dtype xdt, int ldx, int M, void* y,
                          qw_dtype ydt, int ldy, const qw_epilogue* ep, hipStream_t stream) {
    qwk::WideArgs wa{};
    qwk::SkinnyArgs& a = wa.s;
    a.w = W->packed;
    a.scales = W->scales;
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = W->K;
    a.N = W->N;
    a.n_groups = (W->N + 15) / 16;
    a.ksteps = W->ksteps;
    a.flags = ep ? ep->flags : 0u;
    if (ep && (ep->flags & QW_EP_RESIDUAL)) {
        a.res = ep->residual;
        a.res_dt = ep->residual_dtype;
        a.ld_res = ep->ld_residual ? ep->ld_residual : W->N;
    }
    if (ep && (ep->flags & QW_EP_NORM_X)) {
        a.gamma = ep->gamma;
        a.eps = ep->eps;
    }
    a.y = y;
    a.ydt = ydt;
    a.ldy = ldy;
    if (ep && (ep->flags & QW_EP_SPLIT)) {
        a.y2 = ep->y2;
        a.split_period = ep->split_period;
    }
    bool vec = (W->N % 4 == 0) && (ldy % 4 == 0) && aligned(y, 16);
    if (a.flags & QW_EP_SPLIT) vec = vec && aligned(a.y2, 16);
    if (a.flags & QW_EP_RESIDUAL) vec = vec && (a.ld_res % 4 == 0) && aligned(a.res, 16);
    a.vec_store = vec ? 1 : 0;
    a.partials = ctx->partials;
    a.counters = ctx->counters;
    qwk::WidePlan p{};
    if (!qwk::wide_plan(a, W->wf, W->glu != 0, ctx->num_cus, kWidePartialsBytes, kMaxCounters, ctx->wide_s,
                        ctx->wide_cfg, p))
        return QW_ERR_SHAPE;
    if ((uint64_t)W->bytes >= (1ull << 32) || (uint64_t)M * ldx * dsize(xdt) >= (1ull << 32))
        return QW_ERR_SHAPE;
    a.S = p.S;
    wa.nblocks = p.nblocks;
    wa.n_ptiles = p.n_ptiles;
    wa.off_gamma = p.off_gamma;
    wa.off_res = p.off_res;
    wa.off_scales = p.off_scales;
    wa.res_lds = p.res_lds;
    wa.T = p.T;
    wa.Mg = p.Mg;
    wa.ngrp = p.ngrp;
    wa.dbg = ctx->wide_dbg;
    wa.wpart = ctx->wide_partials;
    wa.err = ctx->mlp_ctl + 3;
    if (ctx->wide_dbg & 8)
        fprintf(stderr, "wide N=%d K=%d M=%d glu=%d: S=%d T=%d NB=%d KW=%d CT=%d grid=%d smem=%zu\n", W->N, W->K, M,
                W->glu, p.S, p.T, p.NB, p.KW, p.CT, p.grid, p.smem);
    hipError_t e = qwk::launch_wide(wa, p, W->wf, (int)xdt, W->glu != 0, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "weight-stationary kernel launch");
    return QW_OK;
}

// MFMA GEMM launch for many tokens: BF16 weights with BF16 activations, INT8
// weights with F16 or BF16 activations.
static bool gemm_ok(const qw_weight* W, qw_dtype xdt) {
    return qwk::gemm_supported(W->wf, (int)xdt);
}

// Route of a call with M tokens: 0 = the small-M kernels (32-token groups
// streaming the weights), else the GEMM with 64- or 256-row blocks.
// Measured on MI355X with the weights streamed from HBM (distinct copies
// replayed from a graph, as in a decode step), BF16 and INT8 alike:
//   - up to ~128-192 tokens the small-M kernels win on every shape (gate/up
//     M=128: 15.5 us vs 26.2 us with 64-row blocks);
//   - 1024-row weights (out, down): small-M kernels up to 256 tokens (down
//     M=256: 17.8 us vs 26.2 us for split-K 64-row blocks); past 512 tokens,
//     and past 256 when K > 2048, 64-row blocks with split-K (BF16 down M=384
//     31.2 vs 38.8 us, M=768 42.6 vs 64.5 us; out M=768 29.7 vs 37.4 us; at
//     M=320..512 with K=2048 the small-M kernels win or tie, out M=320 19.3
//     vs 22.3 us);
//   - 4096..8192-row weights from ~256 tokens: 64-row blocks while they make
//     at most 512 tiles (QKV+Z M=256: 26 us vs 38 us with 256-row blocks vs
//     42 us small-M; 4096 rows at M=1024 22.0 vs 27.3 us), 256-row blocks
//     past that (8192 rows at M=768: 30.4 vs 40.3 us; M=1024, 8 distinct
//     weights each: QKV+Z 36.8 vs 61.1 us, gate/up 30.9 vs 44.1 us,
//     Q+gate/K/V 32.6 vs 40.8 us);
//   - lm_head-size weights (>= 128 row blocks): 256-row blocks from 128.
static int gemm_route(const qw_ctx* ctx, const qw_weight* W, qw_dtype xdt, int M) {
    if (!gemm_ok(W, xdt) || M < ctx->gemm_min_m) return 0;
    const int nb256 = (W->phys_tiles * 16 + 255) / 256;
    if (ctx->gemm_forced) return ctx->gemm_rows ? ctx->gemm_rows : (M <= 1024 && nb256 < 128 ? 64 : 256);
    int rows;
    if (nb256 < 16) rows = M >= 1536 ? 256 : ((M > 512 || (M > 256 && W->K > 2048)) ? 64 : 0);
    else if (nb256 >= 128) rows = M >= 128 ? 256 : 0;
    else if (M <= 192) rows = 0;
    else rows = (W->phys_tiles * 16 + 63) / 64 * ((M + 127) / 128) <= 512 ? 64 : 256;
    if (rows && ctx->gemm_rows) rows = ctx->gemm_rows;
    return rows;
}

static qw_status run_gemm(qw_ctx* ctx, const qw_weight* W, int rows, const void* x, qw_dtype xdt, int ldx, int M,
                          void* y, qw_dtype ydt, int ldy, const qw_epilogue* ep, int32_t* ids, float* maxv,
                          hipStream_t stream) {
    qwk::GemmArgs a{};
    a.w = W->packed;
    a.scales = W->scales;
    a.n_tiles = W->phys_tiles;
    a.ksteps = W->ksteps;
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = W->K;
    a.N = W->N;
    a.nblk_n = (W->phys_tiles * 16 + 255) / 256;
    // 256-token blocks (8 waves, half the L2->LDS traffic per FLOP of the
    // 128-token block) once they alone fill the 256 CUs and more than 128
    // tokens exist; 128-token blocks (two workgroups per CU) otherwise;
    // 64-row blocks (always 128 tokens) where gemm_route chose them
    a.tile_m = ctx->gemm_tile_m ? ctx->gemm_tile_m : (M > 128 && a.nblk_n * ((M + 255) / 256) >= 256 ? 256 : 128);
    a.rows = rows;
    if (rows == 64) {
        a.tile_m = 128;
        a.nblk_n = (W->phys_tiles * 16 + 63) / 64;
    }
    a.nblk_m = (M + a.tile_m - 1) / a.tile_m;
    a.waves = W->wf == QW_WFMT_INT8_ROWSCALE ? 8 : (a.tile_m == 256 ? ctx->gemm_waves : 4);
    a.flags = ep ? (ep->flags & ~(unsigned)QW_EP_NORM_X) : 0u;
    if (ep && (ep->flags & QW_EP_RESIDUAL)) {
        a.res = ep->residual;
        a.res_dt = ep->residual_dtype;
        a.ld_res = ep->ld_residual ? ep->ld_residual : W->N;
    }
    a.y = y;
    a.ydt = ydt;
    a.ldy = ldy;
    if (ep && (ep->flags & QW_EP_SPLIT)) {
        a.y2 = ep->y2;
        a.split_period = ep->split_period;
    }
    bool vec = (W->N % 4 == 0) && (ldy % 4 == 0) && aligned(y, 16);
    if (a.flags & QW_EP_SPLIT) vec = vec && aligned(a.y2, 16);
    if (a.flags & QW_EP_RESIDUAL) vec = vec && (a.ld_res % 4 == 0) && aligned(a.res, 16);
    a.vec_store = vec ? 1 : 0;
    a.keys = ctx->keys;
    a.done = ctx->done;
    a.ids = ids;
    a.maxv = maxv;
    // split-K (64-row blocks) where the tiles leave most CUs idle (the
    // 1024-row projections at a few hundred tokens): up to 4 K splits, at
    // least 8 K-blocks each,
    // while the partial tiles fit the workspace (QW_GEMM_SPLITK forces S)
    a.splitk = 1;
    const int tiles = a.nblk_n * a.nblk_m;
    if (!ids && rows == 64) {
        // about one workgroup per CU (M=1024 on 1024 rows: 128 tiles, 2 splits
        // 47 us vs 51 us with 4 for the down projection)
        int S = ctx->gemm_splitk > 0 ? ctx->gemm_splitk
                                     : (tiles * 2 <= ctx->num_cus ? std::min(4, ctx->num_cus / tiles) : 1);
        S = std::max(1, std::min(S, W->ksteps / 8));
        const size_t per = (size_t)qwk::gemm_acc_floats_per_thread(a.rows, a.tile_m, a.waves) * a.waves * 64 * 4;
        while (S > 1 && ((size_t)tiles * S * per > ctx->partials_bytes || tiles > kMaxCounters)) --S;
        a.splitk = S;
        a.partials = reinterpret_cast<float*>(ctx->partials);
        a.counters = ctx->counters;
    }
    if ((uint64_t)W->bytes >= (1ull << 31) || (uint64_t)M * ldx * 2 >= (1ull << 31))
        return fail(ctx, QW_ERR_SHAPE, "operands above 2 GiB are not supported");
    // the direct-A kernel (256 x 128 blocks, two per CU) wherever its blocks
    // occupy at least half the CUs: the prefill shapes, and from a few hundred
    // tokens on the wide projections (measured at 520 / 1024 tokens: gate/up
    // 30.7 / 28.3 -> 23.0 / 23.6 us, QKV+Z 34.3 -> 25.6 us at 520, Q+gate+K+V
    // 30.8 -> 24.2 us at 1024).  Fewer blocks keep the 64-row split-K GEMM: a
    // split-K direct-A kernel measured 1.7-2.9x slower on the 1024-row
    // projections (its last workgroup reads every partial tile through one CU)
    if (ctx->gemm_da && (rows == 256 || rows == 64) && !ctx->gemm_tile_m &&
        (ctx->gemm_da == 2 || 2 * ((W->phys_tiles * 16 + 255) / 256 * ((M + 127) / 128)) >= ctx->num_cus) &&
        qwk::gemm_da_fits(a, W->wf, (int)xdt, ids != nullptr)) {
        a.group_m = ctx->gemm_da_group;
        const int nwv = ctx->gemm_da_waves
                            ? ctx->gemm_da_waves
                            : ((W->phys_tiles * 16 + 511) / 512 * ((M + 127) / 128) >= ctx->num_cus ? 8 : 4);
        hipError_t e = qwk::launch_gemm_da(a, W->glu != 0, ctx->gemm_da_line, stream, nwv,
                                           ctx->gemm_da_persist ? ctx->num_cus : 0);
        if (e != hipSuccess) return hip_fail(ctx, e, "gemm launch");
        return QW_OK;
    }
    // fewer blocks than half the CUs (the 1024-row projections up to ~4000
    // tokens): the direct-A kernel with K split S ways into partial tiles, then
    // the reduce + epilogue kernel.  S is the fewest splits that give half the
    // CUs a workgroup (each split a multiple of the weight ring and >= 8
    // k-steps, the partials within the workspace): at 1024 tokens 128-224
    // workgroups measured best (down 46.8 -> 24 us, out 34.0 -> 20.5 us; 448
    // workgroups 30.5 us), at 3072 tokens S = 2 (down 94 -> 40 us, out 61 ->
    // 30 us).  QW_GEMM_DA_SPLIT forces S (0: off)
    const int da_blocks = (W->phys_tiles * 16 + 255) / 256 * ((M + 127) / 128);
    if (ctx->gemm_da && ctx->gemm_da_split != 0 && (rows == 256 || rows == 64) && !ctx->gemm_tile_m && !ids &&
        (ctx->gemm_da_split > 0 || 2 * da_blocks < ctx->num_cus)) {
        qwk::GemmArgs d = a;
        d.splitk = 1;
        d.group_m = ctx->gemm_da_group;
        d.partials = reinterpret_cast<float*>(ctx->partials);
        int S = 0;
        if (qwk::gemm_da_fits(d, W->wf, (int)xdt, false)) {
            for (int sc = 2; sc <= 32; ++sc) {
                if (W->ksteps % (4 * sc) != 0 || W->ksteps / sc < 8) continue;
                if (qwk::gemm_da_split_bytes(d, sc) > ctx->partials_bytes) break;
                if (ctx->gemm_da_split > 0) {
                    if (sc == ctx->gemm_da_split) S = sc;
                    continue;
                }
                S = sc;
                if (2 * da_blocks * sc >= ctx->num_cus) break;
            }
        }
        if (S >= 2) {
            hipError_t e = qwk::launch_gemm_da_split(d, W->glu != 0, ctx->gemm_da_line, S, stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "gemm launch");
            return QW_OK;
        }
    }
    hipError_t e = qwk::launch_gemm(a, W->wf, (int)xdt, W->glu != 0, ids != nullptr, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "GEMM launch");
    return QW_OK;
}

static qw_status check_linear(qw_ctx* ctx, const qw_weight* W, const void* x, qw_dtype xdt, int ldx,
                              int M, void* y, qw_dtype ydt, int ldy, const qw_epilogue* ep,
                              bool need_y) {
    if (!ctx) return QW_ERR_NULL;
    if (!W) return fail(ctx, QW_ERR_NULL, "weight is NULL");
    if (!x) return fail(ctx, QW_ERR_NULL, "x is NULL");
    if (need_y && !y) return fail(ctx, QW_ERR_NULL, "y is NULL");
    if (M < 1) return fail(ctx, QW_ERR_SHAPE, "M=%d must be >= 1", M);
    qw_status s = check_xdt(ctx, W, xdt);
    if (s != QW_OK) return s;
    if (need_y && !valid_act(ydt)) return fail(ctx, QW_ERR_DTYPE, "output dtype %d unsupported", (int)ydt);
    if (ldx < W->K) return fail(ctx, QW_ERR_SHAPE, "ldx=%d < K=%d", ldx, W->K);
    if (!aligned(x, 16) || ((size_t)ldx * dsize(xdt)) % 16 != 0)
        return fail(ctx, QW_ERR_ALIGN, "x must be 16-byte aligned with 16-byte aligned rows");
    if (need_y) {
        if (ldy < W->N && !(ep && (ep->flags & QW_EP_SPLIT)))
            return fail(ctx, QW_ERR_SHAPE, "ldy=%d < N=%d", ldy, W->N);
        if (!aligned(y, dsize(ydt))) return fail(ctx, QW_ERR_ALIGN, "y misaligned");
    }
    if (ep) {
        if (ep->flags & ~(unsigned)(QW_EP_RESIDUAL | QW_EP_NORM_X | QW_EP_SPLIT))
            return fail(ctx, QW_ERR_INVALID, "unknown epilogue flags 0x%x", ep->flags);
        if (ep->flags & QW_EP_RESIDUAL) {
            if (!ep->residual) return fail(ctx, QW_ERR_NULL, "residual is NULL");
            if (!valid_act(ep->residual_dtype)) return fail(ctx, QW_ERR_DTYPE, "residual dtype unsupported");
            if (!aligned(ep->residual, dsize(ep->residual_dtype))) return fail(ctx, QW_ERR_ALIGN, "residual misaligned");
            if (ep->ld_residual != 0 && ep->ld_residual < W->N) return fail(ctx, QW_ERR_SHAPE, "ld_residual < N");
        }
        if (ep->flags & QW_EP_NORM_X) {
            if (!ep->gamma && !W->norm_folded)
                return fail(ctx, QW_ERR_NULL, "gamma is NULL and the weight carries no folded norm weight");
            if (ep->gamma && W->norm_folded)
                return fail(ctx, QW_ERR_INVALID, "the weight already carries the norm weight: pass gamma = NULL");
            if (ep->gamma && !aligned(ep->gamma, 16)) return fail(ctx, QW_ERR_ALIGN, "gamma must be 16-byte aligned");
            if (!(ep->eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "eps must be > 0");
        }
        if (ep->flags & QW_EP_SPLIT) {
            if (!ep->y2) return fail(ctx, QW_ERR_NULL, "y2 is NULL");
            if (ep->split_period < 16 || (ep->split_period & (ep->split_period - 1)) != 0 ||
                W->N % (2 * ep->split_period) != 0)
                return fail(ctx, QW_ERR_SHAPE, "split_period must be a power of two >= 16 dividing N/2");
            if (W->glu) return fail(ctx, QW_ERR_INVALID, "split epilogue not available on GLU weights");
            if (ldy < W->N / 2) return fail(ctx, QW_ERR_SHAPE, "ldy < N/2");
        }
    }
    return QW_OK;
}

qw_status qw_linear(qw_ctx* ctx, const qw_weight* W, const void* x, qw_dtype xdt, int ldx, int M,
                    void* y, qw_dtype ydt, int ldy, const qw_epilogue* ep, hipStream_t stream) {
    if (W && ldx == 0) ldx = W->K;
    if (W && ldy == 0) ldy = (ep && (ep->flags & QW_EP_SPLIT)) ? W->N / 2 : W->N;
    qw_status s = check_linear(ctx, W, x, xdt, ldx, M, y, ydt, ldy, ep, true);
    if (s != QW_OK) return s;
    // weight-stationary kernel: every weight byte once for all tokens
    if (ctx->wide && !(ctx->gemm_forced && M >= ctx->gemm_min_m) && M >= ctx->wide_min && M <= ctx->wide_max &&
        qwk::wide_supported(W->wf, (int)xdt, M)) {
        const bool norm = ep && (ep->flags & QW_EP_NORM_X);
        if (norm && ctx->wide_norm_sep && (size_t)M * W->K * dsize(xdt) <= ctx->xnorm_bytes) {
            // RMSNorm into the workspace (one row per workgroup), then the
            // projection of the normalized activations: cheaper than the
            // in-kernel LDS pass, whose conversions are VALU-bound at many tokens
            hipError_t e = qwk::launch_rmsnorm_ld(x, (int)xdt, ldx, ep->gamma, ep->eps, ctx->xnorm, (int)xdt, W->K,
                                                  M, W->K, stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
            qw_epilogue e2 = *ep;
            e2.flags &= ~(unsigned)QW_EP_NORM_X;
            s = run_wide(ctx, W, ctx->xnorm, xdt, W->K, M, y, ydt, ldy, &e2, stream);
        } else {
            s = run_wide(ctx, W, x, xdt, ldx, M, y, ydt, ldy, ep, stream);
        }
        if (s != QW_ERR_SHAPE) return s;
    }
    if (const int rows = gemm_route(ctx, W, xdt, M)) {
        const bool norm = ep && (ep->flags & QW_EP_NORM_X);
        if (!norm) return run_gemm(ctx, W, rows, x, xdt, ldx, M, y, ydt, ldy, ep, nullptr, nullptr, stream);
        // RMSNorm into the workspace, then the GEMM, in token chunks that fit.
        // INT8 weights take F16 (their MFMA type: a BF16 copy would add ~1e-3
        // of rounding error, the whole INT8 tolerance).
        const qw_dtype ndt = W->wf == QW_WFMT_INT8_ROWSCALE ? QW_F16 : QW_BF16;
        const int chunk = (int)std::min<size_t>((size_t)M, ctx->xnorm_bytes / ((size_t)W->K * 2));
        if (chunk < 1) return fail(ctx, QW_ERR_WORKSPACE, "workspace too small for the RMSNorm-ed activations");
        qw_epilogue e3 = *ep;
        for (int m0 = 0; m0 < M; m0 += chunk) {
            const int mc = std::min(chunk, M - m0);
            const void* xc = static_cast<const uint8_t*>(x) + (size_t)m0 * ldx * dsize(xdt);
            hipError_t e = qwk::launch_rmsnorm_ld(xc, (int)xdt, ldx, ep->gamma, ep->eps, ctx->xnorm, (int)ndt,
                                                  W->K, mc, W->K, stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
            void* yc = static_cast<uint8_t*>(y) + (size_t)m0 * ldy * dsize(ydt);
            if (ep->flags & QW_EP_RESIDUAL) {
                const int ldr = ep->ld_residual ? ep->ld_residual : W->N;
                e3.residual = static_cast<const uint8_t*>(ep->residual) + (size_t)m0 * ldr * dsize(ep->residual_dtype);
            }
            if (ep->flags & QW_EP_SPLIT) e3.y2 = static_cast<uint8_t*>(ep->y2) + (size_t)m0 * ldy * dsize(ydt);
            s = run_gemm(ctx, W, rows, ctx->xnorm, ndt, W->K, mc, yc, ydt, ldy, &e3, nullptr, nullptr, stream);
            if (s != QW_OK) return s;
        }
        return QW_OK;
    }
    // small-M kernels: up to 32 tokens per workgroup (16 with the RMSNorm
    // prologue, which the register-direct GEMV takes 16 at a time); more
    // tokens run as token groups of one launch
    const bool norm = ep && (ep->flags & QW_EP_NORM_X);
    const int tg = (norm && ctx->gemv && qwk::gemv_supported(W->wf, (int)xdt, 16, true)) ? 16 : kSkinnyMaxM;
    return run_skinny(ctx, W, x, xdt, ldx, M, y, ydt, ldy, ep, nullptr, nullptr, stream, tg);
}

// The lm_head route shared by the context and no-allocation entry points:
// the weight-stationary argmax from wide_min tokens where it applies, else
// the GEMM or the small-M kernels.
static qw_status lmhead_route(qw_ctx* ctx, const qw_weight* E, const void* h, qw_dtype hdt, int M, int32_t* ids,
                              float* maxv, hipStream_t stream) {
    // INT8 E takes the weight-stationary argmax from 8 tokens (8 / 12 / 16
    // tokens: 50.4 / 50.5 / 50.6 us against 58.0 / 58.1 / 59.4 us for the
    // skinny kernel); BF16 E from wide_min (the two measure alike at 8..16)
    const int wmin = E->wf == QW_WFMT_INT8_ROWSCALE ? std::min(ctx->wide_min, ctx->argmax_wide_min_i8) : ctx->wide_min;
    if (ctx->wide && !(ctx->gemm_forced && M >= ctx->gemm_min_m) && M >= wmin && M <= ctx->wide_max &&
        !E->glu && aligned(E->packed, 16)) {
        qwk::WideArgmaxArgs a{};
        a.nw = ctx->argmax_nw;
        a.wcache = ctx->argmax_cache;
        int grid = 0;
        size_t smem = 0;
        // BF16 E at 65..128 tokens: the activation-stationary form streams E
        // once instead of once per 64-token group (96-98 against 99-101 us)
        const bool as = ctx->argmax_as && M >= ctx->argmax_as_min &&
                        qwk::as_argmax_plan(E->wf, (int)hdt, M, E->K, ctx->num_cus, grid, smem);
        if (as || qwk::wide_argmax_plan(E->wf, (int)hdt, M, E->K, ctx->num_cus, a, grid, smem)) {
            a.w = E->packed;
            a.scales = E->scales;
            a.x = h;
            a.ldx = E->K;
            a.M = M;
            a.K = E->K;
            a.V = E->N;
            a.n_tiles = E->phys_tiles;
            a.n_blk = (E->phys_tiles + 1) / 2;
            a.keys = ctx->keys;
            a.done = ctx->done;
            a.ids = ids;
            a.maxv = maxv;
            a.dbg = ctx->wide_dbg;
            hipError_t e = as ? qwk::launch_as_argmax(a, E->wf, (int)hdt, grid, smem, stream)
                              : qwk::launch_wide_argmax(a, E->wf, (int)hdt, grid, smem, stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "weight-stationary lm_head launch");
            return QW_OK;
        }
    }
    if (const int rows = gemm_route(ctx, E, hdt, M))
        return run_gemm(ctx, E, rows, h, hdt, E->K, M, nullptr, QW_F32, 0, nullptr, ids, maxv, stream);
    return run_skinny(ctx, E, h, hdt, E->K, M, nullptr, QW_F32, 0, nullptr, ids, maxv, stream, kSkinnyMaxM);
}

qw_status qw_lmhead_argmax(qw_ctx* ctx, const qw_weight* E, const void* h, qw_dtype hdt, int M,
                           int32_t* token_ids, float* max_logit, hipStream_t stream) {
    qw_status s = check_linear(ctx, E, h, hdt, E ? E->K : 0, M, nullptr, QW_F32, 0, nullptr, false);
    if (s != QW_OK) return s;
    if (!token_ids) return fail(ctx, QW_ERR_NULL, "token_ids is NULL");
    if (E->glu) return fail(ctx, QW_ERR_INVALID, "lm_head weight cannot be a GLU pair");
    if (M > kMaxKeys) return fail(ctx, QW_ERR_WORKSPACE, "M=%d exceeds %d argmax slots", M, kMaxKeys);
    return lmhead_route(ctx, E, h, hdt, M, token_ids, max_logit, stream);
}

}  // extern "C"

namespace qwi {

qw_status lmhead_argmax_scratch(int device, const void* packed, const float* scales, qw_wfmt fmt, int V, int K,
                                const void* h, qw_dtype hdt, int M, int32_t* token_ids, float* max_logit,
                                unsigned long long* keys, unsigned* done, hipStream_t stream) {
    if (!packed || !h || !token_ids) return QW_ERR_NULL;
    if (fmt != QW_WFMT_F32 && fmt != QW_WFMT_BF16 && fmt != QW_WFMT_INT8_ROWSCALE) return QW_ERR_DTYPE;
    if (fmt == QW_WFMT_INT8_ROWSCALE && !scales) return QW_ERR_NULL;
    if (V < 1 || K < 64 || K % 64 != 0 || M < 1) return QW_ERR_SHAPE;
    if (!aligned(packed, 16) || (scales && !aligned(scales, 16))) return QW_ERR_ALIGN;
    // a context and a weight descriptor on the stack: nothing is allocated
    qw_ctx c;
    c.device = device;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        c.num_cus = cus;
    c.keys = keys;
    c.done = done;
    qw_weight W;
    W.packed = static_cast<uint8_t*>(const_cast<void*>(packed));
    W.scales = fmt == QW_WFMT_INT8_ROWSCALE ? const_cast<float*>(scales) : nullptr;
    W.N = V;
    W.K = K;
    W.wf = fmt;
    W.phys_tiles = (V + 15) / 16;
    W.ksteps = K / (4 * ke_of(fmt));
    W.bytes = (size_t)W.phys_tiles * W.ksteps * 1024;
    W.owns = false;
    qw_status s = check_linear(&c, &W, h, hdt, K, M, nullptr, QW_F32, 0, nullptr, false);
    if (s != QW_OK) return s;
    return lmhead_route(&c, &W, h, hdt, M, token_ids, max_logit, stream);
}

}  // namespace qwi

extern "C" {

static qw_status gdn_run(qw_ctx* ctx, const qw_gdn_params* p, int batch, int tokens, const void* mixed_qkv,
                         const void* z, const void* a, const void* b, qw_dtype in_dtype, int ld_in,
                         float* conv_state, float* recurrent_state, void* out, qw_dtype out_dtype, int ld_out,
                         hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!p || !mixed_qkv || !z || !a || !b || !recurrent_state || !out || !p->conv_weight || !p->A_log ||
        !p->dt_bias || !p->norm_weight || (!conv_state && p->conv_kernel > 1))
        return fail(ctx, QW_ERR_NULL, "gdn: NULL argument");
    if (batch < 1 || tokens < 1)
        return fail(ctx, QW_ERR_SHAPE, "gdn: batch=%d, tokens=%d must be >= 1", batch, tokens);
    if (p->num_heads < 1 || p->key_dim != 128 || p->value_dim != 128 || p->conv_kernel < 1 || p->conv_kernel > 8)
        return fail(ctx, QW_ERR_SHAPE, "gdn: needs key_dim = value_dim = 128, 1 <= conv_kernel <= 8 (got %d, %d, %d)",
                    p->key_dim, p->value_dim, p->conv_kernel);
    if (!valid_act(in_dtype) || !valid_act(out_dtype)) return fail(ctx, QW_ERR_DTYPE, "gdn: dtype unsupported");
    const int vdim = p->num_heads * p->value_dim;
    if (ld_in < 1 || ld_out < vdim) return fail(ctx, QW_ERR_SHAPE, "gdn: ld_in=%d, ld_out=%d < %d", ld_in, ld_out, vdim);
    if ((int64_t)batch * p->num_heads > 65535 * 64 || batch > 65535)
        return fail(ctx, QW_ERR_SHAPE, "gdn: batch=%d too large", batch);
    qwk::GdnArgs g{};
    g.B = batch;
    g.T = tokens;
    g.nh = p->num_heads;
    g.kd = p->key_dim;
    g.vd = p->value_dim;
    g.K = p->conv_kernel;
    g.mixed = mixed_qkv;
    g.z = z;
    g.a = a;
    g.b = b;
    g.in_dt = (int)in_dtype;
    g.ld_in = ld_in;
    g.conv_w = p->conv_weight;
    g.A_log = p->A_log;
    g.dt_bias = p->dt_bias;
    g.norm_w = p->norm_weight;
    g.conv_state = conv_state;
    g.rec_state = recurrent_state;
    g.out = out;
    g.out_dt = (int)out_dtype;
    g.ld_out = ld_out;
    // long runs: the chunked form, when the workspace (normalized-activation and
    // intermediate regions, unused by this call) holds at least one chunk per sequence
    const size_t ws_free = ctx->xnorm_bytes + ctx->scratch_bytes;
    const bool chunked = tokens >= ctx->gdn_chunk_min &&
                         ws_free >= (size_t)batch * 64 * qwk::gdn_chunked_bytes_per_token(p->num_heads);
    hipError_t e = chunked ? qwk::launch_gdn_chunked(g, ctx->xnorm, ws_free, stream) : qwk::launch_gdn(g, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "gdn launch");
    return QW_OK;
}

qw_status qw_gdn_decode(qw_ctx* ctx, const qw_gdn_params* p, int batch, const void* mixed_qkv,
                        const void* z, const void* a, const void* b, qw_dtype in_dtype, int ld_in,
                        float* conv_state, float* recurrent_state, void* out, qw_dtype out_dtype,
                        int ld_out, hipStream_t stream) {
    return gdn_run(ctx, p, batch, 1, mixed_qkv, z, a, b, in_dtype, ld_in, conv_state, recurrent_state, out,
                   out_dtype, ld_out, stream);
}

qw_status qw_gdn_prefill(qw_ctx* ctx, const qw_gdn_params* p, int batch, int tokens, const void* mixed_qkv,
                         const void* z, const void* a, const void* b, qw_dtype in_dtype, int ld_in,
                         float* conv_state, float* recurrent_state, void* out, qw_dtype out_dtype, int ld_out,
                         hipStream_t stream) {
    return gdn_run(ctx, p, batch, tokens, mixed_qkv, z, a, b, in_dtype, ld_in, conv_state, recurrent_state, out,
                   out_dtype, ld_out, stream);
}

qw_status qw_attn_forward(qw_ctx* ctx, const qw_attn_params* p, const qw_kv_cache* cache, int batch, int tokens,
                          const int* positions, int max_len, const void* q, const void* gate, int q_head_stride,
                          const void* k, const void* v, qw_dtype in_dtype, int ld_in, void* out,
                          qw_dtype out_dtype, int ld_out, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!p || !cache || !positions || !q || !gate || !k || !v || !out || !p->q_norm_weight || !p->k_norm_weight ||
        !cache->k || !cache->v || (cache->dtype == QW_I8 && (!cache->k_scale || !cache->v_scale)))
        return fail(ctx, QW_ERR_NULL, "attn: NULL argument");
    if (batch < 1 || tokens < 1) return fail(ctx, QW_ERR_SHAPE, "attn: batch=%d, tokens=%d must be >= 1", batch, tokens);
    const int nh = p->num_heads, nkv = p->num_kv_heads, hd = p->head_dim;
    if (nkv < 1 || nh < nkv || nh % nkv || nh / nkv > 4 || (hd != 128 && hd != 256) || p->rotary_dim < 0 ||
        p->rotary_dim % 2 || p->rotary_dim > hd || !(p->rope_theta > 0.0f))
        return fail(ctx, QW_ERR_SHAPE, "attn: unsupported shape (heads %d/%d, head_dim %d, rotary %d)", nh, nkv, hd,
                    p->rotary_dim);
    if (cache->dtype != QW_I8 && cache->dtype != QW_F32) return fail(ctx, QW_ERR_DTYPE, "attn: cache dtype must be I8 or F32");
    if (cache->capacity < 1) return fail(ctx, QW_ERR_SHAPE, "attn: cache capacity %d", cache->capacity);
    if (!valid_act(in_dtype) || !valid_act(out_dtype)) return fail(ctx, QW_ERR_DTYPE, "attn: dtype unsupported");
    if (q_head_stride < hd || ld_in < 1 || ld_out < nh * hd)
        return fail(ctx, QW_ERR_SHAPE, "attn: q_head_stride=%d, ld_in=%d, ld_out=%d", q_head_stride, ld_in, ld_out);
    const int64_t rows_all = (int64_t)batch * tokens;
    int len = max_len > 0 ? std::min(max_len, cache->capacity) : cache->capacity;
    qwk::AttnArgs a{};
    a.B = batch;
    a.T = tokens;
    a.nh = nh;
    a.nkv = nkv;
    a.hd = hd;
    a.rot = p->rotary_dim;
    a.theta = p->rope_theta;
    a.qn_w = p->q_norm_weight;
    a.kn_w = p->k_norm_weight;
    a.q = q;
    a.gate = gate;
    a.k = k;
    a.v = v;
    a.q_hs = q_head_stride;
    a.in_dt = (int)in_dtype;
    a.ld_in = ld_in;
    a.kv_dt = (int)cache->dtype;  // qw_dtype codes are the kernels' DType codes
    a.kc = cache->k;
    a.vc = cache->v;
    a.ks = cache->k_scale;
    a.vs = cache->v_scale;
    a.cap = cache->capacity;
    a.pos = positions;
    a.out = out;
    a.out_dt = (int)out_dtype;
    a.ld_out = ld_out;
    a.err = ctx->mlp_ctl + 3;
    const size_t ws = ctx->xnorm_bytes + ctx->scratch_bytes;
    a.qn = reinterpret_cast<float*>(ctx->xnorm);
    if (tokens >= ctx->attn_prefill_min) {
        // query blocks of 16 tokens; segments of whole sequences, or of 16-token
        // chunks of one sequence, whose normalized q fit the workspace
        a.prefill = 1;
        if (cache->dtype == QW_I8) {
            // key splits of >= 256 keys, at most 8 per query block (the longest
            // block's chain is then <= 1/8 of the context)
            const int s8 = (len + 7) / 8;
            a.split = std::max(256, (s8 + 31) / 32 * 32);
            a.nsplit = (len + a.split - 1) / a.split;
        } else {
            a.split = len;
            a.nsplit = 1;
        }
        const size_t per_row = (size_t)nh * hd * 4 + (a.nsplit > 1 ? (size_t)nh * a.nsplit * (hd + 2) * 4 : 0);
        const int64_t seq_fit = (int64_t)(ws / (per_row * (size_t)tokens));
        if (seq_fit >= 1) {
            const int64_t nbseg = std::min<int64_t>({(int64_t)batch, seq_fit, (int64_t)65535});
            for (int b0 = 0; b0 < batch; b0 += (int)nbseg) {
                a.b0 = b0;
                a.nb = (int)std::min<int64_t>(nbseg, batch - b0);
                a.tb = 0;
                a.ntok = tokens;
                a.row0 = b0 * tokens;
                a.rows = a.nb * tokens;
                a.part = a.qn + (size_t)a.rows * nh * hd;
                hipError_t e = qwk::launch_attn(a, stream);
                if (e != hipSuccess) return hip_fail(ctx, e, "attn launch");
            }
        } else {
            const int chunk = (int)(ws / per_row) / 16 * 16;
            if (chunk < 16) return fail(ctx, QW_ERR_WORKSPACE, "attn: workspace too small for 16 tokens");
            for (int b0 = 0; b0 < batch; ++b0)
                for (int tb = 0; tb < tokens; tb += chunk) {
                    a.b0 = b0;
                    a.nb = 1;
                    a.tb = tb;
                    a.ntok = std::min(chunk, tokens - tb);
                    a.row0 = b0 * tokens + tb;
                    a.rows = a.ntok;
                    a.part = a.qn + (size_t)a.rows * nh * hd;
                    hipError_t e = qwk::launch_attn(a, stream);
                    if (e != hipSuccess) return hip_fail(ctx, e, "attn launch");
                }
        }
        return QW_OK;
    }
    // few tokens per sequence: key-split rows.  Keys per split (a multiple
    // of 64 in 128..1024) minimize the busiest CU's work: the workgroups
    // spread round-robin over the CUs, so a CU gets ceil(W / CUs) of them,
    // each costing its keys plus ~64 keys' worth of fixed work (q, partials).
    // B=1 at context 32769: 320 keys (206 workgroups) 30 us against 34 us
    // for 128 keys (514 workgroups: a second round for two of them).
    int split = 128;
    {
        int64_t best = -1;
        for (int sp = 128; sp <= 1024; sp += 64) {
            const int64_t w = (int64_t)rows_all * nkv * ((len + sp - 1) / sp);
            const int64_t cost = (w + ctx->num_cus - 1) / ctx->num_cus * (sp + 64);
            if (best < 0 || cost < best) {
                best = cost;
                split = sp;
            }
        }
    }
    if (ctx->attn_split > 0) split = ctx->attn_split;  // forced (QW_ATTN_SPLIT, multiple of 64)
    const int nsplit = (len + split - 1) / split;
    const size_t per_row = qwk::attn_bytes_per_row(nh, hd, nsplit);
    const int64_t seg = std::min<int64_t>({rows_all, (int64_t)(ws / per_row), (int64_t)65535});
    if (seg < 1) return fail(ctx, QW_ERR_WORKSPACE, "attn: workspace too small for one row");
    a.split = split;
    a.nsplit = nsplit;
    // one new token per sequence over an INT8 cache: one launch per segment
    // (q/k/v preparation and the split merge inside the attention kernel)
    // when the launch is small (at most 16 splits: one wave merges a head's
    // splits with device-coherent loads, which at hundreds of splits costs
    // more than the two launches; at most one workgroup per CU: with more,
    // every workgroup redoing its q heads and the hand-off cost more than the
    // launches save -- measured B=1 context 512: 21.3 vs 23.3 us, B=32
    // context 4096: 100.7 vs 96.2 us)
    a.cnt = (tokens == 1 && ctx->attn_fused && (int)cache->dtype == (int)QW_I8 && nsplit <= 16 &&
             seg * nkv * nsplit <= ctx->num_cus && seg * nkv <= kMaxCounters)
                ? ctx->counters
                : nullptr;
    // coalesced V loads once the launch has a workgroup per CU (see attn_decode_i8h)
    a.vcoal = ctx->attn_vcoal < 0 ? ((int64_t)std::min<int64_t>(seg, rows_all) * nkv * nsplit >= ctx->num_cus ? 1 : 0)
                                  : ctx->attn_vcoal;
    // rows in order, so every row finds the keys of the rows before it in the cache
    for (int64_t r0 = 0; r0 < rows_all; r0 += seg) {
        a.row0 = (int)r0;
        a.rows = (int)std::min<int64_t>(seg, rows_all - r0);
        a.part = a.qn + (size_t)a.rows * nh * hd;
        hipError_t e = qwk::launch_attn(a, stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "attn launch");
    }
    return QW_OK;
}

qw_status qw_embedding_gather(qw_ctx* ctx, const void* table, qw_dtype table_dtype, int vocab, int hidden,
                              const int32_t* ids, int M, void* out, qw_dtype out_dtype, int ld_out,
                              hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!table || !ids || !out) return fail(ctx, QW_ERR_NULL, "embedding: NULL argument");
    if (table_dtype != QW_F32 && table_dtype != QW_BF16) return fail(ctx, QW_ERR_DTYPE, "embedding: table must be F32 or BF16");
    if (!valid_act(out_dtype)) return fail(ctx, QW_ERR_DTYPE, "embedding: output dtype unsupported");
    if (vocab < 1 || hidden < 4 || hidden % 4 || M < 1)
        return fail(ctx, QW_ERR_SHAPE, "embedding: vocab=%d, hidden=%d, M=%d", vocab, hidden, M);
    if (ld_out == 0) ld_out = hidden;
    if (ld_out < hidden || ld_out % 4) return fail(ctx, QW_ERR_SHAPE, "embedding: ld_out=%d", ld_out);
    hipError_t e = qwk::launch_embed_gather(table, (int)table_dtype, vocab, hidden, ids, M, out, (int)out_dtype, ld_out,
                                            ctx->mlp_ctl + 3, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "embedding launch");
    return QW_OK;
}

qw_status qw_positions_add(qw_ctx* ctx, int32_t* positions, int n, int delta, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!positions) return fail(ctx, QW_ERR_NULL, "positions: NULL");
    if (n < 1) return fail(ctx, QW_ERR_SHAPE, "positions: n=%d", n);
    hipError_t e = qwk::launch_positions_add(positions, n, delta, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "positions launch");
    return QW_OK;
}

qw_status qw_mlp_fused(qw_ctx* ctx, const qw_weight* gateup, const qw_weight* down, const void* x,
                       qw_dtype xdt, const float* gamma, float eps, const void* residual,
                       qw_dtype residual_dtype, void* y, qw_dtype ydt, int M, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!gateup || !down) return fail(ctx, QW_ERR_NULL, "weights are NULL");
    if (!gateup->glu) return fail(ctx, QW_ERR_INVALID, "gateup must be a GLU weight");
    if (down->glu) return fail(ctx, QW_ERR_INVALID, "down must not be a GLU weight");
    const int H = gateup->K, I = gateup->N;
    if (down->K != I || down->N != H)
        return fail(ctx, QW_ERR_SHAPE, "down is [%d][%d], expected [%d][%d]", down->N, down->K, H, I);
    if (M < 1) return fail(ctx, QW_ERR_SHAPE, "M=%d must be >= 1", M);
    if (gateup->norm_folded && gamma)
        return fail(ctx, QW_ERR_INVALID, "gateup already carries the norm weight: pass gamma = NULL");
    const bool norm = gamma != nullptr || gateup->norm_folded;
    // intermediate h keeps the precision the down projection consumes
    const qw_dtype hdt = gateup->wf == QW_WFMT_F32 ? QW_F32 : (gateup->wf == QW_WFMT_BF16 ? QW_BF16 : QW_F16);
    const size_t per_tok = (size_t)I * dsize(hdt);
    int chunk = (int)std::min<size_t>((size_t)M, ctx->scratch_bytes / per_tok);
    if (chunk < 1) return fail(ctx, QW_ERR_WORKSPACE, "workspace too small for one token of the MLP");
    // decode: the whole block in one launch (BF16 or INT8 weights, up to 16
    // tokens of 16-bit activations or 4 of FP32, Qwen-sized projections)
    const int wfi = (int)gateup->wf;
    const bool one_launch = ctx->mlp_fused > 0 || (ctx->mlp_fused < 0 && gateup->wf == QW_WFMT_BF16);
    if (one_launch && M <= qwk::mlp_fused_max_m((int)xdt) && (size_t)M * per_tok <= ctx->scratch_bytes &&
        ((gateup->wf == QW_WFMT_BF16 && (xdt == QW_BF16 || xdt == QW_F32)) ||
         (gateup->wf == QW_WFMT_INT8_ROWSCALE && (xdt == QW_F16 || xdt == QW_BF16 || xdt == QW_F32))) &&
        valid_act(ydt) && (!residual || valid_act(residual_dtype)) && down->wf == gateup->wf &&
        gateup->ksteps <= qwk::mlp_fused_max_ksteps(wfi, false) && qwk::mlp_counter_words() <= kMlpCounterWords &&
        down->ksteps <= qwk::mlp_fused_max_ksteps(wfi, true) &&
        aligned(x, 16) && (H * dsize(xdt)) % 16 == 0 && (!gamma || aligned(gamma, 16))) {
        if (norm && !(eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "eps must be > 0");
        qwk::MlpArgs p{};
        qwk::SkinnyArgs& u = p.up;
        u.w = gateup->packed; u.scales = gateup->scales; u.x = x; u.ldx = H; u.M = M; u.K = H; u.N = I;
        u.n_groups = (I + 15) / 16; u.S = 1; u.ksteps = gateup->ksteps; u.n_items = u.n_groups;
        u.flags = norm ? QW_EP_NORM_X : 0u; u.gamma = gamma; u.eps = eps;
        u.y = ctx->scratch; u.ydt = hdt; u.ldy = I;
        qwk::SkinnyArgs& d = p.down;
        d.w = down->packed; d.scales = down->scales; d.x = ctx->scratch; d.ldx = I; d.M = M; d.K = I; d.N = H;
        d.n_groups = (H + 15) / 16; d.S = 1; d.ksteps = down->ksteps; d.n_items = d.n_groups;
        d.flags = residual ? QW_EP_RESIDUAL : 0u; d.res = residual; d.res_dt = residual_dtype; d.ld_res = H;
        d.y = y; d.ydt = ydt; d.ldy = H;
        d.vec_store = (H % 4 == 0) && aligned(y, 16) && (!residual || aligned(residual, 16));
        p.ctl = ctx->mlp_ctl;
        p.cnt = ctx->counters + kMaxCounters;

        p.n_up = u.n_groups;
        p.n_down = d.n_groups;
        hipError_t e = qwk::launch_mlp_fused(p, wfi, (int)xdt, stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "fused MLP launch");
        return QW_OK;
    }
    qw_epilogue e1{};
    if (norm) {
        e1.flags = QW_EP_NORM_X;
        e1.gamma = gamma;
        e1.eps = eps;
    }
    qw_epilogue e2{};
    if (residual) {
        e2.flags = QW_EP_RESIDUAL;
        e2.residual_dtype = residual_dtype;
    }
    for (int m0 = 0; m0 < M; m0 += chunk) {
        const int mc = std::min(chunk, M - m0);
        const void* xc = static_cast<const uint8_t*>(x) + (size_t)m0 * H * dsize(xdt);
        void* yc = static_cast<uint8_t*>(y) + (size_t)m0 * H * dsize(ydt);
        qw_status s = qw_linear(ctx, gateup, xc, xdt, H, mc, ctx->scratch, hdt, I, norm ? &e1 : nullptr, stream);
        if (s != QW_OK) return s;
        if (residual) e2.residual = static_cast<const uint8_t*>(residual) + (size_t)m0 * H * dsize(residual_dtype);
        s = qw_linear(ctx, down, ctx->scratch, hdt, I, mc, yc, ydt, H, residual ? &e2 : nullptr, stream);
        if (s != QW_OK) return s;
    }
    return QW_OK;
}

qw_status qw_layer_tail(qw_ctx* ctx, const qw_weight* w_out, const void* core, qw_dtype core_dtype, int ld_core,
                        const qw_weight* gateup, const qw_weight* down, const float* gamma, float eps, float* x,
                        int M, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!w_out || !core || !gateup || !down || !x) return fail(ctx, QW_ERR_NULL, "layer_tail: NULL argument");
    if (w_out->glu) return fail(ctx, QW_ERR_INVALID, "layer_tail: w_out must not be a GLU weight");
    if (!gateup->glu || down->glu) return fail(ctx, QW_ERR_INVALID, "layer_tail: gateup must be GLU, down not");
    const int H = gateup->K;
    if (w_out->N != H || down->N != H || down->K != gateup->N)
        return fail(ctx, QW_ERR_SHAPE, "layer_tail: w_out [%d][%d], gateup [%d][%d], down [%d][%d] do not chain",
                    w_out->N, w_out->K, gateup->N, gateup->K, down->N, down->K);
    if (M < 1) return fail(ctx, QW_ERR_SHAPE, "layer_tail: M=%d must be >= 1", M);
    const int ldc = ld_core ? ld_core : w_out->K;
    if (ldc < w_out->K) return fail(ctx, QW_ERR_SHAPE, "layer_tail: ld_core %d < K %d", ldc, w_out->K);
    if (gateup->norm_folded && gamma)
        return fail(ctx, QW_ERR_INVALID, "layer_tail: gateup already carries the norm weight: pass gamma = NULL");
    const bool norm = gamma != nullptr || gateup->norm_folded;
    const int wfi = (int)gateup->wf;
    const qw_dtype hdt = gateup->wf == QW_WFMT_BF16 ? QW_BF16 : QW_F16;
    // one launch: the fused MLP's decode route with the out-projection stage
    const bool one = ctx->layer_tail && ctx->mlp_fused != 0 && core_dtype == QW_BF16 &&
                     (gateup->wf == QW_WFMT_BF16 || gateup->wf == QW_WFMT_INT8_ROWSCALE) &&
                     w_out->wf == gateup->wf && down->wf == gateup->wf && M <= qwk::mlp_fused_max_m(QW_F32) &&
                     H <= 1024 && H % 16 == 0 && (H + 15) / 16 <= (gateup->N + 15) / 16 &&
                     w_out->ksteps <= qwk::mlp_pre_max_ksteps(wfi) &&
                     w_out->K % (gateup->wf == QW_WFMT_BF16 ? 32 : 64) == 0 &&
                     gateup->ksteps <= qwk::mlp_fused_max_ksteps(wfi, false) &&
                     down->ksteps <= qwk::mlp_fused_max_ksteps(wfi, true) &&
                     qwk::mlp_counter_words() <= kMlpCounterWords && (size_t)M * gateup->N * dsize(hdt) <= ctx->scratch_bytes &&
                     (size_t)M * H * 4 <= ctx->partials_bytes && aligned(x, 16) && aligned(core, 16) && ldc % 8 == 0 &&
                     (!gamma || aligned(gamma, 16));
    if (one) {
        if (norm && !(eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "eps must be > 0");
        float* xmid = reinterpret_cast<float*>(ctx->partials);
        qwk::MlpArgs p{};
        qwk::SkinnyArgs& o = p.pre;
        o.w = w_out->packed; o.scales = w_out->scales; o.x = core; o.ldx = ldc; o.M = M; o.K = w_out->K; o.N = H;
        o.n_groups = (H + 15) / 16; o.S = 1; o.ksteps = w_out->ksteps; o.n_items = o.n_groups;
        o.flags = QW_EP_RESIDUAL; o.res = x; o.res_dt = QW_F32; o.ld_res = H;
        o.y = xmid; o.ydt = QW_F32; o.ldy = H;
        p.xmid = xmid;
        qwk::SkinnyArgs& u = p.up;
        u.w = gateup->packed; u.scales = gateup->scales; u.x = x; u.ldx = H; u.M = M; u.K = H; u.N = gateup->N;
        u.n_groups = (gateup->N + 15) / 16; u.S = 1; u.ksteps = gateup->ksteps; u.n_items = u.n_groups;
        u.flags = norm ? QW_EP_NORM_X : 0u; u.gamma = gamma; u.eps = eps;
        u.y = ctx->scratch; u.ydt = hdt; u.ldy = gateup->N;
        qwk::SkinnyArgs& d = p.down;
        d.w = down->packed; d.scales = down->scales; d.x = ctx->scratch; d.ldx = gateup->N; d.M = M; d.K = gateup->N;
        d.N = H; d.n_groups = (H + 15) / 16; d.S = 1; d.ksteps = down->ksteps; d.n_items = d.n_groups;
        d.flags = QW_EP_RESIDUAL; d.res = xmid; d.res_dt = QW_F32; d.ld_res = H;
        d.y = x; d.ydt = QW_F32; d.ldy = H;
        d.vec_store = 1;
        p.ctl = ctx->mlp_ctl;
        p.cnt = ctx->counters + kMaxCounters;
        p.n_up = u.n_groups;
        p.n_down = d.n_groups;
        hipError_t e = qwk::launch_mlp_fused(p, wfi, (int)QW_F32, stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "layer tail launch");
        return QW_OK;
    }
    qw_epilogue ep{};
    ep.flags = QW_EP_RESIDUAL;
    ep.residual = x;
    ep.residual_dtype = QW_F32;
    ep.ld_residual = H;
    qw_status s = qw_linear(ctx, w_out, core, core_dtype, ldc, M, x, QW_F32, H, &ep, stream);
    if (s != QW_OK) return s;
    return qw_mlp_fused(ctx, gateup, down, x, QW_F32, gamma, eps, x, QW_F32, x, QW_F32, M, stream);
}

qw_status qw_mlp_stack(qw_ctx* ctx, int L, const qw_weight* const* gateup, const qw_weight* const* down,
                       const float* const* gamma, float eps, const void* x, qw_dtype xdt, void* y, int M,
                       hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!gateup || !down || !x || !y) return fail(ctx, QW_ERR_NULL, "mlp_stack: NULL argument");
    if (L < 1) return fail(ctx, QW_ERR_SHAPE, "mlp_stack: L=%d must be >= 1", L);
    if (M < 1) return fail(ctx, QW_ERR_SHAPE, "mlp_stack: M=%d must be >= 1", M);
    if (!valid_act(xdt)) return fail(ctx, QW_ERR_DTYPE, "mlp_stack: activation dtype unsupported");
    bool one = ctx->mlp_stack && L <= qwk::kMlpStackMaxLayers && M <= qwk::mlp_stack_max_m() &&
               ctx->num_cus >= qwk::mlp_stack_grid() && aligned(x, 16) && aligned(y, 16) &&
               qwk::mlp_stack_ws_bytes() <= kStackBytes && eps > 0.0f;
    for (int l = 0; l < L; ++l) {
        if (!gateup[l] || !down[l]) return fail(ctx, QW_ERR_NULL, "mlp_stack: layer %d weight is NULL", l);
        const qw_weight* gu = gateup[l];
        const qw_weight* dn = down[l];
        const bool g = gamma && gamma[l];
        one = one && gu->glu && !dn->glu && gu->K == 1024 && gu->N == 3584 && dn->K == 3584 && dn->N == 1024 &&
              gu->wf == gateup[0]->wf && dn->wf == gu->wf &&
              ((gu->wf == QW_WFMT_BF16 && xdt == QW_BF16) || (gu->wf == QW_WFMT_INT8_ROWSCALE && xdt == QW_F16)) &&
              (g ? !gu->norm_folded : gu->norm_folded) && (g == (gamma && gamma[0] != nullptr));
    }
    if (one) {
        qwk::MlpStackArgs a{};
        for (int l = 0; l < L; ++l) {
            a.gu[l] = gateup[l]->packed;
            a.dn[l] = down[l]->packed;
            a.gu_scales[l] = gateup[l]->scales;
            a.dn_scales[l] = down[l]->scales;
            a.gamma[l] = gamma ? gamma[l] : nullptr;
        }
        a.x = x;
        a.y = y;
        a.M = M;
        a.L = L;
        a.eps = eps;
        a.hbuf = ctx->stack_words;
        a.epoch = ctx->stack_epoch;
        a.err = ctx->mlp_ctl + 3;
        a.dbg = ctx->stack_dbg;
        a.trace = ctx->stack_trace;
        a.gap = ctx->stack_gap >= 0 ? ctx->stack_gap : (gateup[0]->wf == QW_WFMT_INT8_ROWSCALE ? 120 : 20);
        hipError_t e = qwk::launch_mlp_stack(a, (int)gateup[0]->wf, (int)xdt, stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "MLP stack launch");
        return QW_OK;
    }
    // one qw_mlp_fused per block, in place on y
    const void* in = x;
    for (int l = 0; l < L; ++l) {
        qw_status s = qw_mlp_fused(ctx, gateup[l], down[l], in, xdt, gamma ? gamma[l] : nullptr, eps, in, xdt, y, xdt,
                                   M, stream);
        if (s != QW_OK) return s;
        in = y;
    }
    return QW_OK;
}

// ---------------------------------------------------------------------------
// projection chains
// ---------------------------------------------------------------------------

struct qw_chain {
    qw_ctx* ctx = nullptr;
    qwk::ChainArgs args{};
    int wf = 0, adt = 0;
    uint8_t* mem = nullptr;  // op table, epoch words, slot words
    uint64_t* trace = nullptr;  // QW_CHAIN_TRACE=<file>: per-op stamps of the last launch, written at destroy
    std::string trace_path;
};

qw_status qw_chain_create(qw_ctx* ctx, qw_dtype act_dtype, int M, int n_slots, const qw_chain_slot* slots,
                          int n_ops, const qw_chain_op* ops, qw_chain** out) {
    if (!ctx) return QW_ERR_NULL;
    if (!slots || !ops || !out) return fail(ctx, QW_ERR_NULL, "chain: NULL argument");
    *out = nullptr;
    if (M < 1 || M > qwk::chain_max_m()) return fail(ctx, QW_ERR_SHAPE, "chain: M=%d outside 1..%d", M, qwk::chain_max_m());
    if (n_slots < 1 || n_slots > 64 || n_ops < 1 || n_ops > qwk::kChainMaxOps)
        return fail(ctx, QW_ERR_SHAPE, "chain: %d slots / %d ops out of range", n_slots, n_ops);
    if (ctx->num_cus < qwk::chain_grid()) return fail(ctx, QW_ERR_INVALID, "chain: needs %d CUs", qwk::chain_grid());
    const int wf = ops[0].w ? (int)ops[0].w->wf : -1;
    if (!((wf == QW_WFMT_BF16 && act_dtype == QW_BF16) || (wf == QW_WFMT_INT8_ROWSCALE && act_dtype == QW_F16)))
        return fail(ctx, QW_ERR_DTYPE, "chain: BF16 weights with BF16 slots or INT8 weights with F16 slots");
    size_t words = 0;
    std::vector<size_t> slot_word0(n_slots);
    int n_imports = 0;
    for (int s = 0; s < n_slots; ++s) {
        const qw_chain_slot& sl = slots[s];
        if (sl.len < 16 || sl.len % 16) return fail(ctx, QW_ERR_SHAPE, "chain: slot %d length %d", s, sl.len);
        if (sl.init && ((sl.ld_init ? sl.ld_init : sl.len) < sl.len || (sl.ld_init % 2) || !aligned(sl.init, 4)))
            return fail(ctx, QW_ERR_SHAPE, "chain: slot %d init layout", s);
        if (sl.out && ((sl.ld_out ? sl.ld_out : sl.len) < sl.len || (sl.ld_out % 2) || !aligned(sl.out, 4)))
            return fail(ctx, QW_ERR_SHAPE, "chain: slot %d out layout", s);
        if (sl.init && ++n_imports > qwk::kChainMaxImports)
            return fail(ctx, QW_ERR_SHAPE, "chain: more than %d imported slots", qwk::kChainMaxImports);
        slot_word0[s] = words;
        words += (size_t)M * (sl.len / 2);
    }
    // per slot: the writer of its current values (op index + 1, 0 = imported,
    // -1 = none) and how many rows of it that writer produced
    std::vector<int> writer(n_slots), rows(n_slots);
    for (int s = 0; s < n_slots; ++s) {
        writer[s] = slots[s].init ? 0 : -1;
        rows[s] = slots[s].init ? slots[s].len : 0;
    }
    std::vector<qwk::ChainOp> dev(n_ops);
    int base = 0;
    for (int i = 0; i < n_ops; ++i) {
        const qw_chain_op& op = ops[i];
        const qw_weight* W = op.w;
        if (!W) return fail(ctx, QW_ERR_NULL, "chain: op %d weight is NULL", i);
        if ((int)W->wf != wf) return fail(ctx, QW_ERR_DTYPE, "chain: op %d weight format differs", i);
        if (op.in < 0 || op.in >= n_slots || op.out < 0 || op.out >= n_slots || op.in == op.out)
            return fail(ctx, QW_ERR_INVALID, "chain: op %d slots %d -> %d", i, op.in, op.out);
        if (i > 0 && op.in != ops[i - 1].out)
            return fail(ctx, QW_ERR_INVALID, "chain: op %d must read op %d's output slot", i, i - 1);
        if (writer[op.in] < 0) return fail(ctx, QW_ERR_INVALID, "chain: op %d reads slot %d before any value", i, op.in);
        if (W->K > qwk::kChainMaxK || op.in_offset < 0 || op.in_offset % 64 || op.in_offset + W->K > rows[op.in])
            return fail(ctx, QW_ERR_SHAPE, "chain: op %d input [%d, %d) of %d rows", i, op.in_offset,
                        op.in_offset + W->K, rows[op.in]);
        if (W->N % 16 || W->N > slots[op.out].len) return fail(ctx, QW_ERR_SHAPE, "chain: op %d N=%d", i, W->N);
        if (op.residual && (writer[op.out] < 0 || rows[op.out] < W->N))
            return fail(ctx, QW_ERR_INVALID, "chain: op %d residual rows not written before", i);
        if (op.norm && !op.gamma && !W->norm_folded)
            return fail(ctx, QW_ERR_NULL, "chain: op %d norm without gamma or folded weight", i);
        if (op.gamma && (W->norm_folded || !op.norm)) return fail(ctx, QW_ERR_INVALID, "chain: op %d gamma", i);
        if (op.norm && !(op.eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "chain: op %d eps", i);
        const int n_blk = W->glu ? W->N / 16 : W->phys_tiles;
        if (n_blk > qwk::chain_max_blocks()) return fail(ctx, QW_ERR_SHAPE, "chain: op %d has %d blocks", i, n_blk);
        const int RT = W->glu ? 2 : 1;
        const int per_wg = (n_blk + qwk::chain_grid() - 1) / qwk::chain_grid();
        const int units = per_wg * W->ksteps;
        const int per_wave = (units + qwk::chain_compute_waves() - 1) / qwk::chain_compute_waves();
        if (per_wave * RT > qwk::chain_max_loads(wf) || W->ksteps < 10)
            return fail(ctx, QW_ERR_SHAPE, "chain: op %d needs %d weight loads per wave", i, per_wave * RT);
        qwk::ChainOp& d = dev[i];
        d.w = W->packed;
        d.scales = W->scales;
        d.glu = W->glu;
        d.n_blk = n_blk;
        d.ksteps = W->ksteps;
        d.K = W->K;
        d.N = W->N;
        d.in_ld = slots[op.in].len / 2;
        d.in_off = op.in_offset;
        d.in_tag = writer[op.in];
        d.gamma = op.gamma;
        d.norm = op.norm ? 1 : 0;
        d.eps = op.eps;
        d.out_ld = slots[op.out].len / 2;
        d.exp = static_cast<uint16_t*>(slots[op.out].out);
        d.exp_ld = slots[op.out].ld_out ? slots[op.out].ld_out : slots[op.out].len;
        d.residual = op.residual ? 1 : 0;
        d.res_tag = op.residual ? writer[op.out] : 0;
        // consecutive ops continue the round robin where the last one ended,
        // so a small op after a small op lands on other CUs
        d.base = base;
        base = (base + n_blk) % qwk::chain_grid();
        writer[op.out] = i + 1;
        rows[op.out] = std::max(rows[op.out], W->N);
    }
    qw_chain* ch = new qw_chain();
    ch->ctx = ctx;
    ch->wf = wf;
    ch->adt = (int)act_dtype;
    const size_t op_bytes = ((sizeof(qwk::ChainOp) * n_ops + 255) / 256) * 256;
    const size_t total = op_bytes + 256 + words * 8;
    hipSetDevice(ctx->device);
    if (hipMalloc(&ch->mem, total) != hipSuccess) {
        delete ch;
        return fail(ctx, QW_ERR_NOMEM, "chain: hipMalloc of %zu bytes failed", total);
    }
    uint64_t* wbase = reinterpret_cast<uint64_t*>(ch->mem + op_bytes + 256);
    for (int i = 0; i < n_ops; ++i) {
        dev[i].in_words = wbase + slot_word0[ops[i].in];
        dev[i].out_words = wbase + slot_word0[ops[i].out];
    }
    hipError_t e = hipMemcpy(ch->mem, dev.data(), sizeof(qwk::ChainOp) * n_ops, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(ch->mem + op_bytes, 0, 256 + words * 8);
    // epoch 1: the zeroed slot words (tag 0) never match a tag of a launch
    const unsigned one = 1u;
    if (e == hipSuccess) e = hipMemcpy(ch->mem + op_bytes, &one, sizeof one, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        hipFree(ch->mem);
        delete ch;
        return hip_fail(ctx, e, "chain setup");
    }
    qwk::ChainArgs& A = ch->args;
    A.ops = reinterpret_cast<const qwk::ChainOp*>(ch->mem);
    A.n_ops = n_ops;
    A.M = M;
    A.epoch = reinterpret_cast<unsigned*>(ch->mem + op_bytes);
    A.words = wbase;
    A.n_words = (uint32_t)words;
    A.err = ctx->mlp_ctl + 3;
    for (int s = 0; s < n_slots; ++s) {
        if (!slots[s].init) continue;
        qwk::ChainImport& im = A.imports[A.n_imports++];
        im.words_ptr = wbase + slot_word0[s];
        im.words = slots[s].len / 2;
        im.src = slots[s].init;
        im.ld = slots[s].ld_init ? slots[s].ld_init : slots[s].len;
    }
    if (const char* tp = getenv("QW_CHAIN_TRACE")) {
        // timing probe: [op][4][256] s_memrealtime stamps (input polled, input
        // seen by compute wave 0, its MFMAs done, epilogue issued) of the last
        // launch, dumped to the file at destroy
        if (hipMalloc(&ch->trace, (size_t)n_ops * 4 * 256 * 8) == hipSuccess) {
            hipMemset(ch->trace, 0, (size_t)n_ops * 4 * 256 * 8);
            A.trace = ch->trace;
            ch->trace_path = tp;
        }
    }
    *out = ch;
    return QW_OK;
}

qw_status qw_chain_launch(qw_chain* ch, hipStream_t stream) {
    if (!ch) return QW_ERR_NULL;
    hipError_t e = qwk::launch_chain(ch->args, ch->wf, ch->adt, stream);
    if (e != hipSuccess) return hip_fail(ch->ctx, e, "chain launch");
    return QW_OK;
}

qw_status qw_chain_destroy(qw_chain* ch) {
    if (!ch) return QW_ERR_NULL;
    hipSetDevice(ch->ctx->device);
    hipDeviceSynchronize();
    if (ch->trace) {
        std::vector<uint64_t> h((size_t)ch->args.n_ops * 4 * 256);
        if (hipMemcpy(h.data(), ch->trace, h.size() * 8, hipMemcpyDeviceToHost) == hipSuccess) {
            if (FILE* f = fopen(ch->trace_path.c_str(), "wb")) {
                fwrite(h.data(), 8, h.size(), f);
                fclose(f);
            }
        }
        hipFree(ch->trace);
    }
    hipFree(ch->mem);
    delete ch;
    return QW_OK;
}

// Test hooks: read and/or set the launch epoch of the persistent kernels'
// hand-off words (synchronous; no launch may be in flight on the device).
static qw_status epoch_rw(qw_ctx* ctx, unsigned* word, const unsigned* set, unsigned* get) {
    hipSetDevice(ctx->device);
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess && get) e = hipMemcpy(get, word, sizeof(unsigned), hipMemcpyDeviceToHost);
    if (e == hipSuccess && set) e = hipMemcpy(word, set, sizeof(unsigned), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(ctx, e, "epoch word access");
    return QW_OK;
}

qw_status qw_mlp_stack_epoch(qw_ctx* ctx, const unsigned* set, unsigned* get) {
    if (!ctx) return QW_ERR_NULL;
    return epoch_rw(ctx, ctx->stack_epoch, set, get);
}

qw_status qw_chain_epoch(qw_chain* ch, const unsigned* set, unsigned* get) {
    if (!ch) return QW_ERR_NULL;
    if (set && (*set & ((1u << 22) - 1u)) == 0u) return fail(ch->ctx, QW_ERR_INVALID, "chain epoch: the low 22 bits may not be 0");
    return epoch_rw(ch->ctx, ch->args.epoch, set, get);
}

qw_status qw_device_error(qw_ctx* ctx, int* flag) {
    if (!ctx || !flag) return QW_ERR_NULL;
    unsigned v = 0;
    hipSetDevice(ctx->device);
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(&v, ctx->mlp_ctl + 3, sizeof v, hipMemcpyDeviceToHost);
    if (e == hipSuccess && v) {
        // A one-launch MLP whose bounded wait expired left its down workgroups'
        // exit counts reset while late gate/up workgroups still counted
        // themselves done: with every kernel finished (the synchronize above),
        // return the MLP's counter slots to zero together with the flag, so
        // that the next launch waits for its own gate/up results.
        e = hipMemset(ctx->counters + kMaxCounters, 0, (size_t)kMlpCounterWords * sizeof(unsigned));
        if (e == hipSuccess) e = hipMemset(ctx->mlp_ctl + 3, 0, sizeof(unsigned));
        if (e == hipSuccess) e = hipDeviceSynchronize();
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "reading the device error flag");
    *flag = (int)v;
    return QW_OK;
}

// ---------------------------------------------------------------------------
// norms
// ---------------------------------------------------------------------------

qw_status qw_rmsnorm(qw_ctx* ctx, const void* x, qw_dtype xdt, const float* gamma, float eps, void* y,
                     qw_dtype ydt, int M, int K, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!x || !gamma || !y) return fail(ctx, QW_ERR_NULL, "x, gamma and y are required");
    if (!valid_act(xdt) || !valid_act(ydt)) return fail(ctx, QW_ERR_DTYPE, "dtype unsupported");
    if (M < 1 || K < 1 || K > 4096) return fail(ctx, QW_ERR_SHAPE, "M=%d K=%d (K <= 4096)", M, K);
    if (!(eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "eps must be > 0");
    hipError_t e = qwk::launch_rmsnorm(x, xdt, nullptr, nullptr, gamma, eps, y, ydt, M, K, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "rmsnorm launch");
    return QW_OK;
}

qw_status qw_residual_rmsnorm(qw_ctx* ctx, const void* residual_in, const void* a, qw_dtype dt,
                              void* residual_out, void* normed, qw_dtype normed_dt,
                              const float* gamma, float eps, int M, int K, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!residual_in || !a || !residual_out || !normed || !gamma)
        return fail(ctx, QW_ERR_NULL, "all pointers are required");
    if (!valid_act(dt) || !valid_act(normed_dt)) return fail(ctx, QW_ERR_DTYPE, "dtype unsupported");
    if (M < 1 || K < 1 || K > 4096) return fail(ctx, QW_ERR_SHAPE, "M=%d K=%d (K <= 4096)", M, K);
    if (!(eps > 0.0f)) return fail(ctx, QW_ERR_INVALID, "eps must be > 0");
    hipError_t e = qwk::launch_rmsnorm(residual_in, dt, a, residual_out, gamma, eps, normed,
                                       normed_dt, M, K, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "residual rmsnorm launch");
    return QW_OK;
}

qw_status qw_silu_mul(qw_ctx* ctx, const void* g, const void* u, void* h, qw_dtype dt, int64_t n,
                      hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!g || !u || !h) return fail(ctx, QW_ERR_NULL, "g, u and h are required");
    if (!valid_act(dt)) return fail(ctx, QW_ERR_DTYPE, "dtype unsupported");
    if (n < 1) return fail(ctx, QW_ERR_SHAPE, "n must be >= 1");
    hipError_t e = qwk::launch_silu_mul(g, u, h, dt, n, stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "silu_mul launch");
    return QW_OK;
}

qw_status qw_argmax_rows(qw_ctx* ctx, const void* logits, qw_dtype dt, int M, int V, int ld, int32_t* token_ids,
                         float* max_logit, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    if (!logits || !token_ids) return fail(ctx, QW_ERR_NULL, "logits and token_ids are required");
    if (dt != QW_F32 && dt != QW_BF16 && dt != QW_F16) return fail(ctx, QW_ERR_DTYPE, "logits dtype unsupported");
    if (M < 1 || V < 1) return fail(ctx, QW_ERR_SHAPE, "M and V must be >= 1");
    if (ld == 0) ld = V;
    if (ld < V) return fail(ctx, QW_ERR_SHAPE, "ld must be >= V");
    if (M > kMaxKeys) return fail(ctx, QW_ERR_WORKSPACE, "M=%d exceeds %d argmax slots", M, kMaxKeys);
    hipError_t e = qwk::launch_argmax_rows(logits, (int)dt, M, V, ld, ctx->keys, ctx->done, token_ids, max_logit,
                                           stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "argmax launch");
    return QW_OK;
}

// ---------------------------------------------------------------------------
// graphs
// ---------------------------------------------------------------------------

qw_status qw_graph_begin(qw_ctx* ctx, hipStream_t stream) {
    if (!ctx) return QW_ERR_NULL;
    hipError_t e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamBeginCapture");
    return QW_OK;
}

qw_status qw_graph_end(qw_ctx* ctx, hipStream_t stream, qw_graph** out) {
    if (!ctx || !out) return QW_ERR_NULL;
    *out = nullptr;
    qw_graph* g = new qw_graph();
    hipError_t e = hipStreamEndCapture(stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g->graph) hipGraphDestroy(g->graph);
        delete g;
        return hip_fail(ctx, e, "graph capture");
    }
    *out = g;
    return QW_OK;
}

qw_status qw_graph_launch(qw_graph* g, hipStream_t stream) {
    if (!g) return QW_ERR_NULL;
    return hipGraphLaunch(g->exec, stream) == hipSuccess ? QW_OK : QW_ERR_HIP;
}

qw_status qw_graph_destroy(qw_graph* g) {
    if (!g) return QW_ERR_NULL;
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return QW_OK;
}

}  // extern "C"
