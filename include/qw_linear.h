/*
 * qw_linear.h -- C ABI of the MI355X (gfx950) projection-matmul library.
 *
 * The library replaces the projection/matmul layer of the Qwen3.5-0.8B engine
 * (reference: zhils/Qwen3.5_0.8B_Deploy, src/backend).  Every entry point is
 * plain C: device pointers, sizes, dtype tags and a hipStream_t.  Nothing here
 * allocates on the hot path: scratch (split-K partials, counters, argmax keys,
 * the MLP intermediate) lives in a workspace arena sized at qw_init().
 *
 * Conventions
 *   - Weights are row-major W[N][K] (N = output features, K = input features),
 *     the reference convention (language_mlp.cpp:69-70, lm_head.cpp:30-36).
 *   - Activations are row-major x[M][ldx] with M tokens; outputs y[M][ldy].
 *     ld* of 0 means "packed" (ldx = K, ldy = N).
 *   - y[m][o] = sum_k W[o][k] * x[m][k], FP32 accumulate.
 *   - Calls are asynchronous on the given stream and never synchronize the
 *     host.  One qw_ctx per stream: calls made through one context share its
 *     workspace, so two streams must not use the same context concurrently.
 *   - Errors are returned as qw_status; qw_last_error() gives the message of
 *     the most recent failure on that context.
 */
#ifndef QW_LINEAR_H
#define QW_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QW_ABI_VERSION 1

typedef enum {
    QW_OK = 0,
    QW_ERR_INVALID = 1,   /* bad argument value (flags, eps, ...)            */
    QW_ERR_NULL = 2,      /* required pointer is NULL                        */
    QW_ERR_SHAPE = 3,     /* M/N/K out of range or not a supported multiple  */
    QW_ERR_DTYPE = 4,     /* dtype / weight-format combination unsupported   */
    QW_ERR_ALIGN = 5,     /* pointer or leading dimension misaligned         */
    QW_ERR_WORKSPACE = 6, /* call needs more workspace than qw_init reserved */
    QW_ERR_HIP = 7,       /* a HIP runtime call failed                       */
    QW_ERR_NOMEM = 8,     /* device allocation failed (weight packing)       */
    QW_ERR_STATE = 9      /* call not valid in the current state             */
} qw_status;

typedef enum { QW_F32 = 0, QW_BF16 = 1, QW_F16 = 2, QW_I8 = 3 } qw_dtype;

/* Stored weight formats.  INT8_ROWSCALE is weight-only INT8 with one FP32
 * scale per output row (symmetric, the reference recipe mlp_cuda.cu:22-39). */
typedef enum { QW_WFMT_F32 = 0, QW_WFMT_BF16 = 1, QW_WFMT_INT8_ROWSCALE = 2 } qw_wfmt;

typedef struct qw_ctx qw_ctx;
typedef struct qw_weight qw_weight;
typedef struct qw_graph qw_graph;

/* ---- context -------------------------------------------------------------
 * Replaces the per-operator lazily grown scratch of the reference
 * (CudaMLP::ensure_buffers, mlp_cuda.cu:229-259, and the per-call
 * cudaMalloc/cudaFree of CudaMLP::forward, mlp_cuda.cu:302-303,328-329)
 * with one arena reserved up front.  workspace_bytes = 0 picks the default
 * (qw_workspace_query(4096, 8224, 4096)). */
qw_status qw_init(qw_ctx** ctx, int device, size_t workspace_bytes);
qw_status qw_destroy(qw_ctx* ctx);
/* Workspace needed for calls with up to max_M tokens, max_N output rows
 * (a GLU weight counts its gate+up rows) and max_K inputs. */
size_t qw_workspace_query(int max_M, int max_N, int max_K);
const char* qw_last_error(const qw_ctx* ctx);
const char* qw_status_string(qw_status s);
int qw_abi_version(void);

/* ---- weights ---------------------------------------------------------------
 * Replaces CudaMLP::set_weights (mlp_cuda.cu:261-293: H2D + on-device INT8
 * quantization), CudaLMHead::set_weight (lm_head_cuda.cu:163-187: host
 * FP32->BF16) and the set_weights of the attention operators
 * (linear_attention_cuda.cu:412-466, full_attention_cuda.cu:230-250).
 *
 * `w` is a HOST pointer to W[N][K] in dtype `src` (F32, BF16, F16, or I8 when
 * `scales` gives the per-row FP32 scales of an already quantized matrix).
 * The library re-lays the matrix out in gfx950 MFMA tile order on the device
 * and owns the result.  For dst = INT8_ROWSCALE with a floating source the
 * reference quantization recipe is applied on the device.  K must be a
 * multiple of 64; any N >= 1 is accepted (rows are padded to 16). */
qw_status qw_weight_pack(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N, int K,
                         const float* scales, qw_weight** out);
/* Gate/up pair for the SiLU*mul epilogue: both W[N][K]; packed interleaved so
 * one pass computes silu(gate.x) * (up.x).  Scales as in qw_weight_pack. */
qw_status qw_weight_pack_glu(qw_ctx* ctx, const void* gate, const void* up, qw_dtype src,
                             qw_wfmt dst, int N, int K, const float* gate_scales,
                             const float* up_scales, qw_weight** out);
/* Same as qw_weight_pack / qw_weight_pack_glu with `w`/`gate`/`up` and the
 * optional scales given as DEVICE pointers (weights already resident in HBM,
 * e.g. produced by another loader); nothing is copied through the host. */
qw_status qw_weight_pack_device(qw_ctx* ctx, const void* w, qw_dtype src, qw_wfmt dst, int N,
                                int K, const float* scales, qw_weight** out);
qw_status qw_weight_pack_glu_device(qw_ctx* ctx, const void* gate, const void* up, qw_dtype src,
                                    qw_wfmt dst, int N, int K, const float* gate_scales,
                                    const float* up_scales, qw_weight** out);
/* Several projections of the same input stacked into one weight: part i
 * (W_i[N_i][K], host or device source, optional per-row INT8 scales) takes
 * output rows [N_0 + ... + N_{i-1}, +N_i) of W[sum N_i][K].  One qw_linear
 * then computes all parts in one launch (e.g. the Gated-DeltaNet in_proj_qkv,
 * in_proj_z, in_proj_a and in_proj_b of language_linear_attn.cpp:136-168, or
 * the full-attention q/k/v projections of language_full_attn.cpp:127-156);
 * the caller reads part i at column offset N_0 + ... + N_{i-1} of y.  Every
 * part but the last must have a multiple of 16 rows. */
qw_status qw_weight_pack_concat(qw_ctx* ctx, int parts, const void* const* ws, const int* Ns, qw_dtype src,
                                qw_wfmt dst, int K, const float* const* scales, qw_weight** out);
qw_status qw_weight_pack_concat_device(qw_ctx* ctx, int parts, const void* const* ws, const int* Ns, qw_dtype src,
                                       qw_wfmt dst, int K, const float* const* scales, qw_weight** out);
/* Borrow: build a weight object over device memory already in packed order
 * (e.g. a tied embedding shared with the lm_head, as
 * CudaLMHead::set_weight_bf16_ptr borrows, lm_head_cuda.cu:189-196).  The
 * caller keeps ownership of `packed` and `scales`. */
qw_status qw_weight_wrap_packed(qw_ctx* ctx, void* packed, float* scales, qw_wfmt fmt, int N,
                                int K, qw_weight** out);
/* Fold an RMSNorm weight into a BF16 or F32 weight: W[o][k] *= (1 + gamma[k])
 * (device gamma[K], asynchronous on `stream`).  Afterwards the weight is used
 * with QW_EP_NORM_X and gamma = NULL (qw_mlp_fused: gamma = NULL, the norm is
 * implied), and the kernels only scale by 1/rms(x): no per-call gamma
 * traffic.  Same math as RMSNorm(x)*(1+gamma) followed by the projection
 * (rounding moves from the activation to the weight).  No reference
 * counterpart: the reference applies the norm weight to the activation
 * (language_common.cpp:21-36) before the MLP (language_mlp.cpp:53-91).
 * INT8 weights are refused (QW_ERR_DTYPE): folding would change their
 * quantization. */
qw_status qw_weight_fold_norm(qw_ctx* ctx, qw_weight* w, const float* gamma, hipStream_t stream);
qw_status qw_weight_free(qw_weight* w);
/* Size, shape and format of a packed weight (any out pointer may be NULL). */
qw_status qw_weight_info(const qw_weight* w, int* N, int* K, qw_wfmt* fmt, int* is_glu,
                         size_t* packed_bytes);
/* Device pointers of the packed data and of the per-row scales (NULL for
 * non-INT8 formats). */
qw_status qw_weight_device_ptrs(const qw_weight* w, const void** packed, const float** scales);
/* Copy the stored values back to the host in row-major order: dst receives
 * W[N][K] in the stored dtype (F32, BF16 bits, or INT8) and, for INT8,
 * scales_dst receives N scales.  For a GLU weight, rows [0,N) are the gate
 * and [N,2N) the up projection.  Synchronous; used by tests and tools. */
qw_status qw_weight_unpack(qw_ctx* ctx, const qw_weight* w, void* dst, float* scales_dst);

/* ---- epilogue --------------------------------------------------------------
 * Fusions available on qw_linear / qw_gemm. */
enum {
    QW_EP_RESIDUAL = 1u << 0, /* y = acc + residual[m][o] (residual may alias y) */
    QW_EP_NORM_X = 1u << 1,   /* x := RMSNorm(x)*(1+gamma) before the product
                                 (gamma NULL: weight folded, qw_weight_fold_norm) */
    QW_EP_SPLIT = 1u << 2     /* rows alternate in blocks of split_period between
                                 y and y2 (full-attention Q / output gate) */
};

typedef struct {
    unsigned flags;
    const void* residual;   /* QW_EP_RESIDUAL: [M][ld_residual]                */
    qw_dtype residual_dtype;
    int ld_residual;        /* 0 = N                                           */
    const float* gamma;     /* QW_EP_NORM_X: [K] RMSNorm weight, (1+gamma) form */
    float eps;              /* QW_EP_NORM_X epsilon (reference: 1e-6)           */
    int split_period;       /* QW_EP_SPLIT: block length (power of two >= 16)   */
    void* y2;               /* QW_EP_SPLIT: second output [M][ldy]              */
} qw_epilogue;

/* ---- projections -------------------------------------------------------------
 * y = W.x with the epilogue.  A GLU weight yields y[m][o] = silu(g)*u for its
 * N logical rows.  Replaces launch_cutlass_gemv[_bf16|_fused_silu]
 * (cutlass_gemm_wrapper.cuh:202-263), the INT8 GEMV of CudaMLP
 * (mlp_cuda.cu:158-180), the projection kernels of the attention operators
 * (linear_attention_cuda.cu:33-45,174-187; full_attention_cuda.cu:31-76,
 * 78-148,161-172), cublas_sgemm[_add_residual] (cublas_utils.cuh:48-93) and
 * bf16_gemv[_add] (bf16_gemm.cuh:82-122).  Picks the skinny MFMA kernel for
 * small M and the LDS-tiled MFMA GEMM for large M.
 * Supported x dtypes: F32 (any weight), BF16 (BF16/INT8 weights), F16
 * (BF16/INT8 weights).  y dtype: F32, BF16 or F16. */
qw_status qw_linear(qw_ctx* ctx, const qw_weight* W, const void* x, qw_dtype xdt, int ldx, int M,
                    void* y, qw_dtype ydt, int ldy, const qw_epilogue* ep, hipStream_t stream);

/* ---- fused MLP ---------------------------------------------------------------
 * y = [residual +] down( silu(gate.xn) * up.xn ),  xn = gamma ? RMSNorm(x) : x.
 * Replaces CudaMLP::forward / forward_add_residual (mlp_cuda.cu:295-337; the
 * residual is ADDED, unlike mlp_cuda.cu:332-337) and the fused post-norm +
 * MLP + residual of fusion_microbench_kernels.cu:583-609.  `gateup` must be a
 * GLU weight [I][H], `down` a weight [H][I].  residual may alias y. */
qw_status qw_mlp_fused(qw_ctx* ctx, const qw_weight* gateup, const qw_weight* down, const void* x,
                       qw_dtype xdt, const float* gamma, float eps, const void* residual,
                       qw_dtype residual_dtype, void* y, qw_dtype ydt, int M, hipStream_t stream);

/* The tail of a decoder layer: the out-projection with its residual, then
 * the post-norm MLP with its residual, on the FP32 residual stream x [M][H]:
 *     x = x + W_out . core;   x = x + down(silu(gate.n(x)) * up.n(x)),
 *     n(x) = RMSNorm(x) * (1 + gamma)   (gamma NULL: the norm folded into gateup)
 * core [M][>= K_out] (row stride ld_core, 0 = K_out) in the MFMA input type
 * (BF16).  The equivalent of qw_linear(W_out, core, residual = x, y = x)
 * followed by qw_mlp_fused(x, gamma, residual = x, y = x), which is what it
 * runs by default.  With QW_LAYER_TAIL=1 in the environment of qw_init, at
 * decode sizes (M <= 4, BF16 or INT8 weights, W_out [H][<= 2048]) it runs as
 * one launch in which the first gate/up workgroups compute the out-projection
 * and hand x_mid to the rest (same results within rounding; measured ~0.7 us
 * per layer slower than the two launches in a replayed decode graph).  Replaces the out-projection + post_norm forward_with_residual + MLP
 * forward_add_residual steps of CudaLayer::forward (cuda_engine.cu:118-124,
 * with the out-projections of linear_attention_cuda.cu:174-187 and
 * full_attention_cuda.cu:708-714). */
qw_status qw_layer_tail(qw_ctx* ctx, const qw_weight* w_out, const void* core, qw_dtype core_dtype, int ld_core,
                        const qw_weight* gateup, const qw_weight* down, const float* gamma, float eps, float* x,
                        int M, hipStream_t stream);

/* L consecutive MLP blocks: for l < L, x = x + down_l(silu(gate_l.n_l(x)) *
 * (up_l.n_l(x))) with n_l(x) = RMSNorm(x) * (1 + gamma[l]) (eps), x rounded
 * to xdt after every block; x [M][1024] in, y [M][1024] out (y may alias x).
 * The chain of CudaLayer::forward's post-norm + MLP + residual steps
 * (cuda_engine.cu:119-124) over consecutive layers, i.e. L calls of
 * qw_mlp_fused(x, gamma[l], residual = x, y), equal to them within FP32
 * summation order.  gamma NULL (or all entries NULL): every gateup weight
 * carries its norm weight (qw_weight_fold_norm).  At decode (M <= 8, BF16
 * weights with BF16 x or INT8 weights with F16 x, the Qwen3.5-0.8B shape
 * H = 1024, I = 3584, a device with >= 256 CUs, L <= 48) all blocks run in
 * ONE persistent launch that streams block l+1's weights while block l's
 * data hand-offs are in flight; otherwise it makes the L qw_mlp_fused calls
 * (QW_MLP_STACK=0 forces those).  The persistent launch needs the GPU to
 * itself (its 256 workgroups must all be resident); a hand-off that does not
 * arrive within 0.2 s raises the device error flag instead of hanging. */
qw_status qw_mlp_stack(qw_ctx* ctx, int L, const qw_weight* const* gateup, const qw_weight* const* down,
                       const float* const* gamma, float eps, const void* x, qw_dtype xdt, void* y, int M,
                       hipStream_t stream);

/* ---- a chain of dependent projections in one launch (decode) -----------------
 * The projection sequence of a decoder layer between its attention /
 * Gated-DeltaNet cores (CudaLayer::forward, cuda_engine.cu:105-124: the input
 * and output projections of CudaLinearAttention / CudaFullAttention,
 * linear_attention_cuda.cu:174-187, full_attention_cuda.cu:451-600, and
 * CudaMLP::forward_add_residual, mlp_cuda.cu:295-337), over several layers,
 * at M <= 2 decode tokens, as ONE persistent launch.  Activations live in
 * "slots" (vectors of `len` 16-bit values per token, BF16 for BF16 weights,
 * F16 for INT8 weights); op i computes
 *     slot[out][m][n] = epi( sum_k W[n][k] * pre(slot[in][m][in_offset + k]) )
 * with pre = RMSNorm(.) * (1 + gamma) over the K inputs (norm = 1; gamma
 * NULL when the weight carries it), epi = SiLU(gate)*up for GLU weights,
 * + the slot's previous value (residual = 1), the result rounded to the
 * slot's type -- the result of the same qw_linear calls with 16-bit outputs,
 * within FP32 summation order.  Every op must read the previous op's output
 * slot (op 0: a slot with `init`), never its own output slot, and K <= 3584;
 * at most 128 ops per chain.
 * The plan (op table, slot storage) is built once on the device by
 * qw_chain_create and replayed by qw_chain_launch (capture-safe: no memset, no
 * allocation).  It needs the GPU to itself (its 256 workgroups of 1024 threads
 * must all be resident); a hand-off that does not arrive within 0.2 s raises
 * the device error flag instead of hanging.  No counterpart class in the
 * reference: its decode runs these projections as separate kernel launches. */
typedef struct qw_chain qw_chain;
typedef struct qw_chain_slot {
    int len;           /* values per token (a multiple of 16) */
    const void* init;  /* device [M][ld_init] values imported at launch start, or NULL */
    int ld_init;       /* 0: len */
    void* out;         /* device [M][ld_out]: ops writing the slot also store their rows here, or NULL */
    int ld_out;        /* 0: len */
} qw_chain_slot;
typedef struct qw_chain_op {
    const qw_weight* w;  /* BF16 or INT8 (one format per chain); GLU allowed */
    int in;              /* input slot */
    int in_offset;       /* first input element (a multiple of 64) */
    int out;             /* output slot (not `in`) */
    int residual;        /* 1: add the output slot's previous values */
    int norm;            /* 1: RMSNorm prologue on the input */
    const float* gamma;  /* its weight [K], or NULL when folded into w */
    float eps;
} qw_chain_op;
qw_status qw_chain_create(qw_ctx* ctx, qw_dtype act_dtype, int M, int n_slots, const qw_chain_slot* slots,
                          int n_ops, const qw_chain_op* ops, qw_chain** out);
qw_status qw_chain_launch(qw_chain* chain, hipStream_t stream);
qw_status qw_chain_destroy(qw_chain* chain);

/* Test hooks of the two persistent kernels above (no counterpart in the
 * reference): read (*get) and/or set (*set) the launch epoch whose low bits
 * tag their hand-off words -- 26 bits for qw_mlp_stack, 22 for a chain (whose
 * low 22 bits may not be 0).  The epoch advances once per launch; the launch
 * at which the tag's field wraps clears the words first, so a word written
 * 2^26 (2^22) launches earlier never matches.  Setting the epoch just below
 * the wrap lets a test run launches across it.  Synchronizes the device. */
qw_status qw_mlp_stack_epoch(qw_ctx* ctx, const unsigned* set, unsigned* get);
qw_status qw_chain_epoch(qw_chain* chain, const unsigned* set, unsigned* get);

/* Reads and clears the context's device error flag: non-zero when a kernel
 * gave up a bounded wait (a fused MLP down task whose gate/up inputs never
 * completed within 0.2 s), when an attention token fell outside its cache, or
 * when an embedding id was outside the vocabulary; the outputs of that call
 * are then invalid.  Synchronizes the device; when the flag was set it also
 * returns the fused MLP's completion counters to zero, so later launches on
 * the context are valid again.  The eager and graph-replayed decode steps do
 * not read the flag themselves: callers check it after a step (engine.py's
 * DecodeEngine does, see check()). */
qw_status qw_device_error(qw_ctx* ctx, int* flag);

/* ---- gated full attention (between the projections) -------------------------
 * One call runs, for `tokens` new tokens of each of `batch` sequences (row
 * b*tokens + t is token t of sequence b, at cache position positions[b] + t):
 *   q_h = RMSNorm(q_h) * (1 + q_norm_weight), k_g likewise (eps 1e-6, per head);
 *   RoPE on the first rotary_dim dims (interleaved pairs (d, d+1), angle
 *   position / rope_theta^(d / rotary_dim)) of q and k;
 *   the K/V cache write at that position;
 *   o_h = softmax(q_h . K_g^T / sqrt(head_dim)) V_g over positions
 *   0 .. position (causal), g = h / (num_heads / num_kv_heads);
 *   out = o * sigmoid(gate).
 * Replaces the attention core of FullAttention::forward
 * (language_full_attn.cpp:117-216) and of CudaFullAttention::forward /
 * forward_batch_prefill (fused_q_path_kernel, fused_kv_cache_int8_kernel,
 * flash attention, gate_sigmoid_kernel: full_attention_cuda.cu:31-166,
 * 353-449, 640-714).  Differences from that CUDA chain, both deliberate: the
 * INT8 cache is read back with each token's own scale (its dequant kernels
 * index the scale by head only, fused_kernels.cu:400-412), and a batch of
 * tokens attends causally (its prefill attends to every cached position up to
 * the batch's maximum, fused_kernels.cu:175-200); both follow the CPU operator.
 * Inputs (in_dtype F32, BF16 or F16, row stride ld_in elements): q and gate,
 * element (row r, head h, dim d) at r*ld_in + h*q_head_stride + d (512 for the
 * interleaved Q|gate projection output with gate = q + 256, 256 for split
 * buffers); k and v at r*ld_in + g*head_dim + d.  positions: device int
 * [batch].  max_len: an upper bound of positions[b] + tokens used to size the
 * launch (0: the cache capacity).  A token whose position falls outside the
 * cache writes nothing, outputs zeros and sets the device error flag
 * (qw_device_error).  head_dim 128 or 256, num_heads / num_kv_heads <= 4. */
typedef struct {
    int num_heads;              /* query heads (8) */
    int num_kv_heads;           /* key/value heads (2) */
    int head_dim;               /* q and kv head dim (256) */
    int rotary_dim;             /* leading dims rotated (64 = head_dim * 0.25) */
    float rope_theta;           /* 1e7 */
    const float* q_norm_weight; /* [head_dim], device */
    const float* k_norm_weight; /* [head_dim], device */
} qw_attn_params;

/* KV cache of one layer, the CudaKVCache layout (full_attention_cuda.hpp:
 * 11-33) with a sequence dimension: k, v [sequences][capacity][num_kv_heads]
 * [head_dim] of dtype QW_I8 (symmetric, one FP32 scale per token and KV head
 * in k_scale / v_scale [sequences][capacity][num_kv_heads]) or QW_F32 (the CPU
 * KVCache, language_full_attn.hpp:8-54; scales unused). */
typedef struct {
    qw_dtype dtype;
    void* k;
    void* v;
    float* k_scale;
    float* v_scale;
    int capacity;  /* tokens per sequence */
} qw_kv_cache;

qw_status qw_attn_forward(qw_ctx* ctx, const qw_attn_params* p, const qw_kv_cache* cache, int batch, int tokens,
                          const int* positions, int max_len, const void* q, const void* gate, int q_head_stride,
                          const void* k, const void* v, qw_dtype in_dtype, int ld_in, void* out,
                          qw_dtype out_dtype, int ld_out, hipStream_t stream);

/* ---- token embedding and decode-step bookkeeping ----------------------------
 * out[m][0..hidden) = table[ids[m]][0..hidden) (table row-major [vocab][hidden],
 * F32 or BF16; out F32, BF16 or F16 with row stride ld_out, 0 = hidden; ids
 * device int32 [M]).  Replaces TokenEmbedding::forward / CudaTokenEmbedding
 * (token_embedding_cuda.cu:28-58, the BF16 table of the tied embedding).  An
 * id outside [0, vocab) gives a zero row and sets the device error flag.
 * hidden must be a multiple of 4. */
qw_status qw_embedding_gather(qw_ctx* ctx, const void* table, qw_dtype table_dtype, int vocab, int hidden,
                              const int32_t* ids, int M, void* out, qw_dtype out_dtype, int ld_out,
                              hipStream_t stream);
/* positions[i] += delta for i < n (device int32), as a kernel, so that a
 * captured decode step advances its own cache positions on every replay.  No
 * counterpart in the reference, whose engine passes the position from the
 * host each step (cuda_engine.cu:308-325). */
qw_status qw_positions_add(qw_ctx* ctx, int32_t* positions, int n, int delta, hipStream_t stream);

/* ---- lm_head + greedy argmax -------------------------------------------------
 * token_ids[m] = argmax_v sum_k E[v][k]*h[m][k]; ties go to the LOWEST index
 * (std::max_element, sampler.cpp:41-43).  max_logit (optional) receives the
 * winning logit.  Replaces CudaLMHead::forward (lm_head_cuda.cu:198-210) +
 * GpuGreedyArgmaxSampler::sample (gpu_sampler_argmax.cu:69-93) with one launch
 * and no host round trip. */
qw_status qw_lmhead_argmax(qw_ctx* ctx, const qw_weight* E, const void* h, qw_dtype hdt, int M,
                           int32_t* token_ids, float* max_logit, hipStream_t stream);

/* The same lm_head + greedy argmax for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): no qw_ctx and no workspace.  No counterpart in the
 * reference.  E is given by the device pointers of an already packed weight
 * (qw_weight_device_ptrs of a qw_weight_pack result, or any buffer in that
 * packed order; E_scales for INT8_ROWSCALE, else NULL) with its V rows and
 * K inputs.  The argmax keys live in a fixed per-device array inside the
 * library (2.3 KB, held until the process ends), so M is at most 256
 * (QW_ERR_SHAPE beyond).  Runs on the current device with the kernels and
 * routes of qw_lmhead_argmax on a default context, so its results equal that
 * entry point's bit for bit on a context created without QW_* routing
 * overrides in the environment (this entry point always takes the default
 * routes and ignores those variables).  Calls that overlap on one device share the
 * array and race: serialize them (one stream, or events).  Errors are
 * status codes only (there is no context for qw_last_error). */
qw_status qw_lmhead_argmax_noalloc(const void* E_packed, const float* E_scales, qw_wfmt fmt, int V, int K,
                                   const void* h, qw_dtype hdt, int M, int32_t* token_ids, float* max_logit,
                                   hipStream_t stream);

/* Greedy argmax of materialized logits [M][ld] (F32, BF16 or F16):
 * token_ids[m] = lowest index of the row maximum.  Replaces
 * GpuGreedyArgmaxSampler::sample (gpu_sampler_argmax.cu:69-93: block argmax +
 * D2H + host scan) with one launch and no host round trip; for the lm_head
 * prefer qw_lmhead_argmax, which never writes the logits.  ld 0 = V. */
qw_status qw_argmax_rows(qw_ctx* ctx, const void* logits, qw_dtype dt, int M, int V, int ld,
                         int32_t* token_ids, float* max_logit, hipStream_t stream);

/* ---- RMSNorm -----------------------------------------------------------------
 * y = x / sqrt(mean(x^2) + eps) * (1 + gamma)  (language_common.cpp:21-78,
 * CudaRMSNorm::forward rmsnorm_cuda.cu:350-368). */
qw_status qw_rmsnorm(qw_ctx* ctx, const void* x, qw_dtype xdt, const float* gamma, float eps,
                     void* y, qw_dtype ydt, int M, int K, hipStream_t stream);
/* residual_out = residual_in + a;  normed = RMSNorm(residual_out)
 * (CudaRMSNorm::forward_with_residual rmsnorm_cuda.cu:370-394,
 * launch_fused_rmsnorm_residual fused_kernels.cuh:9-18).  residual_out may
 * alias residual_in. */
qw_status qw_residual_rmsnorm(qw_ctx* ctx, const void* residual_in, const void* a, qw_dtype dt,
                              void* residual_out, void* normed, qw_dtype normed_dt,
                              const float* gamma, float eps, int M, int K, hipStream_t stream);
/* h[i] = silu(g[i]) * u[i] for n elements (launch_silu_mul_batch,
 * fused_kernels.cuh:29-34); all three in dtype dt. */
qw_status qw_silu_mul(qw_ctx* ctx, const void* g, const void* u, void* h, qw_dtype dt, int64_t n,
                      hipStream_t stream);

/* ---- Gated-DeltaNet decode step ---------------------------------------------------
 * Everything between the input projections and the out projection of a
 * linear-attention layer, one token for each of `batch` sequences:
 * causal conv1d (+SiLU) over the QKV channels with the conv-state shift,
 * per-head L2 norm of q (times 1/sqrt(key_dim)) and k, beta = sigmoid(b),
 * g = -exp(A_log) * softplus(a + dt_bias), the delta rule on the FP32
 * recurrent state (S *= exp(g); S += beta * k (v - S^T k)^T; o = S^T q), and
 * the per-head RMSNorm (eps 1e-6) times norm_weight times SiLU(z).
 * Replaces the core of LinearAttention::forward (language_linear_attn.cpp:
 * 143-256) and the kernel chain of CudaLinearAttention::forward
 * (conv1d_update_fused / l2norm_qk_fused / gated_delta / norm_gate_fused,
 * linear_attention_cuda.cu:47-172, launched at :486-530).
 * Inputs, one row per sequence with stride ld_in elements (typically the rows
 * of one stacked [QKV | Z | a | b] projection output): mixed_qkv
 * [2*nh*kd + nh*vd] (all q, then all k, then all v), z [nh*vd], a [nh],
 * b [nh], all in in_dtype (F32, BF16 or F16).  Parameters (FP32, device):
 * conv_weight [conv_dim][conv_kernel], A_log [nh], dt_bias [nh],
 * norm_weight [vd].  States (FP32, device, updated in place, the reference
 * layouts): conv_state [batch][conv_dim][conv_kernel-1] (index 0 the newest
 * input; may be NULL when conv_kernel is 1), recurrent_state
 * [batch][nh][kd][vd].  out [batch][ld_out] receives nh*vd values.  key_dim = value_dim = 128, 1 <= conv_kernel <= 8. */
typedef struct {
    int num_heads;
    int key_dim;
    int value_dim;
    int conv_kernel;
    const float* conv_weight;
    const float* A_log;
    const float* dt_bias;
    const float* norm_weight;
} qw_gdn_params;
qw_status qw_gdn_decode(qw_ctx* ctx, const qw_gdn_params* p, int batch, const void* mixed_qkv,
                        const void* z, const void* a, const void* b, qw_dtype in_dtype, int ld_in,
                        float* conv_state, float* recurrent_state, void* out, qw_dtype out_dtype,
                        int ld_out, hipStream_t stream);
/* The same step over `tokens` consecutive tokens of each of `batch`
 * sequences, serially in token order: input and output row b*tokens + t
 * holds token t of sequence b; the states carry from one token to the next
 * and hold the state after the last token on return.  Equal to `tokens`
 * calls of qw_gdn_decode, in one launch that reads and writes each state
 * once.  Replaces the state chain of CudaLinearAttention::forward_batch
 * (linear_attention_cuda.cu:529-680; its contract, equality with serial
 * single-token steps, is verify_linear_attn_batch.cu:68-112) and
 * LinearAttention::forward over several tokens (language_linear_attn.cpp:
 * 125-257). */
qw_status qw_gdn_prefill(qw_ctx* ctx, const qw_gdn_params* p, int batch, int tokens, const void* mixed_qkv,
                         const void* z, const void* a, const void* b, qw_dtype in_dtype, int ld_in,
                         float* conv_state, float* recurrent_state, void* out, qw_dtype out_dtype, int ld_out,
                         hipStream_t stream);

/* ---- graphs --------------------------------------------------------------------
 * Capture a sequence of qw_* calls on `stream` into a replayable HIP graph
 * (the role of cudaStreamBeginCapture/cudaGraphLaunch in
 * CudaEngine::forward_batch_prefill_graph, cuda_engine.cu:454-477).  The qw_*
 * calls issue no memset and no allocation, so they are capture-safe. */
qw_status qw_graph_begin(qw_ctx* ctx, hipStream_t stream);
qw_status qw_graph_end(qw_ctx* ctx, hipStream_t stream, qw_graph** out);
qw_status qw_graph_launch(qw_graph* g, hipStream_t stream);
qw_status qw_graph_destroy(qw_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* QW_LINEAR_H */
