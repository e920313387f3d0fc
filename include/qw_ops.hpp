// qw_ops.hpp -- C++ operator facade over the C ABI (qw_linear.h), shaped like
// the reference engine's projection operators so that a caller written
// against them (CudaLayer::forward, cuda_engine.cu:109-125) switches by
// changing the class names.  Header-only; links against libqw_linear.so.
//
// Reference classes mirrored (zhils/Qwen3.5_0.8B_Deploy, src/backend/cuda/include):
//   qwen::cuda::CudaMLP                 mlp_cuda.hpp:11-59       -> qwen::hip::HipMLP
//   qwen::cuda::CudaLMHead              lm_head_cuda.hpp:10-38   -> qwen::hip::HipLMHead
//   qwen::cuda::GpuGreedyArgmaxSampler  gpu_sampler_argmax.hpp:6-20 -> qwen::hip::HipGreedyArgmaxSampler
//   qwen::cuda::CudaRMSNorm             rmsnorm_cuda.hpp:9-29    -> qwen::hip::HipRMSNorm
//   projection parts of CudaLinearAttention (linear_attention_cuda.hpp:24-90) and
//   CudaFullAttention (full_attention_cuda.hpp:35-90)
//                                       -> HipLinearAttnProjections / HipFullAttnProjections
//   qwen::cuda::CudaLinearAttention / CudaLinearAttnState (whole decode layer,
//   linear_attention_cuda.hpp:11-90)   -> HipLinearAttention / HipLinearAttnState
//   qwen::cuda::CudaFullAttention / CudaKVCache (whole layer,
//   full_attention_cuda.hpp:11-90)     -> HipFullAttention / HipKVCache
//   qwen::cuda::CudaEngine (whole model, one sequence,
//   cuda_engine.hpp:85-133)            -> HipEngine
//
// Same argument meaning as the reference: weights arrive as host
// std::vector<float> in row-major [out][in]; activations are caller-owned
// device pointers (FP32); batch = number of tokens.  Differences:
//   - every call takes an optional hipStream_t (the reference uses stream 0);
//   - forward_add_residual ADDS the MLP output to the residual (the INT8
//     CudaMLP overwrites it, mlp_cuda.cu:332-337);
//   - errors throw qwen::hip::Error carrying the library's status and message
//     (the reference mixes exceptions, printf and exit).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qw_linear.h"

namespace qwen {
namespace hip {

class Error : public std::runtime_error {
  public:
    Error(qw_status s, const std::string& what) : std::runtime_error(what), status(s) {}
    qw_status status;
};

// One library context (workspace arena) per device, shared by the operators
// created on it; use one Context per stream when streams run concurrently.
class Context {
  public:
    explicit Context(int device = 0, size_t workspace_bytes = 0) {
        check(qw_init(&ctx_, device, workspace_bytes), "qw_init");
    }
    ~Context() { qw_destroy(ctx_); }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    qw_ctx* get() const { return ctx_; }

    void check(qw_status s, const char* what) const {
        if (s != QW_OK) {
            std::string msg = std::string(what) + ": " + qw_status_string(s);
            if (ctx_) msg += std::string(" (") + qw_last_error(ctx_) + ")";
            throw Error(s, msg);
        }
    }

    // process-wide default context of the current device
    static std::shared_ptr<Context> default_for_current_device() {
        static std::shared_ptr<Context> per_device[64];
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) throw Error(QW_ERR_HIP, "hipGetDevice");
        if (!per_device[dev]) per_device[dev] = std::make_shared<Context>(dev);
        return per_device[dev];
    }

  private:
    qw_ctx* ctx_ = nullptr;
};

namespace detail {
struct WeightDeleter {
    void operator()(qw_weight* w) const { qw_weight_free(w); }
};
using WeightPtr = std::unique_ptr<qw_weight, WeightDeleter>;

inline WeightPtr pack(const Context& c, const std::vector<float>& w, int N, int K, qw_wfmt fmt, const char* name) {
    if ((int64_t)w.size() != (int64_t)N * K)
        throw Error(QW_ERR_SHAPE, std::string(name) + ": expected " + std::to_string((int64_t)N * K) + " floats");
    qw_weight* out = nullptr;
    c.check(qw_weight_pack(c.get(), w.data(), QW_F32, fmt, N, K, nullptr, &out), name);
    return WeightPtr(out);
}

inline void require(const void* p, const char* what) {
    if (!p) throw Error(QW_ERR_STATE, std::string(what) + ": weights not set");
}
}  // namespace detail

// ---------------------------------------------------------------------------
// MLP: y = down(silu(gate.x) * up.x).  Default storage is INT8 with per-row
// scales (the reference CudaMLP quantizes in set_weights, mlp_cuda.cu:261-293);
// pass QW_WFMT_BF16 or QW_WFMT_F32 for the other formats.
class HipMLP {
  public:
    explicit HipMLP(int hidden_size = 1024, int intermediate_size = 3584,
                    qw_wfmt format = QW_WFMT_INT8_ROWSCALE,
                    std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden_size), inter_(intermediate_size), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {}

    void set_weights(const std::vector<float>& gate_proj_weight, const std::vector<float>& up_proj_weight,
                     const std::vector<float>& down_proj_weight) {
        const int64_t n = (int64_t)inter_ * hidden_;
        if ((int64_t)gate_proj_weight.size() != n || (int64_t)up_proj_weight.size() != n)
            throw Error(QW_ERR_SHAPE, "HipMLP::set_weights: gate/up must be [intermediate][hidden]");
        qw_weight* gu = nullptr;
        ctx_->check(qw_weight_pack_glu(ctx_->get(), gate_proj_weight.data(), up_proj_weight.data(), QW_F32, fmt_,
                                       inter_, hidden_, nullptr, nullptr, &gu),
                    "HipMLP::set_weights gate/up");
        gateup_.reset(gu);
        down_ = detail::pack(*ctx_, down_proj_weight, hidden_, inter_, fmt_, "HipMLP::set_weights down");
    }

    void forward(const float* input, float* output, int batch_size = 1, hipStream_t stream = nullptr) const {
        detail::require(down_.get(), "HipMLP::forward");
        ctx_->check(qw_mlp_fused(ctx_->get(), gateup_.get(), down_.get(), input, QW_F32, nullptr, 1e-6f, nullptr,
                                 QW_F32, output, QW_F32, batch_size, stream),
                    "HipMLP::forward");
    }

    // residual[b] += MLP(input[b])
    void forward_add_residual(const float* input, float* residual, int batch_size = 1,
                              hipStream_t stream = nullptr) const {
        detail::require(down_.get(), "HipMLP::forward_add_residual");
        ctx_->check(qw_mlp_fused(ctx_->get(), gateup_.get(), down_.get(), input, QW_F32, nullptr, 1e-6f, residual,
                                 QW_F32, residual, QW_F32, batch_size, stream),
                    "HipMLP::forward_add_residual");
    }

    // residual[b] += MLP(RMSNorm(residual[b]) * (1 + gamma)): the post-attention
    // norm, MLP and residual of one layer in two launches.
    void forward_norm_add_residual(const float* gamma, float eps, float* residual, int batch_size = 1,
                                   hipStream_t stream = nullptr) const {
        detail::require(down_.get(), "HipMLP::forward_norm_add_residual");
        ctx_->check(qw_mlp_fused(ctx_->get(), gateup_.get(), down_.get(), residual, QW_F32, gamma, eps, residual,
                                 QW_F32, residual, QW_F32, batch_size, stream),
                    "HipMLP::forward_norm_add_residual");
    }

    int hidden_size() const { return hidden_; }

  private:
    int hidden_, inter_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr gateup_, down_;
};

// ---------------------------------------------------------------------------
// lm_head over the tied embedding E[vocab][hidden], stored BF16 (as
// CudaLMHead::set_weight converts, lm_head_cuda.cu:163-187) or INT8.
class HipLMHead {
  public:
    explicit HipLMHead(int hidden_size = 1024, int vocab_size = 248320, qw_wfmt format = QW_WFMT_BF16,
                       std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden_size), vocab_(vocab_size), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {}

    void set_weight(const std::vector<float>& weight) {
        E_ = detail::pack(*ctx_, weight, vocab_, hidden_, fmt_, "HipLMHead::set_weight");
    }

    // A resident row-major BF16 embedding (the tied token embedding).  The
    // reference borrows it (lm_head_cuda.cu:189-196); the packed tile order
    // needs its own copy, made on the device without a host round trip.
    void set_weight_bf16_ptr(const void* d_weight_bf16) {
        qw_weight* out = nullptr;
        ctx_->check(qw_weight_pack_device(ctx_->get(), d_weight_bf16, QW_BF16, fmt_, vocab_, hidden_, nullptr, &out),
                    "HipLMHead::set_weight_bf16_ptr");
        E_.reset(out);
    }

    // logits[b][v] = E[v] . input[b]  (FP32 logits, as the reference writes)
    void forward(const float* input, float* output, int batch_size = 1, hipStream_t stream = nullptr) const {
        detail::require(E_.get(), "HipLMHead::forward");
        ctx_->check(qw_linear(ctx_->get(), E_.get(), input, QW_F32, 0, batch_size, output, QW_F32, 0, nullptr, stream),
                    "HipLMHead::forward");
    }

    // token_ids[b] = argmax_v logits[b][v] without writing the logits
    void forward_argmax(const float* input, int32_t* d_token_ids, int batch_size = 1, float* d_max_logit = nullptr,
                        hipStream_t stream = nullptr) const {
        detail::require(E_.get(), "HipLMHead::forward_argmax");
        ctx_->check(qw_lmhead_argmax(ctx_->get(), E_.get(), input, QW_F32, batch_size, d_token_ids, d_max_logit,
                                     stream),
                    "HipLMHead::forward_argmax");
    }

    int hidden_size() const { return hidden_; }
    int vocab_size() const { return vocab_; }

  private:
    int hidden_, vocab_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr E_;
};

// ---------------------------------------------------------------------------
// Greedy sampler over materialized FP32 logits: returns the lowest index of
// the maximum (synchronous, like the reference's sample()).
class HipGreedyArgmaxSampler {
  public:
    explicit HipGreedyArgmaxSampler(int vocab_size, std::shared_ptr<Context> ctx = nullptr)
        : vocab_(vocab_size), ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {
        if (hipMalloc(&d_id_, sizeof(int32_t)) != hipSuccess) throw Error(QW_ERR_NOMEM, "HipGreedyArgmaxSampler");
    }
    ~HipGreedyArgmaxSampler() { (void)hipFree(d_id_); }
    HipGreedyArgmaxSampler(const HipGreedyArgmaxSampler&) = delete;
    HipGreedyArgmaxSampler& operator=(const HipGreedyArgmaxSampler&) = delete;

    int sample(const float* d_logits, hipStream_t stream = nullptr) {
        ctx_->check(qw_argmax_rows(ctx_->get(), d_logits, QW_F32, 1, vocab_, 0, d_id_, nullptr, stream),
                    "HipGreedyArgmaxSampler::sample");
        int32_t id = -1;
        if (hipMemcpyAsync(&id, d_id_, sizeof(id), hipMemcpyDeviceToHost, stream) != hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipGreedyArgmaxSampler::sample copy");
        return id;
    }

  private:
    int vocab_;
    std::shared_ptr<Context> ctx_;
    int32_t* d_id_ = nullptr;
};

// ---------------------------------------------------------------------------
// RMSNorm, y = x / sqrt(mean(x^2) + eps) * (1 + w).
class HipRMSNorm {
  public:
    explicit HipRMSNorm(int hidden_size = 1024, float eps = 1e-6f, std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden_size), eps_(eps), ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {}
    ~HipRMSNorm() { (void)hipFree(d_w_); }
    HipRMSNorm(const HipRMSNorm&) = delete;
    HipRMSNorm& operator=(const HipRMSNorm&) = delete;

    void set_weights(const std::vector<float>& weight) {
        if ((int)weight.size() != hidden_) throw Error(QW_ERR_SHAPE, "HipRMSNorm::set_weights: size != hidden");
        if (!d_w_ && hipMalloc(&d_w_, sizeof(float) * hidden_) != hipSuccess)
            throw Error(QW_ERR_NOMEM, "HipRMSNorm::set_weights");
        if (hipMemcpy(d_w_, weight.data(), sizeof(float) * hidden_, hipMemcpyHostToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipRMSNorm::set_weights copy");
    }

    void forward(const float* input, float* output, int batch_size = 1, hipStream_t stream = nullptr) const {
        detail::require(d_w_, "HipRMSNorm::forward");
        ctx_->check(qw_rmsnorm(ctx_->get(), input, QW_F32, d_w_, eps_, output, QW_F32, batch_size, hidden_, stream),
                    "HipRMSNorm::forward");
    }

    // residual_out = residual_in + attn_out; normed_out = RMSNorm(residual_out)
    void forward_with_residual(const float* residual_in, const float* attn_out, float* residual_out,
                               float* normed_out, int batch_size = 1, hipStream_t stream = nullptr) const {
        detail::require(d_w_, "HipRMSNorm::forward_with_residual");
        ctx_->check(qw_residual_rmsnorm(ctx_->get(), residual_in, attn_out, QW_F32, residual_out, normed_out, QW_F32,
                                        d_w_, eps_, batch_size, hidden_, stream),
                    "HipRMSNorm::forward_with_residual");
    }

    const float* d_weight() const { return d_w_; }
    int hidden_size() const { return hidden_; }

  private:
    int hidden_;
    float eps_;
    std::shared_ptr<Context> ctx_;
    float* d_w_ = nullptr;
};

// ---------------------------------------------------------------------------
// Projections of a Gated-DeltaNet layer (language_linear_attn.cpp:136-168,
// 258-263; linear_attention_cuda.cu:412-466): in_proj_qkv [6144][1024],
// in_proj_z [2048][1024], in_proj_a / in_proj_b [16][1024],
// out_proj [1024][2048].  Default storage BF16 (as CudaLinearAttention).
class HipLinearAttnProjections {
  public:
    explicit HipLinearAttnProjections(int hidden = 1024, int qkv_dim = 6144, int z_dim = 2048, int num_v_heads = 16,
                                      qw_wfmt format = QW_WFMT_BF16, std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden), qkv_(qkv_dim), z_(z_dim), nh_(num_v_heads), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {}

    void set_weights(const std::vector<float>& in_proj_qkv, const std::vector<float>& in_proj_z,
                     const std::vector<float>& in_proj_a, const std::vector<float>& in_proj_b,
                     const std::vector<float>& out_proj) {
        Wqkv_ = detail::pack(*ctx_, in_proj_qkv, qkv_, hidden_, fmt_, "in_proj_qkv");
        Wz_ = detail::pack(*ctx_, in_proj_z, z_, hidden_, fmt_, "in_proj_z");
        Wa_ = detail::pack(*ctx_, in_proj_a, nh_, hidden_, fmt_, "in_proj_a");
        Wb_ = detail::pack(*ctx_, in_proj_b, nh_, hidden_, fmt_, "in_proj_b");
        Wo_ = detail::pack(*ctx_, out_proj, hidden_, z_, fmt_, "out_proj");
    }

    // qkv[b] = Wqkv.x[b], z[b] = Wz.x[b], a[b] = Wa.x[b], beta_raw[b] = Wb.x[b]
    void project_in(const float* x, float* qkv, float* z, float* a, float* b, int batch_size = 1,
                    hipStream_t stream = nullptr) const {
        detail::require(Wo_.get(), "HipLinearAttnProjections::project_in");
        lin(Wqkv_.get(), x, qkv, batch_size, nullptr, stream, "in_proj_qkv");
        lin(Wz_.get(), x, z, batch_size, nullptr, stream, "in_proj_z");
        lin(Wa_.get(), x, a, batch_size, nullptr, stream, "in_proj_a");
        lin(Wb_.get(), x, b, batch_size, nullptr, stream, "in_proj_b");
    }

    // residual[b] += Wo.core[b]
    void project_out_add_residual(const float* core, float* residual, int batch_size = 1,
                                  hipStream_t stream = nullptr) const {
        detail::require(Wo_.get(), "HipLinearAttnProjections::project_out_add_residual");
        qw_epilogue ep{};
        ep.flags = QW_EP_RESIDUAL;
        ep.residual = residual;
        ep.residual_dtype = QW_F32;
        lin(Wo_.get(), core, residual, batch_size, &ep, stream, "out_proj");
    }

  private:
    void lin(const qw_weight* W, const float* x, float* y, int M, const qw_epilogue* ep, hipStream_t st,
             const char* what) const {
        ctx_->check(qw_linear(ctx_->get(), W, x, QW_F32, 0, M, y, QW_F32, 0, ep, st), what);
    }
    int hidden_, qkv_, z_, nh_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr Wqkv_, Wz_, Wa_, Wb_, Wo_;
};

// ---------------------------------------------------------------------------
// Recurrent and conv state of a Gated-DeltaNet layer (CudaLinearAttnState,
// linear_attention_cuda.hpp:11-22): device FP32, recurrent state
// [sequences][nh][kd][vd], conv state [sequences][conv_dim][conv_kernel-1]
// (index 0 the newest input), conv_dim = 2*nh*kd + nh*vd.  The reference
// state holds one sequence; `sequences` > 1 (an extension) backs
// HipLinearAttention::forward_decode_sequences.
struct HipLinearAttnState {
    float* d_recurrent_state = nullptr;
    float* d_conv_state = nullptr;
    int num_heads = 0, key_dim = 0, value_dim = 0, conv_dim = 0, conv_kernel = 0, sequences = 0;

    HipLinearAttnState() = default;
    HipLinearAttnState(const HipLinearAttnState&) = delete;
    HipLinearAttnState& operator=(const HipLinearAttnState&) = delete;
    ~HipLinearAttnState() { release(); }

    // (re)allocate for `seqs` sequences and zero
    void reset(int nh, int kd, int vd, int conv_k = 4, int seqs = 1) {
        release();
        num_heads = nh;
        key_dim = kd;
        value_dim = vd;
        conv_kernel = conv_k;
        conv_dim = nh * (2 * kd + vd);
        sequences = seqs;
        if (hipMalloc(&d_recurrent_state, rec_bytes()) != hipSuccess ||
            (conv_bytes() && hipMalloc(&d_conv_state, conv_bytes()) != hipSuccess))
            throw Error(QW_ERR_HIP, "HipLinearAttnState::reset: hipMalloc");
        clear();
    }
    void clear() {
        if (hipMemset(d_recurrent_state, 0, rec_bytes()) != hipSuccess ||
            (d_conv_state && hipMemset(d_conv_state, 0, conv_bytes()) != hipSuccess))
            throw Error(QW_ERR_HIP, "HipLinearAttnState::clear: hipMemset");
    }
    size_t rec_bytes() const { return (size_t)sequences * num_heads * key_dim * value_dim * sizeof(float); }
    size_t conv_bytes() const { return (size_t)sequences * conv_dim * (conv_kernel - 1) * sizeof(float); }

  private:
    void release() {
        if (d_recurrent_state) (void)hipFree(d_recurrent_state);
        if (d_conv_state) (void)hipFree(d_conv_state);
        d_recurrent_state = d_conv_state = nullptr;
    }
};

// ---------------------------------------------------------------------------
// A whole Gated-DeltaNet layer (CudaLinearAttention,
// linear_attention_cuda.hpp:24-90; CPU LinearAttention::forward,
// language_linear_attn.cpp:125-257):
//   [qkv | z | a | b] = W_in . x      one stacked projection (all tokens)
//   core = gated delta steps(...)    qw_gdn_prefill (conv, gates, state, norm-gate)
//   output = W_out . core            (all tokens)
// forward_batch(input, output, state, n) runs n consecutive tokens of the
// state's one sequence, serially, as the reference forward_batch is
// specified (equal to n single-token forward calls,
// verify_linear_attn_batch.cu:68-112); forward_decode_sequences (an
// extension) runs one token for each of n sequences with their own states.
// set_weights takes the reference's arguments in the reference's order;
// empty a_log / dt_bias / norm_weight default to 0 / 0 / 1 as there
// (linear_attention_cuda.cu:450-464).  Default storage BF16.  The projection
// and core buffers grow with the batch on first use (as the reference's
// ensure_batch_buffers); the step itself allocates nothing.
class HipLinearAttention {
  public:
    explicit HipLinearAttention(int hidden = 1024, int num_heads = 16, int key_dim = 128, int value_dim = 128,
                                int conv_kernel = 4, qw_wfmt format = QW_WFMT_BF16,
                                std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden), nh_(num_heads), kd_(key_dim), vd_(value_dim), K_(conv_kernel), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {
        conv_dim_ = nh_ * (2 * kd_ + vd_);
        nin_ = conv_dim_ + nh_ * vd_ + 2 * nh_;
    }
    ~HipLinearAttention() {
        for (float* p : {d_conv_w_, d_A_log_, d_dt_bias_, d_norm_w_, d_row_, d_core_})
            if (p) (void)hipFree(p);
    }
    HipLinearAttention(const HipLinearAttention&) = delete;
    HipLinearAttention& operator=(const HipLinearAttention&) = delete;

    void set_weights(const std::vector<float>& in_proj_qkv_weight, const std::vector<float>& in_proj_a_weight,
                     const std::vector<float>& in_proj_b_weight, const std::vector<float>& in_proj_z_weight,
                     const std::vector<float>& conv1d_weight, const std::vector<float>& out_proj_weight,
                     const std::vector<float>& a_log = {}, const std::vector<float>& dt_bias = {},
                     const std::vector<float>& norm_weight = {}) {
        const int H = hidden_;
        check_size(in_proj_qkv_weight, (size_t)conv_dim_ * H, "in_proj_qkv");
        check_size(in_proj_z_weight, (size_t)nh_ * vd_ * H, "in_proj_z");
        check_size(in_proj_a_weight, (size_t)nh_ * H, "in_proj_a");
        check_size(in_proj_b_weight, (size_t)nh_ * H, "in_proj_b");
        check_size(conv1d_weight, (size_t)conv_dim_ * K_, "conv1d");
        check_size(out_proj_weight, (size_t)H * nh_ * vd_, "out_proj");
        const float* parts[4] = {in_proj_qkv_weight.data(), in_proj_z_weight.data(), in_proj_a_weight.data(),
                                 in_proj_b_weight.data()};
        const int Ns[4] = {conv_dim_, nh_ * vd_, nh_, nh_};
        qw_weight* w = nullptr;
        ctx_->check(qw_weight_pack_concat(ctx_->get(), 4, reinterpret_cast<const void* const*>(parts), Ns, QW_F32,
                                          fmt_, H, nullptr, &w),
                    "HipLinearAttention in_proj");
        Win_.reset(w);
        Wout_ = detail::pack(*ctx_, out_proj_weight, H, nh_ * vd_, fmt_, "out_proj");
        upload(d_conv_w_, conv1d_weight, conv1d_weight.size());
        upload(d_A_log_, a_log.empty() ? std::vector<float>(nh_, 0.0f) : a_log, nh_);
        upload(d_dt_bias_, dt_bias.empty() ? std::vector<float>(nh_, 0.0f) : dt_bias, nh_);
        upload(d_norm_w_, norm_weight.empty() ? std::vector<float>(vd_, 1.0f) : norm_weight, vd_);
    }

    void forward(const float* input, float* output, HipLinearAttnState& state, hipStream_t stream = nullptr) const {
        forward_batch(input, output, state, 1, stream);
    }

    // input/output [batch_size][hidden] FP32 device: batch_size consecutive
    // tokens of sequence 0 of `state`
    void forward_batch(const float* input, float* output, HipLinearAttnState& state, int batch_size,
                       hipStream_t stream = nullptr) const {
        run(input, output, state, 1, batch_size, "HipLinearAttention::forward_batch", stream);
    }

    // input/output [n][hidden]: one token for each of sequences 0..n-1 of `state`
    void forward_decode_sequences(const float* input, float* output, HipLinearAttnState& state, int n,
                                  hipStream_t stream = nullptr) const {
        run(input, output, state, n, 1, "HipLinearAttention::forward_decode_sequences", stream);
    }

    // CudaLinearAttention::forward_fused (linear_attention_cuda.cu:686-689) is forward
    void forward_fused(const float* input, float* output, HipLinearAttnState& state,
                       hipStream_t stream = nullptr) const {
        forward_batch(input, output, state, 1, stream);
    }

  private:
    void run(const float* input, float* output, HipLinearAttnState& state, int seqs, int tokens, const char* what,
             hipStream_t stream) const {
        detail::require(Wout_.get(), what);
        if (state.num_heads != nh_ || state.key_dim != kd_ || state.value_dim != vd_ ||
            state.conv_kernel != K_ || state.sequences < seqs)
            throw Error(QW_ERR_SHAPE, std::string(what) + ": state shape does not match");
        if (seqs < 1 || tokens < 1) throw Error(QW_ERR_SHAPE, std::string(what) + ": empty batch");
        const int rows = seqs * tokens;
        ensure(rows);
        ctx_->check(qw_linear(ctx_->get(), Win_.get(), input, QW_F32, 0, rows, d_row_, QW_F32, nin_, nullptr, stream),
                    what);
        qw_gdn_params p{nh_, kd_, vd_, K_, d_conv_w_, d_A_log_, d_dt_bias_, d_norm_w_};
        const float* z = d_row_ + conv_dim_;
        const float* a = z + nh_ * vd_;
        const float* b = a + nh_;
        ctx_->check(qw_gdn_prefill(ctx_->get(), &p, seqs, tokens, d_row_, z, a, b, QW_F32, nin_, state.d_conv_state,
                                   state.d_recurrent_state, d_core_, QW_F32, nh_ * vd_, stream),
                    what);
        ctx_->check(
            qw_linear(ctx_->get(), Wout_.get(), d_core_, QW_F32, 0, rows, output, QW_F32, 0, nullptr, stream), what);
    }
    static void check_size(const std::vector<float>& v, size_t n, const char* name) {
        if (v.size() != n) throw Error(QW_ERR_SHAPE, std::string(name) + ": expected " + std::to_string(n) + " floats");
    }
    static void upload(float*& d, const std::vector<float>& h, size_t n) {
        if (!d && hipMalloc(&d, n * sizeof(float)) != hipSuccess) throw Error(QW_ERR_HIP, "hipMalloc");
        if (hipMemcpy(d, h.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "hipMemcpy");
    }
    void ensure(int batch) const {
        if (batch <= cap_) return;
        if (d_row_) (void)hipFree(d_row_);
        if (d_core_) (void)hipFree(d_core_);
        if (hipMalloc(&d_row_, (size_t)batch * nin_ * sizeof(float)) != hipSuccess ||
            hipMalloc(&d_core_, (size_t)batch * nh_ * vd_ * sizeof(float)) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipLinearAttention: hipMalloc");
        cap_ = batch;
    }
    int hidden_, nh_, kd_, vd_, K_, conv_dim_, nin_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr Win_, Wout_;
    float *d_conv_w_ = nullptr, *d_A_log_ = nullptr, *d_dt_bias_ = nullptr, *d_norm_w_ = nullptr;
    mutable float *d_row_ = nullptr, *d_core_ = nullptr;
    mutable int cap_ = 0;
};

// ---------------------------------------------------------------------------
// Projections of a gated full-attention layer (language_full_attn.cpp:127-156,
// 218-223): q_proj [2*heads*head_dim][hidden] interleaved per head as
// [Q(head_dim) | gate(head_dim)], k_proj / v_proj [kv_heads*head_dim][hidden],
// o_proj [hidden][heads*head_dim].  project_in de-interleaves Q and gate in
// the epilogue.
class HipFullAttnProjections {
  public:
    explicit HipFullAttnProjections(int hidden = 1024, int heads = 8, int kv_heads = 2, int head_dim = 256,
                                    qw_wfmt format = QW_WFMT_F32, std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden), heads_(heads), kvh_(kv_heads), hd_(head_dim), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {}

    void set_weights(const std::vector<float>& q_proj, const std::vector<float>& k_proj,
                     const std::vector<float>& v_proj, const std::vector<float>& o_proj) {
        Wq_ = detail::pack(*ctx_, q_proj, 2 * heads_ * hd_, hidden_, fmt_, "q_proj");
        Wk_ = detail::pack(*ctx_, k_proj, kvh_ * hd_, hidden_, fmt_, "k_proj");
        Wv_ = detail::pack(*ctx_, v_proj, kvh_ * hd_, hidden_, fmt_, "v_proj");
        Wo_ = detail::pack(*ctx_, o_proj, hidden_, heads_ * hd_, fmt_, "o_proj");
    }

    // q[b] / gate[b]: [heads*head_dim] each; k[b], v[b]: [kv_heads*head_dim]
    void project_in(const float* x, float* q, float* gate, float* k, float* v, int batch_size = 1,
                    hipStream_t stream = nullptr) const {
        detail::require(Wo_.get(), "HipFullAttnProjections::project_in");
        qw_epilogue ep{};
        ep.flags = QW_EP_SPLIT;
        ep.split_period = hd_;
        ep.y2 = gate;
        ctx_->check(qw_linear(ctx_->get(), Wq_.get(), x, QW_F32, 0, batch_size, q, QW_F32, heads_ * hd_, &ep, stream),
                    "q_proj");
        ctx_->check(qw_linear(ctx_->get(), Wk_.get(), x, QW_F32, 0, batch_size, k, QW_F32, 0, nullptr, stream),
                    "k_proj");
        ctx_->check(qw_linear(ctx_->get(), Wv_.get(), x, QW_F32, 0, batch_size, v, QW_F32, 0, nullptr, stream),
                    "v_proj");
    }

    // residual[b] += Wo.core[b]
    void project_out_add_residual(const float* core, float* residual, int batch_size = 1,
                                  hipStream_t stream = nullptr) const {
        detail::require(Wo_.get(), "HipFullAttnProjections::project_out_add_residual");
        qw_epilogue ep{};
        ep.flags = QW_EP_RESIDUAL;
        ep.residual = residual;
        ep.residual_dtype = QW_F32;
        ctx_->check(qw_linear(ctx_->get(), Wo_.get(), core, QW_F32, 0, batch_size, residual, QW_F32, 0, &ep, stream),
                    "o_proj");
    }

  private:
    int hidden_, heads_, kvh_, hd_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr Wq_, Wk_, Wv_, Wo_;
};


// ---------------------------------------------------------------------------
// KV cache of all full-attention layers (CudaKVCache, full_attention_cuda.hpp:
// 11-33; grow/ensure_capacity full_attention_cuda.cu:255-330): per layer
// [capacity][kv_heads][head_dim], INT8 with one FP32 scale per token and KV
// head (the reference format) or FP32 (the CPU KVCache format); capacity
// doubles on demand, keeping the contents.  layer_lengths is host-side
// bookkeeping, as in the reference.
struct HipKVCache {
    void* d_k_cache = nullptr;
    void* d_v_cache = nullptr;
    float* d_k_scale = nullptr;
    float* d_v_scale = nullptr;
    std::vector<int> layer_lengths;
    int num_layers = 0, num_kv_heads = 0, head_dim = 0, capacity_seq_len = 0, max_seq_len = 0;
    bool int8 = true;

    HipKVCache() = default;
    HipKVCache(const HipKVCache&) = delete;
    HipKVCache& operator=(const HipKVCache&) = delete;
    ~HipKVCache() { release(); }

    void reset(int nl, int nkh, int hd, int init_capacity = 1024, bool int8_cache = true) {
        release();
        num_layers = nl;
        num_kv_heads = nkh;
        head_dim = hd;
        int8 = int8_cache;
        max_seq_len = 0;
        layer_lengths.assign(nl, 0);
        allocate(init_capacity, &d_k_cache, &d_v_cache, &d_k_scale, &d_v_scale);
        capacity_seq_len = init_capacity;
    }
    void clear() {
        zero(d_k_cache, d_v_cache, d_k_scale, d_v_scale, capacity_seq_len);
        std::fill(layer_lengths.begin(), layer_lengths.end(), 0);
        max_seq_len = 0;
    }
    int length(int layer_idx) const { return layer_lengths[layer_idx]; }
    void ensure_capacity(int required) {
        if (required <= capacity_seq_len) return;
        int cap = capacity_seq_len * 2;
        while (cap < required) cap *= 2;
        void *k, *v;
        float *ks, *vs;
        allocate(cap, &k, &v, &ks, &vs);
        for (int l = 0; l < num_layers; ++l) {  // copy each layer's slice into the larger stride
            copy_layer(k, d_k_cache, cap, l, (size_t)num_kv_heads * head_dim * esize());
            copy_layer(v, d_v_cache, cap, l, (size_t)num_kv_heads * head_dim * esize());
            if (int8) {
                copy_layer(ks, d_k_scale, cap, l, (size_t)num_kv_heads * sizeof(float));
                copy_layer(vs, d_v_scale, cap, l, (size_t)num_kv_heads * sizeof(float));
            }
        }
        release_buffers();
        d_k_cache = k;
        d_v_cache = v;
        d_k_scale = ks;
        d_v_scale = vs;
        capacity_seq_len = cap;
    }
    // the C-ABI view of one layer (one sequence)
    qw_kv_cache layer(int l) const {
        const size_t per = (size_t)capacity_seq_len * num_kv_heads;
        qw_kv_cache c{};
        c.dtype = int8 ? QW_I8 : QW_F32;
        c.k = static_cast<uint8_t*>(d_k_cache) + (size_t)l * per * head_dim * esize();
        c.v = static_cast<uint8_t*>(d_v_cache) + (size_t)l * per * head_dim * esize();
        c.k_scale = int8 ? d_k_scale + (size_t)l * per : nullptr;
        c.v_scale = int8 ? d_v_scale + (size_t)l * per : nullptr;
        c.capacity = capacity_seq_len;
        return c;
    }

  private:
    size_t esize() const { return int8 ? 1 : 4; }
    void allocate(int cap, void** k, void** v, float** ks, float** vs) const {
        const size_t n = (size_t)num_layers * cap * num_kv_heads * head_dim * esize();
        const size_t ns = (size_t)num_layers * cap * num_kv_heads * sizeof(float);
        *ks = *vs = nullptr;
        if (hipMalloc(k, n) != hipSuccess || hipMalloc(v, n) != hipSuccess ||
            (int8 && (hipMalloc(reinterpret_cast<void**>(ks), ns) != hipSuccess ||
                      hipMalloc(reinterpret_cast<void**>(vs), ns) != hipSuccess)))
            throw Error(QW_ERR_HIP, "HipKVCache: hipMalloc");
        zero(*k, *v, *ks, *vs, cap);
    }
    void zero(void* k, void* v, float* ks, float* vs, int cap) const {
        const size_t n = (size_t)num_layers * cap * num_kv_heads * head_dim * esize();
        const size_t ns = (size_t)num_layers * cap * num_kv_heads * sizeof(float);
        if (hipMemset(k, 0, n) != hipSuccess || hipMemset(v, 0, n) != hipSuccess ||
            (ks && hipMemset(ks, 0, ns) != hipSuccess) || (vs && hipMemset(vs, 0, ns) != hipSuccess))
            throw Error(QW_ERR_HIP, "HipKVCache: hipMemset");
    }
    void copy_layer(void* dst, const void* src, int new_cap, int l, size_t token_bytes) const {
        if (hipMemcpy(static_cast<uint8_t*>(dst) + (size_t)l * new_cap * token_bytes,
                      static_cast<const uint8_t*>(src) + (size_t)l * capacity_seq_len * token_bytes,
                      (size_t)capacity_seq_len * token_bytes, hipMemcpyDeviceToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipKVCache: hipMemcpy");
    }
    void release_buffers() {
        for (void* p : {d_k_cache, d_v_cache, static_cast<void*>(d_k_scale), static_cast<void*>(d_v_scale)})
            if (p) (void)hipFree(p);
        d_k_cache = d_v_cache = nullptr;
        d_k_scale = d_v_scale = nullptr;
    }
    void release() { release_buffers(); }
};

// ---------------------------------------------------------------------------
// A whole gated full-attention layer (CudaFullAttention,
// full_attention_cuda.hpp:35-90; CPU FullAttention::forward,
// language_full_attn.cpp:117-216):
//   [q|gate interleaved per head | k | v] = W_in . x   one stacked projection
//   core = qw_attn_forward(...)   norms, RoPE, cache write, causal attention, gate
//   output = W_o . core
// forward(input, output, cache, layer, position) runs one token;
// forward_batch_prefill(..., positions, batch_size, max_seq) runs batch_size
// consecutive tokens of one sequence starting at positions[0] (device), the
// way the reference engine calls it (positions 0 .. n-1 of a prompt).
// Rotary: 64 of 256 dims, theta 1e7 (the reference's constants).
class HipFullAttention {
  public:
    explicit HipFullAttention(int hidden = 1024, int num_heads = 8, int num_kv_heads = 2, int q_head_dim = 256,
                              int kv_head_dim = 256, qw_wfmt format = QW_WFMT_BF16,
                              std::shared_ptr<Context> ctx = nullptr)
        : hidden_(hidden), nh_(num_heads), nkv_(num_kv_heads), hd_(kv_head_dim), fmt_(format),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {
        if (q_head_dim != kv_head_dim) throw Error(QW_ERR_SHAPE, "HipFullAttention: q_head_dim must equal kv_head_dim");
        nin_ = nh_ * 2 * hd_ + 2 * nkv_ * hd_;
    }
    ~HipFullAttention() {
        for (void* p : {static_cast<void*>(d_qn_), static_cast<void*>(d_kn_), static_cast<void*>(d_row_),
                        static_cast<void*>(d_core_), static_cast<void*>(d_pos_)})
            if (p) (void)hipFree(p);
    }
    HipFullAttention(const HipFullAttention&) = delete;
    HipFullAttention& operator=(const HipFullAttention&) = delete;

    void set_weights(const std::vector<float>& q_proj_weight, const std::vector<float>& k_proj_weight,
                     const std::vector<float>& v_proj_weight, const std::vector<float>& q_norm_weight,
                     const std::vector<float>& k_norm_weight, const std::vector<float>& o_proj_weight) {
        const int H = hidden_;
        check(q_proj_weight, (size_t)nh_ * 2 * hd_ * H, "q_proj");
        check(k_proj_weight, (size_t)nkv_ * hd_ * H, "k_proj");
        check(v_proj_weight, (size_t)nkv_ * hd_ * H, "v_proj");
        check(q_norm_weight, (size_t)hd_, "q_norm");
        check(k_norm_weight, (size_t)hd_, "k_norm");
        check(o_proj_weight, (size_t)H * nh_ * hd_, "o_proj");
        const float* parts[3] = {q_proj_weight.data(), k_proj_weight.data(), v_proj_weight.data()};
        const int Ns[3] = {nh_ * 2 * hd_, nkv_ * hd_, nkv_ * hd_};
        qw_weight* w = nullptr;
        ctx_->check(qw_weight_pack_concat(ctx_->get(), 3, reinterpret_cast<const void* const*>(parts), Ns, QW_F32,
                                          fmt_, H, nullptr, &w),
                    "HipFullAttention in_proj");
        Win_.reset(w);
        Wo_ = detail::pack(*ctx_, o_proj_weight, H, nh_ * hd_, fmt_, "o_proj");
        upload(d_qn_, q_norm_weight);
        upload(d_kn_, k_norm_weight);
        if (!d_pos_ && hipMalloc(&d_pos_, sizeof(int)) != hipSuccess) throw Error(QW_ERR_HIP, "hipMalloc");
    }

    void forward(const float* input, float* output, HipKVCache& kv_cache, int layer_idx, int position,
                 hipStream_t stream = nullptr) const {
        kv_cache.ensure_capacity(position + 1);
        kv_cache.max_seq_len = std::max(kv_cache.max_seq_len, position + 1);
        if (hipMemcpyAsync(d_pos_, &position, sizeof(int), hipMemcpyHostToDevice, stream) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipFullAttention: position upload");
        run(input, output, kv_cache, layer_idx, d_pos_, 1, position + 1, stream);
        if (hipStreamSynchronize(stream) != hipSuccess) throw Error(QW_ERR_HIP, "HipFullAttention: sync");
        kv_cache.layer_lengths[layer_idx] = std::max(kv_cache.layer_lengths[layer_idx], position + 1);
    }

    // batch_size consecutive tokens of one sequence from positions[0] (device int)
    void forward_batch_prefill(const float* input, float* output, HipKVCache& kv_cache, int layer_idx,
                               const int* positions, int batch_size, int max_seq = 0,
                               hipStream_t stream = nullptr) const {
        int end = max_seq;
        if (end == 0) {  // as the reference: read the positions back to size the cache
            int p0 = 0;
            if (hipMemcpy(&p0, positions, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
                throw Error(QW_ERR_HIP, "HipFullAttention: positions read");
            end = p0 + batch_size;
        }
        kv_cache.ensure_capacity(end);
        kv_cache.max_seq_len = std::max(kv_cache.max_seq_len, end);
        run(input, output, kv_cache, layer_idx, positions, batch_size, end, stream);
        kv_cache.layer_lengths[layer_idx] = std::max(kv_cache.layer_lengths[layer_idx], end);
    }

  private:
    void run(const float* input, float* output, HipKVCache& kv, int layer, const int* pos, int T, int max_len,
             hipStream_t stream) const {
        detail::require(Wo_.get(), "HipFullAttention::forward");
        if (kv.num_kv_heads != nkv_ || kv.head_dim != hd_ || layer < 0 || layer >= kv.num_layers)
            throw Error(QW_ERR_SHAPE, "HipFullAttention: cache shape does not match");
        ensure(T);
        ctx_->check(qw_linear(ctx_->get(), Win_.get(), input, QW_F32, 0, T, d_row_, QW_F32, nin_, nullptr, stream),
                    "HipFullAttention in_proj");
        qw_attn_params p{nh_, nkv_, hd_, hd_ / 4, 1.0e7f, d_qn_, d_kn_};
        const qw_kv_cache c = kv.layer(layer);
        const float* q = d_row_;
        ctx_->check(qw_attn_forward(ctx_->get(), &p, &c, 1, T, pos, max_len, q, q + hd_, 2 * hd_,
                                    q + nh_ * 2 * hd_, q + nh_ * 2 * hd_ + nkv_ * hd_, QW_F32, nin_, d_core_, QW_F32,
                                    nh_ * hd_, stream),
                    "HipFullAttention core");
        ctx_->check(qw_linear(ctx_->get(), Wo_.get(), d_core_, QW_F32, 0, T, output, QW_F32, 0, nullptr, stream),
                    "HipFullAttention o_proj");
    }
    static void check(const std::vector<float>& v, size_t n, const char* name) {
        if (v.size() != n) throw Error(QW_ERR_SHAPE, std::string(name) + ": expected " + std::to_string(n) + " floats");
    }
    static void upload(float*& d, const std::vector<float>& h) {
        if (!d && hipMalloc(&d, h.size() * sizeof(float)) != hipSuccess) throw Error(QW_ERR_HIP, "hipMalloc");
        if (hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "hipMemcpy");
    }
    void ensure(int T) const {
        if (T <= cap_) return;
        if (d_row_) (void)hipFree(d_row_);
        if (d_core_) (void)hipFree(d_core_);
        if (hipMalloc(&d_row_, (size_t)T * nin_ * sizeof(float)) != hipSuccess ||
            hipMalloc(&d_core_, (size_t)T * nh_ * hd_ * sizeof(float)) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipFullAttention: hipMalloc");
        cap_ = T;
    }
    int hidden_, nh_, nkv_, hd_, nin_;
    qw_wfmt fmt_;
    std::shared_ptr<Context> ctx_;
    detail::WeightPtr Win_, Wo_;
    float *d_qn_ = nullptr, *d_kn_ = nullptr;
    int* d_pos_ = nullptr;
    mutable float *d_row_ = nullptr, *d_core_ = nullptr;
    mutable int cap_ = 0;
};


// ---------------------------------------------------------------------------
// Whole model for one sequence: the drop-in for CudaEngine
// (cuda_engine.hpp:85-133, cuda_engine.cu:244-479).
//   set_layer_weights(i, flat)  slices the reference flat layer layout
//       (cuda_engine.cu:244-298, WEIGHT_FORMAT.md): norms and MLP, then the
//       whole linear-attention section, then the whole full-attention
//       section, matrices [out][in]; the section of the layer's type is packed;
//   forward(in, out, position)  one token: every layer, then the final norm
//       (out = RMSNorm(x) * (1 + w), as CudaEngine::forward);
//   forward_batch_prefill / _graph / _decode(in, out, positions, n)  n
//       consecutive tokens of the sequence from host positions[0] on (the
//       reference's contract for these calls: positions[b] = positions[0] + b).
// Layer types follow the CPU backbone: layer i is Gated-DeltaNet unless
// i % 4 == 3 (language_common.hpp is_linear_layer).  The reference CUDA
// engine instead runs every layer as full attention (cuda_engine.cu:252-254);
// the CPU operator is the specification here.  Each layer is
//   x += attn(RMSNorm(x) * (1 + w_in));  x += MLP(RMSNorm(x) * (1 + w_post))
// with the norms inside the projections' prologues, the residual adds in
// their epilogues and the MLP in qw_mlp_fused (language_backbone.cpp:54-88).
// Weights are stored in `format` (FP32 default, the reference's precision);
// the KV cache is FP32 by default (the CPU KVCache) or INT8.
class HipEngine {
  public:
    static constexpr int LNH = 16, LKD = 128, LVD = 128, LCK = 4;  // Gated-DeltaNet heads, dims, conv taps
    static constexpr int FNH = 8, FNKV = 2, FHD = 256;             // full attention heads, KV heads, head dim

    HipEngine(int num_layers, int hidden_size, int intermediate_size, int vocab_size, int max_seq_len,
              qw_wfmt format = QW_WFMT_F32, bool int8_kv_cache = false, std::shared_ptr<Context> ctx = nullptr)
        : nl_(num_layers), H_(hidden_size), I_(intermediate_size), V_(vocab_size), max_seq_(max_seq_len),
          fmt_(format), kv_int8_(int8_kv_cache),
          ctx_(ctx ? std::move(ctx) : Context::default_for_current_device()) {
        if (nl_ < 1 || H_ < 64 || H_ % 64 || I_ < 64 || I_ % 64 || max_seq_ < 1)
            throw Error(QW_ERR_SHAPE, "HipEngine: bad model shape");
        layers_.resize(nl_);
        for (int i = 0; i < nl_; ++i) layers_[i].linear = is_linear_layer(i);
        alloc(d_pos_, 1);
        ensure(1);
    }
    ~HipEngine() {
        for (auto& L : layers_) free_layer(L);
        for (void* p : {(void*)d_x_, (void*)d_row_, (void*)d_core_, (void*)d_pos_, (void*)d_final_norm_, (void*)d_out_})
            if (p) (void)hipFree(p);
    }
    HipEngine(const HipEngine&) = delete;
    HipEngine& operator=(const HipEngine&) = delete;

    static bool is_linear_layer(int i) { return i % 4 != 3; }

    // floats of one flat layer vector (every section present, as the reference slices it)
    size_t flat_layer_size() const {
        const size_t H = H_, I = I_, cd = LNH * (2 * LKD + LVD);
        return 2 * H + 3 * I * H + cd * H + 2 * (size_t)LNH * H + (size_t)LNH * LVD * H + cd * LCK + H * LNH * LVD +
               2 * LNH + LVD + (size_t)FNH * FHD * 2 * H + 2 * (size_t)FNKV * FHD * H + 2 * FHD + H * FNH * FHD;
    }

    void set_layer_weights(int layer_idx, const std::vector<float>& weights_flat) {
        if (layer_idx < 0 || layer_idx >= nl_) throw Error(QW_ERR_INVALID, "HipEngine::set_layer_weights: layer index");
        if (weights_flat.size() < flat_layer_size())
            throw Error(QW_ERR_SHAPE, "HipEngine::set_layer_weights: flat vector shorter than " +
                                          std::to_string(flat_layer_size()) + " floats");
        Layer& L = layers_[layer_idx];
        free_layer(L);
        const float* p = weights_flat.data();
        auto take = [&](size_t n) {
            const float* q = p;
            p += n;
            return q;
        };
        const size_t H = H_, I = I_, cd = LNH * (2 * LKD + LVD), lv = (size_t)LNH * LVD;
        const float* in_norm = take(H);
        const float* post_norm = take(H);
        const float* gate = take(I * H);
        const float* up = take(I * H);
        const float* down = take(H * I);
        const float* qkv = take(cd * H);
        const float* la = take((size_t)LNH * H);
        const float* lb = take((size_t)LNH * H);
        const float* lz = take(lv * H);
        const float* conv = take(cd * LCK);
        const float* lout = take(H * lv);
        const float* alog = take(LNH);
        const float* dtb = take(LNH);
        const float* lnorm = take(LVD);
        const float* fq = take((size_t)FNH * FHD * 2 * H);
        const float* fk = take((size_t)FNKV * FHD * H);
        const float* fv = take((size_t)FNKV * FHD * H);
        const float* fqn = take(FHD);
        const float* fkn = take(FHD);
        const float* fo = take(H * FNH * FHD);
        L.in_norm = upload(in_norm, H);
        L.post_norm = upload(post_norm, H);
        qw_weight* w = nullptr;
        ctx_->check(qw_weight_pack_glu(ctx_->get(), gate, up, QW_F32, fmt_, I_, H_, nullptr, nullptr, &w),
                    "HipEngine gate/up");
        L.gateup.reset(w);
        L.down = pack_ptr(down, H_, I_, "HipEngine down");
        if (L.linear) {
            const void* parts[4] = {qkv, lz, la, lb};
            const int Ns[4] = {(int)cd, (int)lv, LNH, LNH};
            ctx_->check(qw_weight_pack_concat(ctx_->get(), 4, parts, Ns, QW_F32, fmt_, H_, nullptr, &w),
                        "HipEngine linear in_proj");
            L.in.reset(w);
            L.out = pack_ptr(lout, H_, (int)lv, "HipEngine linear out_proj");
            L.conv = upload(conv, cd * LCK);
            L.A_log = upload(alog, LNH);
            L.dt_bias = upload(dtb, LNH);
            L.norm_w = upload(lnorm, LVD);
            alloc(L.conv_state, cd * (LCK - 1));
            alloc(L.rec_state, (size_t)LNH * LKD * LVD);
        } else {
            const void* parts[3] = {fq, fk, fv};
            const int Ns[3] = {FNH * FHD * 2, FNKV * FHD, FNKV * FHD};
            ctx_->check(qw_weight_pack_concat(ctx_->get(), 3, parts, Ns, QW_F32, fmt_, H_, nullptr, &w),
                        "HipEngine full in_proj");
            L.in.reset(w);
            L.out = pack_ptr(fo, H_, FNH * FHD, "HipEngine full o_proj");
            L.q_norm = upload(fqn, FHD);
            L.k_norm = upload(fkn, FHD);
            const size_t es = kv_int8_ ? 1 : 4, n = (size_t)max_seq_ * FNKV * FHD;
            if (hipMalloc(&L.kc, n * es) != hipSuccess || hipMalloc(&L.vc, n * es) != hipSuccess)
                throw Error(QW_ERR_HIP, "HipEngine: KV cache hipMalloc");
            if (kv_int8_) {
                alloc(L.ks, (size_t)max_seq_ * FNKV);
                alloc(L.vs, (size_t)max_seq_ * FNKV);
            }
        }
        L.ready = true;
        reset_layer_state(L);
    }

    void set_final_norm_weight(const std::vector<float>& weight) {
        if ((int)weight.size() != H_) throw Error(QW_ERR_SHAPE, "HipEngine::set_final_norm_weight: expected hidden floats");
        if (d_final_norm_) (void)hipFree(d_final_norm_);
        d_final_norm_ = upload(weight.data(), H_);
    }

    // the tied lm_head (CudaEngine keeps one for its callers; forward does not apply it)
    void set_lm_head_weight(const std::vector<float>& weight) {
        if ((int64_t)weight.size() != (int64_t)V_ * H_) throw Error(QW_ERR_SHAPE, "HipEngine::set_lm_head_weight");
        lm_head_ = std::make_unique<HipLMHead>(H_, V_, QW_WFMT_BF16, ctx_);
        lm_head_->set_weight(weight);
    }
    HipLMHead* lm_head() const { return lm_head_.get(); }

    void forward(const float* d_input, float* d_output, int position, hipStream_t stream = nullptr) {
        run(d_input, d_output, position, 1, stream);
    }
    void forward_batch_prefill(const float* d_input, float* d_output, const int* positions, int batch_size,
                               hipStream_t stream = nullptr) {
        if (!positions || batch_size < 1) throw Error(QW_ERR_INVALID, "HipEngine::forward_batch_prefill: positions");
        run(d_input, d_output, positions[0], batch_size, stream);
    }
    void forward_batch_prefill_graph(const float* d_input, float* d_output, const int* positions, int batch_size,
                                     hipStream_t stream = nullptr) {
        forward_batch_prefill(d_input, d_output, positions, batch_size, stream);
    }
    void forward_batch_decode(const float* d_input, float* d_output, const int* positions, int batch_size,
                              hipStream_t stream = nullptr) {
        forward_batch_prefill(d_input, d_output, positions, batch_size, stream);
    }
    void forward_host(const std::vector<float>& input, std::vector<float>& output, int position) {
        if ((int)input.size() != H_) throw Error(QW_ERR_SHAPE, "HipEngine::forward_host: expected hidden floats");
        ensure(1);
        if (hipMemcpy(d_row_, input.data(), H_ * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipEngine::forward_host upload");
        float* in = d_row_;  // staged in the projection buffer, copied into x before any projection writes it
        run(in, d_out_, position, 1, nullptr);
        output = get_output();
    }
    // the last forward_host output
    std::vector<float> get_output() const {
        std::vector<float> h(H_);
        if (hipMemcpy(h.data(), d_out_, H_ * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipEngine::get_output");
        return h;
    }
    void reset_cache() {
        for (auto& L : layers_)
            if (L.ready) reset_layer_state(L);
        length_ = 0;
    }
    bool ready() const {
        if (!d_final_norm_) return false;
        for (const auto& L : layers_)
            if (!L.ready) return false;
        return true;
    }
    int num_layers() const { return nl_; }
    int length() const { return length_; }  // tokens in the cache (one past the last position)

  private:
    struct Layer {
        bool linear = false, ready = false;
        float *in_norm = nullptr, *post_norm = nullptr;
        detail::WeightPtr in, out, gateup, down;
        float *conv = nullptr, *A_log = nullptr, *dt_bias = nullptr, *norm_w = nullptr;
        float *conv_state = nullptr, *rec_state = nullptr;
        float *q_norm = nullptr, *k_norm = nullptr;
        void *kc = nullptr, *vc = nullptr;
        float *ks = nullptr, *vs = nullptr;
    };

    void run(const float* d_input, float* d_output, int p0, int T, hipStream_t stream) {
        if (!ready()) throw Error(QW_ERR_STATE, "HipEngine: weights not set");
        if (p0 < 0 || p0 + T > max_seq_)
            throw Error(QW_ERR_SHAPE, "HipEngine: positions " + std::to_string(p0) + ".." + std::to_string(p0 + T - 1) +
                                          " outside max_seq_len " + std::to_string(max_seq_));
        ensure(T);
        qw_ctx* c = ctx_->get();
        const int cd = LNH * (2 * LKD + LVD), lv = LNH * LVD, lin_in = cd + lv + 2 * LNH;
        const int full_in = FNH * 2 * FHD + 2 * FNKV * FHD, ld_row = std::max(lin_in, full_in);
        if (hipMemcpyAsync(d_x_, d_input, (size_t)T * H_ * sizeof(float), hipMemcpyDeviceToDevice, stream) !=
                hipSuccess ||
            hipMemcpyAsync(d_pos_, &p0, sizeof(int), hipMemcpyHostToDevice, stream) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipEngine: input upload");
        qw_epilogue norm{}, res{};
        norm.flags = QW_EP_NORM_X;
        norm.eps = 1e-6f;
        res.flags = QW_EP_RESIDUAL;
        res.residual = d_x_;
        res.residual_dtype = QW_F32;
        for (auto& L : layers_) {
            norm.gamma = L.in_norm;
            ctx_->check(qw_linear(c, L.in.get(), d_x_, QW_F32, 0, T, d_row_, QW_F32, ld_row, &norm, stream),
                        "HipEngine in_proj");
            if (L.linear) {
                qw_gdn_params gp{LNH, LKD, LVD, LCK, L.conv, L.A_log, L.dt_bias, L.norm_w};
                const float* r = d_row_;
                ctx_->check(qw_gdn_prefill(c, &gp, 1, T, r, r + cd, r + cd + lv, r + cd + lv + LNH, QW_F32, ld_row,
                                           L.conv_state, L.rec_state, d_core_, QW_F32, lv, stream),
                            "HipEngine Gated-DeltaNet");
            } else {
                qw_attn_params ap{FNH, FNKV, FHD, FHD / 4, 1.0e7f, L.q_norm, L.k_norm};
                qw_kv_cache kv{kv_int8_ ? QW_I8 : QW_F32, L.kc, L.vc, L.ks, L.vs, max_seq_};
                const float* r = d_row_;
                ctx_->check(qw_attn_forward(c, &ap, &kv, 1, T, d_pos_, p0 + T, r, r + FHD, 2 * FHD, r + FNH * 2 * FHD,
                                            r + FNH * 2 * FHD + FNKV * FHD, QW_F32, ld_row, d_core_, QW_F32, lv,
                                            stream),
                            "HipEngine attention");
            }
            ctx_->check(qw_linear(c, L.out.get(), d_core_, QW_F32, 0, T, d_x_, QW_F32, 0, &res, stream),
                        "HipEngine out_proj");
            ctx_->check(qw_mlp_fused(c, L.gateup.get(), L.down.get(), d_x_, QW_F32, L.post_norm, 1e-6f, d_x_, QW_F32,
                                     d_x_, QW_F32, T, stream),
                        "HipEngine MLP");
        }
        ctx_->check(qw_rmsnorm(c, d_x_, QW_F32, d_final_norm_, 1e-6f, d_output, QW_F32, T, H_, stream),
                    "HipEngine final norm");
        if (hipStreamSynchronize(stream) != hipSuccess) throw Error(QW_ERR_HIP, "HipEngine: sync");
        length_ = std::max(length_, p0 + T);
    }

    void ensure(int T) {
        if (T <= cap_) return;
        const int cd = LNH * (2 * LKD + LVD), lv = LNH * LVD;
        const int ld_row = std::max(cd + lv + 2 * LNH, FNH * 2 * FHD + 2 * FNKV * FHD);
        for (float** p : {&d_x_, &d_row_, &d_core_, &d_out_})
            if (*p) {
                (void)hipFree(*p);
                *p = nullptr;
            }
        alloc(d_x_, (size_t)T * H_);
        alloc(d_row_, (size_t)T * ld_row);
        alloc(d_core_, (size_t)T * std::max(lv, FNH * FHD));
        alloc(d_out_, (size_t)H_);
        cap_ = T;
    }
    void reset_layer_state(Layer& L) {
        const int cd = LNH * (2 * LKD + LVD);
        if (L.linear) {
            zero(L.conv_state, (size_t)cd * (LCK - 1) * sizeof(float));
            zero(L.rec_state, (size_t)LNH * LKD * LVD * sizeof(float));
        } else {
            const size_t n = (size_t)max_seq_ * FNKV * FHD * (kv_int8_ ? 1 : 4);
            zero(L.kc, n);
            zero(L.vc, n);
            if (kv_int8_) {
                zero(L.ks, (size_t)max_seq_ * FNKV * sizeof(float));
                zero(L.vs, (size_t)max_seq_ * FNKV * sizeof(float));
            }
        }
    }
    static void zero(void* p, size_t bytes) {
        if (p && hipMemset(p, 0, bytes) != hipSuccess) throw Error(QW_ERR_HIP, "HipEngine: hipMemset");
    }
    static void alloc(float*& p, size_t n) {
        if (hipMalloc(&p, n * sizeof(float)) != hipSuccess) throw Error(QW_ERR_HIP, "HipEngine: hipMalloc");
    }
    static void alloc(int*& p, size_t n) {
        if (hipMalloc(&p, n * sizeof(int)) != hipSuccess) throw Error(QW_ERR_HIP, "HipEngine: hipMalloc");
    }
    static float* upload(const float* h, size_t n) {
        float* d = nullptr;
        alloc(d, n);
        if (hipMemcpy(d, h, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            throw Error(QW_ERR_HIP, "HipEngine: upload");
        return d;
    }
    detail::WeightPtr pack_ptr(const float* w, int N, int K, const char* name) {
        qw_weight* out = nullptr;
        ctx_->check(qw_weight_pack(ctx_->get(), w, QW_F32, fmt_, N, K, nullptr, &out), name);
        return detail::WeightPtr(out);
    }
    static void free_layer(Layer& L) {
        for (void* p : {(void*)L.in_norm, (void*)L.post_norm, (void*)L.conv, (void*)L.A_log, (void*)L.dt_bias,
                        (void*)L.norm_w, (void*)L.conv_state, (void*)L.rec_state, (void*)L.q_norm, (void*)L.k_norm,
                        L.kc, L.vc, (void*)L.ks, (void*)L.vs})
            if (p) (void)hipFree(p);
        const bool linear = L.linear;
        L = Layer{};
        L.linear = linear;
    }

    int nl_, H_, I_, V_, max_seq_;
    qw_wfmt fmt_;
    bool kv_int8_;
    std::shared_ptr<Context> ctx_;
    std::vector<Layer> layers_;
    std::unique_ptr<HipLMHead> lm_head_;
    float *d_x_ = nullptr, *d_row_ = nullptr, *d_core_ = nullptr, *d_out_ = nullptr, *d_final_norm_ = nullptr;
    int* d_pos_ = nullptr;
    int cap_ = 0, length_ = 0;
};

}  // namespace hip
}  // namespace qwen
