// qw_noalloc.hip -- qw_lmhead_argmax_noalloc: the tied lm_head + greedy argmax
// for callers that cannot allocate device memory (code under graph capture,
// serving loops, harnesses that forbid hipMalloc).  The argmax keys and the
// completion counter live in a file-scope device array instead of a qw_ctx
// workspace; the launch is the one qw_lmhead_argmax makes (same kernels, same
// routes as a default context).
//
// The array is per device (each GPU that loads the library holds its own copy
// until the process ends).  Host code never passes the array's name to a
// kernel: at the first call on a device, with that device current, its device
// address is looked up with hipGetSymbolAddress and kept per device.  The
// loader zero-fills the array and every launch returns the keys and the
// counter to zero; the first call on a device also zero-fills them with a
// kernel on the caller's stream (a kernel rather than a memset, so that a
// capturing caller records no memset node).  Calls that overlap on one device
// share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/qw_linear.h"
#include "qw_internal.hpp"

namespace {

constexpr int kNoallocMaxM = 256;     // argmax keys, one per token
constexpr int kDoneWord = kNoallocMaxM;  // the completion counter, on its own 256-byte line
constexpr int kScratchWords = kNoallocMaxM + 32;

__device__ __align__(256) unsigned long long scratch[kScratchWords];

constexpr int kMaxDevices = 64;
unsigned long long* g_scratch[kMaxDevices];
std::once_flag g_once[kMaxDevices];
hipError_t g_setup_err[kMaxDevices];
bool g_cleared[kMaxDevices];
std::mutex g_clear_mu;

__global__ void zero_scratch_kernel(unsigned long long* p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0ull;
}

hipError_t setup(int device) {
    std::call_once(g_once[device], [device] {
        void* ptr = nullptr;
        g_setup_err[device] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch[device] = static_cast<unsigned long long*>(ptr);
    });
    return g_setup_err[device];
}

}  // namespace

extern "C" qw_status qw_lmhead_argmax_noalloc(const void* E_packed, const float* E_scales, qw_wfmt fmt, int V,
                                              int K, const void* h, qw_dtype hdt, int M, int32_t* token_ids,
                                              float* max_logit, hipStream_t stream) {
    if (M < 1 || M > kNoallocMaxM) return QW_ERR_SHAPE;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return QW_ERR_HIP;
    if (setup(device) != hipSuccess || !g_scratch[device]) return QW_ERR_HIP;
    unsigned long long* keys = g_scratch[device];
    {
        std::lock_guard<std::mutex> lk(g_clear_mu);
        if (!g_cleared[device]) {
            hipLaunchKernelGGL(zero_scratch_kernel, dim3(1), dim3(256), 0, stream, keys, kScratchWords);
            if (hipGetLastError() != hipSuccess) return QW_ERR_HIP;
            g_cleared[device] = true;
        }
    }
    unsigned* done = reinterpret_cast<unsigned*>(keys + kDoneWord);
    return qwi::lmhead_argmax_scratch(device, E_packed, E_scales, fmt, V, K, h, hdt, M, token_ids, max_logit, keys,
                                      done, stream);
}
