// qw_embed.hip -- token-embedding gather and the decode-step position advance.
//
// Gather: out[m][k] = table[ids[m]][k] (the CPU TokenEmbedding row copy,
// src/backend/cpu/core/embedding/token_embedding.cpp; CUDA
// embedding_lookup_batch[_bf16]_kernel, token_embedding_cuda.cu:28-58).  One
// workgroup per row, 16-byte loads; an id outside [0, vocab) writes zeros and
// raises the device error flag.
// Advance: positions[i] += delta, a kernel rather than a memset or copy so
// that a captured decode step can move its own positions on every replay.
#include "qw_stream.hpp"

namespace qwk {

__global__ __launch_bounds__(256) void embed_gather_kernel(const void* table, int tdt, int vocab, int K,
                                                           const int32_t* ids, void* out, int odt, int ld_out,
                                                           unsigned* err) {
    const int m = blockIdx.x;
    const int id = ids[m];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0) *err = 1u;
    const int64_t src = (int64_t)(ok ? id : 0) * K;
    const int64_t dst = (int64_t)m * ld_out;
    for (int k = threadIdx.x * 4; k < K; k += 256 * 4) {
        f32x4 v = ok ? load_act4(table, tdt, src + k) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        store_act4(out, odt, dst + k, v);
    }
}

__global__ __launch_bounds__(256) void positions_add_kernel(int32_t* pos, int n, int delta) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) pos[i] += delta;
}

hipError_t launch_embed_gather(const void* table, int tdt, int vocab, int K, const int32_t* ids, int M, void* out,
                               int odt, int ld_out, unsigned* err, hipStream_t stream) {
    hipLaunchKernelGGL(embed_gather_kernel, dim3(M), dim3(256), 0, stream, table, tdt, vocab, K, ids, out, odt, ld_out,
                       err);
    return hipGetLastError();
}

hipError_t launch_positions_add(int32_t* pos, int n, int delta, hipStream_t stream) {
    hipLaunchKernelGGL(positions_add_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, pos, n, delta);
    return hipGetLastError();
}

}  // namespace qwk
