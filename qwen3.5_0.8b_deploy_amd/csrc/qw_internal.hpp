// qw_internal.hpp -- host-side entry points shared between the C-ABI source
// files (not exported).
#pragma once

#include "../../include/qw_linear.h"

namespace qwi {

// The lm_head + greedy argmax of qw_lmhead_argmax over a packed weight given
// by its device pointers, with the argmax keys [M] and the completion counter
// supplied by the caller (both zero on entry; the kernels return them to
// zero).  Allocates nothing: no context, no workspace.  Routes like a default
// context on `device`.
qw_status lmhead_argmax_scratch(int device, const void* packed, const float* scales, qw_wfmt fmt, int V, int K,
                                const void* h, qw_dtype hdt, int M, int32_t* token_ids, float* max_logit,
                                unsigned long long* keys, unsigned* done, hipStream_t stream);

}  // namespace qwi
