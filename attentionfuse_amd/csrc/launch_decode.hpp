// Decode launcher declarations shared by decode_inst.hip and the C ABI
// entry points (api.hip, decode_noalloc.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "attnfuse_hip.h"
#include "decode_kernel.hpp"

namespace af {
// Enqueue split + combine.  Returns 0, or -1 when (dtype, d, bias) has no
// instantiation.
int launch_decode(const DecodeParams& p, int dtype, int d, int bias, dim3 gs,
                  dim3 gc, hipStream_t s);

// Validate a decode call and fill every DecodeParams field except the
// workspace pointers; *need = partial-sum bytes for the split count chosen.
// max_ws > 0 caps those bytes: a library-chosen split count is lowered to
// fit, an explicit one that does not fit is an AF_ERR_WORKSPACE error.
int plan_decode(const af_decode_args* a, size_t max_ws, DecodeParams* p, size_t* need);
// Point p at `workspace` and enqueue the split and combine kernels.
int enqueue_decode(DecodeParams& p, const af_decode_args* a, void* workspace, hipStream_t s);
}  // namespace af
