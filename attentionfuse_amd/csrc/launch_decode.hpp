// Decode launcher declaration shared by decode_inst.hip and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "decode_kernel.hpp"

namespace af {
// Enqueue split + combine.  Returns 0, or -1 when (dtype, d, bias) has no
// instantiation.
int launch_decode(const DecodeParams& p, int dtype, int d, int bias, dim3 gs,
                  dim3 gc, hipStream_t s);
}  // namespace af
