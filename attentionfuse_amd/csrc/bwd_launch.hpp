// Backward entry points shared by the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "attnfuse_hip.h"

namespace af {
size_t bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q);
int run_bwd(const af_bwd_args* a, const af_blockmask* bm, void* workspace,
            size_t workspace_bytes, hipStream_t stream);
}  // namespace af
