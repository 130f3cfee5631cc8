// Backward launch declarations shared by the instantiation units and the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "attnfuse_hip.h"
#include "bwd_kernel.hpp"

namespace af {

struct BwdGrids {
  unsigned delta, dkv, dq;
  int waves_kv, waves_q;
};

size_t bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q);
int run_bwd(const af_bwd_args* a, const af_blockmask* bm, void* workspace, size_t workspace_bytes,
            hipStream_t stream);

#define AF_DECLARE_BWD(NAME) \
  int NAME(const BwdParams& p, int mask, int bias, int rope, const BwdGrids& g, hipStream_t s);
AF_DECLARE_BWD(launch_bwd_f16_d32)
AF_DECLARE_BWD(launch_bwd_f16_d64)
AF_DECLARE_BWD(launch_bwd_f16_d128)
AF_DECLARE_BWD(launch_bwd_bf16_d32)
AF_DECLARE_BWD(launch_bwd_bf16_d64)
AF_DECLARE_BWD(launch_bwd_bf16_d128)
#undef AF_DECLARE_BWD

}  // namespace af
