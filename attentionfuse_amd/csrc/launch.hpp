// Host-side launch helpers shared by the instantiation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attnfuse_hip.h"
#include "fwd_kernel.hpp"
#include "rope_kernel.hpp"

namespace af {

// Thread-local error text behind af_last_error().
void set_error(const char* fmt, ...);

// Per-(dtype, head_dim) forward launchers, defined in fwd_inst.hip (one
// object per pair).  `waves` is the workgroup width (32 query rows per wave).
// Return 0, or AF_ERR_UNSUPPORTED when the pair has no instantiation for the
// (mask, bias, norm, rope, waves) combination.
#define AF_DECLARE_FWD(NAME) \
  int NAME(const FwdParams& p, int mask, int bias, int norm, int rope, \
           int waves, dim3 grid, hipStream_t stream);
AF_DECLARE_FWD(launch_fwd_f16_d32)
AF_DECLARE_FWD(launch_fwd_f16_d64)
AF_DECLARE_FWD(launch_fwd_f16_d128)
AF_DECLARE_FWD(launch_fwd_f16_d256)
AF_DECLARE_FWD(launch_fwd_bf16_d32)
AF_DECLARE_FWD(launch_fwd_bf16_d64)
AF_DECLARE_FWD(launch_fwd_bf16_d128)
AF_DECLARE_FWD(launch_fwd_bf16_d256)
#undef AF_DECLARE_FWD

// bf16, head dim 256, causal + additive bias + ReLU + RoPE, built in
// fwd_d256_alt.hip with the compiler's default MFMA register form.
void launch_fwd_bf16_d256_causal_add_relu_rope(const FwdParams& p, dim3 grid, hipStream_t stream);

// rope_rows_kernel launchers, defined next to the forward launchers.
#define AF_DECLARE_ROPE(NAME) int NAME(const RopeRowsParams& p, hipStream_t stream);
AF_DECLARE_ROPE(launch_rope_f16_d32)
AF_DECLARE_ROPE(launch_rope_f16_d64)
AF_DECLARE_ROPE(launch_rope_f16_d128)
AF_DECLARE_ROPE(launch_rope_f16_d256)
AF_DECLARE_ROPE(launch_rope_bf16_d32)
AF_DECLARE_ROPE(launch_rope_bf16_d64)
AF_DECLARE_ROPE(launch_rope_bf16_d128)
AF_DECLARE_ROPE(launch_rope_bf16_d256)
#undef AF_DECLARE_ROPE

// Heads per XCD group of a block-sparse grid over BH heads
// (xcd_head_groups): the largest divisor of BH / 8 whose heads' re-read rows
// (head_bytes each) fit AF_BS_L2_BUDGET bytes, at least 1; 0 (the default
// order) when BH is not a multiple of 8.  An XCD's L2 is 4 MiB and also
// holds the rows read once and the outputs.
#ifndef AF_BS_L2_BUDGET
#define AF_BS_L2_BUDGET (3 << 20)
#endif
inline int bs_xcd_heads(int BH, int64_t head_bytes) {
  if (AF_BS_L2_BUDGET <= 0 || BH <= 0 || BH % 8 != 0) return 0;
  const int per = BH / 8;
  int gh = 1;
  for (int d = 1; d <= per; ++d)
    if (per % d == 0 && (int64_t)d * head_bytes <= (int64_t)AF_BS_L2_BUDGET) gh = d;
  return gh;
}

// fp32 forward and fp32 key rotation, defined in fwd_f32.hip; return -1 for
// a head dim with no instantiation.
struct FwdF32Params;
int launch_fwd_f32(const FwdF32Params& p, int head_dim, dim3 grid, hipStream_t s);
struct BwdParams;
int launch_bwd_f32(BwdParams p, const af_bwd_args& a, hipStream_t s);
int launch_rope_f32(const float* x, float* out, const float* cs, const float* sn, const int64_t* xs, int64_t rs,
                    int H, int N, int64_t rows, int head_dim, hipStream_t s);

}  // namespace af
