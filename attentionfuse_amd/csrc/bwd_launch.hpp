// Backward launch declarations shared by the instantiation units and the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "attnfuse_hip.h"
#include "bwd_kernel.hpp"

namespace af {

struct BwdGrids {
  unsigned prep, dkv, dq, combine;   // combine: 0 unless the dK/dV head groups are split
  int waves_kv, waves_q;
};

// Workspace layout: (L log2 e, delta) fp32 pairs (B*Hq*Nq), then with RoPE
// q~ (B*Hq*Nq*D) and k~ (B*Hkv*Nkv*D) in the input dtype, then with a
// head-group split the fp32 dK and dV partials (g_split*B*Hkv*Nkv*D each);
// each section 256-byte aligned.
// With a block mask's work plans, the fp32 partials of split lists follow:
// dQ rows (Q-major slots, B*Hq, BLOCK_M, D), then dK and dV rows (K-major
// slots, B*Hkv, BLOCK_N, D) each.
struct BwdWorkspace {
  size_t ld, qr, kr, dkp, dvp, pdq, pdk, pdv, total;   // byte offsets and size
  int g_split;
  bool q_plan, kv_plan;   // the dQ / dK-dV launches walk the mask's plans
};
// Workgroups of the dK/dV kernel per key block and key/value head: the
// query heads of a group are split (a power of two dividing G) while the
// grid stays within two workgroups per CU (512), so that a causal mask's
// long key blocks do not leave most CUs idle.  Measured at config 5 (256
// workgroups unsplit, one per CU): backward 1153 us unsplit, 796 us split 4
// ways, 773 us split 2 ways; at B = 2 (512 workgroups) splitting lost.  The
// fp32 kernels use the same rule: with dK/dV and dQ in one launch, config 5
// in fp32 takes 8.97 ms unsplit, 6.38-6.39 ms split 2 ways, 6.44 ms 4 ways.
// The args' group_split when it is set, else the choice described above.
int bwd_group_split(const af_bwd_args& a);
bool group_split_valid(const af_bwd_args& a);
// The split the launch uses: 1 for a block mask whose K-major plan splits
// columns (unless the caller sets group_split), else bwd_group_split.
int bwd_group_split_for(const af_bwd_args& a, const af_blockmask* bm);
BwdWorkspace bwd_workspace_layout(const af_bwd_args& a, const af_blockmask* bm = nullptr);
size_t bwd_workspace_bytes(const af_bwd_args& a, const af_blockmask* bm = nullptr);
int run_bwd(const af_bwd_args* a, const af_blockmask* bm, void* workspace, size_t workspace_bytes,
            hipStream_t stream);

// dK/dV with ALiBi at head dim 256 (any dtype code 0/1, mask, rope, 2 or 4
// waves), built in bwd_d256_alt.hip with the compiler's default MFMA
// register form.  Returns -1 for a combination it does not hold.
int launch_bwd_dkv_d256_alibi(const BwdParams& p, int dtype, int mask, bool rope, int waves, dim3 grid,
                              hipStream_t s);

#define AF_DECLARE_BWD(NAME) \
  int NAME(const BwdParams& p, int mask, int bias, int rope, const BwdGrids& g, hipStream_t s);
AF_DECLARE_BWD(launch_bwd_f16_d32)
AF_DECLARE_BWD(launch_bwd_f16_d64)
AF_DECLARE_BWD(launch_bwd_f16_d128)
AF_DECLARE_BWD(launch_bwd_f16_d256)
AF_DECLARE_BWD(launch_bwd_bf16_d32)
AF_DECLARE_BWD(launch_bwd_bf16_d64)
AF_DECLARE_BWD(launch_bwd_bf16_d128)
AF_DECLARE_BWD(launch_bwd_bf16_d256)
#undef AF_DECLARE_BWD

}  // namespace af
