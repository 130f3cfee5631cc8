// Backward-kernel instantiations for one (dtype, head_dim) pair, selected at
// compile time with -DAF_DT=<0 f16 | 1 bf16> -DAF_D=<head_dim>.
#include "bwd_kernel.hpp"
#include "bwd_launch.hpp"

#ifndef AF_DT
#error "compile with -DAF_DT=0|1 -DAF_D=<head_dim>"
#endif

namespace af {

#if AF_DT == 0
using Elem = F16;
#define AF_DT_NAME f16
#else
using Elem = BF16;
#define AF_DT_NAME bf16
#endif

#define AF_FN_(dt, d) launch_bwd_##dt##_d##d
#define AF_FN(dt, d) AF_FN_(dt, d)

namespace {

template <int MASK, int BIAS, bool ROPE, int WK, int WQ>
void go(const BwdParams& p, const BwdGrids& g, hipStream_t s) {
  hipLaunchKernelGGL((bwd_prep_kernel<Elem, AF_D, ROPE>), dim3(g.prep), dim3(256), 0, s, p);
  if constexpr (AF_D == 256 && BIAS == BIAS_ALIBI) {
    // at head dim 256 the ALiBi dK/dV kernels crash the compiler's backend
    // with MFMAs forced into the VGPR form; they are built in
    // bwd_d256_alt.hip, and run as their own launch
    launch_bwd_dkv_d256_alibi(p, AF_DT, MASK, ROPE, WK, dim3(g.dkv), s);
    hipLaunchKernelGGL((bwd_dq_kernel<Elem, AF_D, MASK, BIAS, ROPE, WQ>), dim3(g.dq), dim3(64 * WQ), 0, s, p);
  } else if constexpr (WK == WQ && !(AF_D == 128 && BIAS == BIAS_ALIBI)) {
    // dK/dV and dQ in one launch, dK/dV workgroups first.  Not with ALiBi at
    // head dim 128: the dQ side then needs more than the 256 registers of
    // two waves per SIMD, at which the dK/dV side runs alone (fused at two
    // waves it spills 40-54 registers).
    BwdParams q = p;
    q.n_dkv_wg = (int32_t)g.dkv;
    hipLaunchKernelGGL((bwd_dkvdq_kernel<Elem, AF_D, MASK, BIAS, ROPE, WK>), dim3(g.dkv + g.dq), dim3(64 * WK), 0,
                       s, q);
  } else {
    hipLaunchKernelGGL((bwd_dkv_kernel<Elem, AF_D, MASK, BIAS, ROPE, WK>), dim3(g.dkv), dim3(64 * WK), 0, s, p);
    hipLaunchKernelGGL((bwd_dq_kernel<Elem, AF_D, MASK, BIAS, ROPE, WQ>), dim3(g.dq), dim3(64 * WQ), 0, s, p);
  }
  if (g.combine > 0)
    hipLaunchKernelGGL((bwd_dkv_combine_kernel<Elem, AF_D, ROPE>), dim3(g.combine), dim3(256), 0, s, p);
}

template <int MASK, int BIAS, bool ROPE>
int pick_waves(const BwdParams& p, const BwdGrids& g, hipStream_t s) {
  if constexpr (kIsBs<MASK>) {
    if (g.waves_kv == 2 && g.waves_q == 2) { go<MASK, BIAS, ROPE, 2, 2>(p, g, s); return 0; }
    if (g.waves_kv == 2 && g.waves_q == 4) { go<MASK, BIAS, ROPE, 2, 4>(p, g, s); return 0; }
    if (g.waves_kv == 4 && g.waves_q == 2) { go<MASK, BIAS, ROPE, 4, 2>(p, g, s); return 0; }
    if (g.waves_kv == 4 && g.waves_q == 4) { go<MASK, BIAS, ROPE, 4, 4>(p, g, s); return 0; }
    return -1;
  } else {
    if (g.waves_kv != 4 || g.waves_q != 4) return -1;
    go<MASK, BIAS, ROPE, 4, 4>(p, g, s);
    return 0;
  }
}

template <int MASK, int BIAS>
int pick_rope(const BwdParams& p, int rope, const BwdGrids& g, hipStream_t s) {
  return rope ? pick_waves<MASK, BIAS, true>(p, g, s) : pick_waves<MASK, BIAS, false>(p, g, s);
}

template <int MASK>
int pick_bias(const BwdParams& p, int bias, int rope, const BwdGrids& g, hipStream_t s) {
  if (bias == BIAS_NONE) return pick_rope<MASK, BIAS_NONE>(p, rope, g, s);
  if (bias == BIAS_ALIBI) return pick_rope<MASK, BIAS_ALIBI>(p, rope, g, s);
  return -1;
}

}  // namespace

int AF_FN(AF_DT_NAME, AF_D)(const BwdParams& p, int mask, int bias, int rope, const BwdGrids& g,
                           hipStream_t s) {
  switch (mask) {
    case MASK_FULL: return pick_bias<MASK_FULL>(p, bias, rope, g, s);
    case MASK_CAUSAL: return pick_bias<MASK_CAUSAL>(p, bias, rope, g, s);
    case MASK_SW: return pick_bias<MASK_SW>(p, bias, rope, g, s);
    case MASK_BS: return pick_bias<MASK_BS>(p, bias, rope, g, s);
#if AF_D <= 128
    case MASK_BSE: return pick_bias<MASK_BSE>(p, bias, rope, g, s);
#endif
    case MASK_CSW: return pick_bias<MASK_CSW>(p, bias, rope, g, s);
    default: return -1;
  }
}

}  // namespace af
