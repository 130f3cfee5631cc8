// The ALiBi dK/dV kernels at head dim 256, built apart from bwd_inst.hip:
// with the MFMA operands forced into the VGPR form (the flag the other units
// use) the compiler's backend crashes on several of them; this unit keeps the
// compiler's own choice of register form.
#include "bwd_launch.hpp"

namespace af {

namespace {
template <class E, int MASK, bool ROPE, int W>
void go(const BwdParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((bwd_dkv_kernel<E, 256, MASK, BIAS_ALIBI, ROPE, W>), grid, dim3(64 * W), 0, s, p);
}
template <class E, int MASK>
int pick(const BwdParams& p, bool rope, int waves, dim3 grid, hipStream_t s) {
  if (waves == 4) {
    rope ? go<E, MASK, true, 4>(p, grid, s) : go<E, MASK, false, 4>(p, grid, s);
    return 0;
  }
  if constexpr (MASK == MASK_BS) {
    if (waves == 2) {
      rope ? go<E, MASK, true, 2>(p, grid, s) : go<E, MASK, false, 2>(p, grid, s);
      return 0;
    }
  }
  return -1;
}
template <class E>
int pick_mask(const BwdParams& p, int mask, bool rope, int waves, dim3 grid, hipStream_t s) {
  switch (mask) {
    case MASK_FULL: return pick<E, MASK_FULL>(p, rope, waves, grid, s);
    case MASK_CAUSAL: return pick<E, MASK_CAUSAL>(p, rope, waves, grid, s);
    case MASK_SW: return pick<E, MASK_SW>(p, rope, waves, grid, s);
    case MASK_BS: return pick<E, MASK_BS>(p, rope, waves, grid, s);
    case MASK_CSW: return pick<E, MASK_CSW>(p, rope, waves, grid, s);
    default: return -1;
  }
}
}  // namespace

int launch_bwd_dkv_d256_alibi(const BwdParams& p, int dtype, int mask, bool rope, int waves, dim3 grid,
                              hipStream_t s) {
  return dtype == 0 ? pick_mask<F16>(p, mask, rope, waves, grid, s) : pick_mask<BF16>(p, mask, rope, waves, grid, s);
}

}  // namespace af
