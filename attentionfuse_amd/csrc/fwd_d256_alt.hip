// One forward instantiation built apart from fwd_inst.hip: bf16, head dim
// 256, causal mask, additive bias, ReLU normalisation, fused RoPE.  With the
// MFMA operands forced into the VGPR form (the flag every other unit uses)
// the compiler's backend crashes on it; this unit keeps the compiler's own
// choice of register form.
#include "launch.hpp"

namespace af {

void launch_fwd_bf16_d256_causal_add_relu_rope(const FwdParams& p, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((fwd_kernel<BF16, 256, MASK_CAUSAL, BIAS_ADD, NORM_RELU, true, 4>), grid, dim3(256), 0, stream,
                     p);
}

}  // namespace af
