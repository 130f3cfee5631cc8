// Forward-kernel instantiations for one (dtype, head_dim) pair, selected at
// compile time with -DAF_DT=<0 f16 | 1 bf16> -DAF_D=<head_dim>.  Splitting
// the instantiations over several objects keeps each compile short and lets
// the build run them in parallel.
#include "launch.hpp"

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

#define AF_FN_(dt, d) launch_fwd_##dt##_d##d
#define AF_FN(dt, d) AF_FN_(dt, d)
#define AF_RFN_(dt, d) launch_rope_##dt##_d##d
#define AF_RFN(dt, d) AF_RFN_(dt, d)

namespace {

// bf16, head dim 256, causal + additive bias + ReLU + RoPE crashes the
// compiler's backend when MFMAs are forced into the VGPR form; that one
// kernel is built in fwd_d256_alt.hip without the flag.
constexpr bool alt_unit(int mask, int bias, int norm, bool rope, int waves) {
  return AF_DT == 1 && AF_D == 256 && mask == MASK_CAUSAL && bias == BIAS_ADD && norm == NORM_RELU && rope &&
         waves == 4;
}

template <int MASK, int BIAS, int NORM, bool ROPE, int WAVES>
int go(const FwdParams& p, dim3 grid, hipStream_t s) {
  if constexpr (alt_unit(MASK, BIAS, NORM, ROPE, WAVES)) {
    launch_fwd_bf16_d256_causal_add_relu_rope(p, grid, s);
  } else {
    hipLaunchKernelGGL((fwd_kernel<Elem, AF_D, MASK, BIAS, NORM, ROPE, WAVES>),
                       grid, dim3(64 * WAVES), 0, s, p);
  }
  return 0;
}

template <int MASK, int BIAS, int NORM, bool ROPE>
int pick_waves(const FwdParams& p, int waves, dim3 grid, hipStream_t s) {
  if constexpr (kIsBs<MASK>) {
    switch (waves) {
      case 1: return go<MASK, BIAS, NORM, ROPE, 1>(p, grid, s);
      case 2: return go<MASK, BIAS, NORM, ROPE, 2>(p, grid, s);
      case 4: return go<MASK, BIAS, NORM, ROPE, 4>(p, grid, s);
      default: return -1;
    }
  } else {
    if (waves != 4) return -1;
    return go<MASK, BIAS, NORM, ROPE, 4>(p, grid, s);
  }
}

template <int MASK, int BIAS, int NORM>
int pick_rope(const FwdParams& p, int rope, int waves, dim3 grid, hipStream_t s) {
  return rope ? pick_waves<MASK, BIAS, NORM, true>(p, waves, grid, s)
              : pick_waves<MASK, BIAS, NORM, false>(p, waves, grid, s);
}

template <int MASK, int BIAS>
int pick_norm(const FwdParams& p, int norm, int rope, int waves, dim3 grid, hipStream_t s) {
  switch (norm) {
    case NORM_SOFTMAX: return pick_rope<MASK, BIAS, NORM_SOFTMAX>(p, rope, waves, grid, s);
    case NORM_RELU: return pick_rope<MASK, BIAS, NORM_RELU>(p, rope, waves, grid, s);
    default: return -1;
  }
}

template <int MASK>
int pick_bias(const FwdParams& p, int bias, int norm, int rope, int waves, dim3 grid, hipStream_t s) {
  switch (bias) {
    case BIAS_NONE: return pick_norm<MASK, BIAS_NONE>(p, norm, rope, waves, grid, s);
    case BIAS_ALIBI: return pick_norm<MASK, BIAS_ALIBI>(p, norm, rope, waves, grid, s);
    case BIAS_ADD: return pick_norm<MASK, BIAS_ADD>(p, norm, rope, waves, grid, s);
    default: return -1;
  }
}

}  // namespace

int AF_FN(AF_DT_NAME, AF_D)(const FwdParams& p, int mask, int bias, int norm,
                           int rope, int waves, dim3 grid, hipStream_t s) {
  switch (mask) {
    case MASK_FULL: return pick_bias<MASK_FULL>(p, bias, norm, rope, waves, grid, s);
    case MASK_CAUSAL: return pick_bias<MASK_CAUSAL>(p, bias, norm, rope, waves, grid, s);
    case MASK_SW: return pick_bias<MASK_SW>(p, bias, norm, rope, waves, grid, s);
    case MASK_BS: return pick_bias<MASK_BS>(p, bias, norm, rope, waves, grid, s);
#if AF_D <= 128
    case MASK_BSE: return pick_bias<MASK_BSE>(p, bias, norm, rope, waves, grid, s);
#endif
    case MASK_CSW: return pick_bias<MASK_CSW>(p, bias, norm, rope, waves, grid, s);
    default: return -1;
  }
}

// Heads per thread, measured on MI355X with the kernel launched back to back:
// 4 rotates config 2's keys (fp16, D=64, 12 heads) in 8.7-8.8 us against
// 9.1-9.2 us for one head per thread (8 per thread: 16.4 us); at D=128 (bf16,
// 8 heads) 2 is best, 3.79 against 3.92-3.98 us.  Between forward launches,
// whose reads evict the keys from the last-level cache, config 2's rotation
// takes 9.76 us with 4 heads per thread and 9.78 us with one.
int AF_RFN(AF_DT_NAME, AF_D)(const RopeRowsParams& p, hipStream_t s) {
  constexpr int HG = AF_D >= 128 ? 2 : 4;
  constexpr int rows_per_block = 256 / (AF_D / 16);
  if (p.rows <= 0 || p.H <= 0 || p.N <= 0) return 0;
  const int64_t batch = p.rows / ((int64_t)p.H * p.N);
  const int64_t blocks = (p.N + rows_per_block - 1) / rows_per_block * ((p.H + HG - 1) / HG) * batch;
  if (blocks <= 0) return 0;
  hipLaunchKernelGGL((rope_rows_kernel<Elem, AF_D, HG>), dim3((unsigned)blocks), dim3(256), 0, s, p);
  return 0;
}

}  // namespace af
