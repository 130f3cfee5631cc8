// Decode-kernel instantiations: {f16, bf16} x head_dim {32, 64, 128} x
// {no bias, ALiBi}.
#include "decode_kernel.hpp"
#include "launch_decode.hpp"

namespace af {

namespace {
template <class E, int D, int BIAS>
void go(const DecodeParams& p, dim3 gs, dim3 gc, hipStream_t s) {
  hipLaunchKernelGGL((decode_split_kernel<E, D, BIAS>), gs, dim3(256), 0, s, p);
  hipLaunchKernelGGL((decode_combine_kernel<E, D>), gc, dim3(256), 0, s, p);
}
// fp32: the VALU split kernel, then the combine kernel writing fp32
template <int D, int BIAS>
void go_f32(const DecodeParams& p, dim3 gs, dim3 gc, hipStream_t s) {
  hipLaunchKernelGGL((decode_split_f32_kernel<D, BIAS>), gs, dim3(256), 0, s, p);
  hipLaunchKernelGGL((decode_combine_kernel<F16, D, true>), gc, dim3(256), 0, s, p);
}
template <int D>
int pick_bias_f32(const DecodeParams& p, int bias, dim3 gs, dim3 gc, hipStream_t s) {
  if (bias == 0) { go_f32<D, 0>(p, gs, gc, s); return 0; }
  if (bias == 1) { go_f32<D, 1>(p, gs, gc, s); return 0; }
  return -1;
}
int pick_d_f32(const DecodeParams& p, int d, int bias, dim3 gs, dim3 gc, hipStream_t s) {
  switch (d) {
    case 32: return pick_bias_f32<32>(p, bias, gs, gc, s);
    case 64: return pick_bias_f32<64>(p, bias, gs, gc, s);
    case 128: return pick_bias_f32<128>(p, bias, gs, gc, s);
    default: return -1;
  }
}
template <class E, int D>
int pick_bias(const DecodeParams& p, int bias, dim3 gs, dim3 gc, hipStream_t s) {
  if (bias == 0) { go<E, D, 0>(p, gs, gc, s); return 0; }
  if (bias == 1) { go<E, D, 1>(p, gs, gc, s); return 0; }
  return -1;
}
template <class E>
int pick_d(const DecodeParams& p, int d, int bias, dim3 gs, dim3 gc, hipStream_t s) {
  switch (d) {
    case 32: return pick_bias<E, 32>(p, bias, gs, gc, s);
    case 64: return pick_bias<E, 64>(p, bias, gs, gc, s);
    case 128: return pick_bias<E, 128>(p, bias, gs, gc, s);
    case 256: return pick_bias<E, 256>(p, bias, gs, gc, s);
    default: return -1;
  }
}
}  // namespace

int launch_decode(const DecodeParams& p, int dtype, int d, int bias, dim3 gs,
                  dim3 gc, hipStream_t s) {
  if (dtype == 0) return pick_d<F16>(p, d, bias, gs, gc, s);
  if (dtype == 1) return pick_d<BF16>(p, d, bias, gs, gc, s);
  if (dtype == 2) return pick_d_f32(p, d, bias, gs, gc, s);
  return -1;
}

}  // namespace af
