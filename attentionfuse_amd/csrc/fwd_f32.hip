// Launchers of the fp32 forward (fwd_f32_kernel) and its key rotation.
#include "fwd_f32_kernel.hpp"
#include "launch.hpp"

namespace af {

int launch_fwd_f32(const FwdF32Params& p, int head_dim, dim3 grid, hipStream_t s) {
  switch (head_dim) {
    case 32: hipLaunchKernelGGL((fwd_f32_kernel<32>), grid, dim3(kF32Waves * 64), 0, s, p); return 0;
    case 64: hipLaunchKernelGGL((fwd_f32_kernel<64>), grid, dim3(kF32Waves * 64), 0, s, p); return 0;
    case 128: hipLaunchKernelGGL((fwd_f32_kernel<128>), grid, dim3(kF32Waves * 64), 0, s, p); return 0;
  }
  return -1;
}

int launch_rope_f32(const float* x, float* out, const float* cs, const float* sn, const int64_t* xs, int64_t rs,
                    int H, int N, int64_t rows, int head_dim, hipStream_t s) {
  const int64_t threads = rows * (head_dim / 2);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0) return 0;
  switch (head_dim) {
    case 32:
      hipLaunchKernelGGL((rope_f32_kernel<32>), dim3((unsigned)blocks), dim3(256), 0, s, x, out, cs, sn, xs[0], xs[1],
                         xs[2], rs, H, N, rows);
      return 0;
    case 64:
      hipLaunchKernelGGL((rope_f32_kernel<64>), dim3((unsigned)blocks), dim3(256), 0, s, x, out, cs, sn, xs[0], xs[1],
                         xs[2], rs, H, N, rows);
      return 0;
    case 128:
      hipLaunchKernelGGL((rope_f32_kernel<128>), dim3((unsigned)blocks), dim3(256), 0, s, x, out, cs, sn, xs[0],
                         xs[1], xs[2], rs, H, N, rows);
      return 0;
  }
  return -1;
}

}  // namespace af
