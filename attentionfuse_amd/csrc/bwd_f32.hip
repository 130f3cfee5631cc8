// Launch sequence of the fp32 backward (bwd_f32_kernel.hpp): RoPE of q and k
// into the workspace, the per-row prep, then the dK/dV and dQ workgroups
// (one launch when both use the same workgroup width) and the sum of the
// group-split dK/dV partials.
#include "attnfuse_hip.h"
#include "bwd_f32_kernel.hpp"
#include "launch.hpp"

namespace af {

// wkv / wq: waves of the dK/dV and dQ workgroups (4; with a block mask the
// mask's block sizes / 32, 2 or 4)
template <int D>
static void launch_bwd_f32_d(BwdParams p, int mask, int bias, int rope, int wkv, int wq, hipStream_t s) {
  const int64_t rows_q = (int64_t)p.B * p.Hq * p.Nq;
  if (rows_q > 0)
    hipLaunchKernelGGL((bwd_prep_f32_kernel<D>), dim3((unsigned)((rows_q + 255) / 256)), dim3(256), 0, s, p);
  const unsigned grid_kv = (unsigned)(p.n_kblocks * p.g_split * p.B * p.Hkv);
  const unsigned grid_q = (unsigned)(p.n_qblocks * p.B * p.Hq);
  if (wkv == wq && grid_kv > 0 && grid_q > 0) {
    // dK/dV and dQ workgroups in one launch, dK/dV first
    BwdParams q = p;
    q.n_dkv_wg = (int32_t)grid_kv;
    if (wkv == 2)
      hipLaunchKernelGGL((bwd_dkvdq_f32_kernel<D, 2>), dim3(grid_kv + grid_q), dim3(128), 0, s, q, mask, bias, rope);
    else
      hipLaunchKernelGGL((bwd_dkvdq_f32_kernel<D, 4>), dim3(grid_kv + grid_q), dim3(256), 0, s, q, mask, bias, rope);
  } else {
    if (grid_kv > 0) {
      if (wkv == 2)
        hipLaunchKernelGGL((bwd_dkv_f32_kernel<D, 2>), dim3(grid_kv), dim3(128), 0, s, p, mask, bias, rope);
      else
        hipLaunchKernelGGL((bwd_dkv_f32_kernel<D, 4>), dim3(grid_kv), dim3(256), 0, s, p, mask, bias, rope);
    }
    if (grid_q > 0) {
      if (wq == 2)
        hipLaunchKernelGGL((bwd_dq_f32_kernel<D, 2>), dim3(grid_q), dim3(128), 0, s, p, mask, bias, rope);
      else
        hipLaunchKernelGGL((bwd_dq_f32_kernel<D, 4>), dim3(grid_q), dim3(256), 0, s, p, mask, bias, rope);
    }
  }
  if (grid_kv > 0 && p.g_split > 1) {
    const int64_t threads = (int64_t)p.B * p.Hkv * p.Nkv * (D / 4);
    hipLaunchKernelGGL((bwd_dkv_combine_f32_kernel<D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p);
  }
}

int launch_bwd_f32(BwdParams p, const af_bwd_args& a, hipStream_t s) {
  const int D = a.key.head_dim;
  const bool bs = a.key.mask == AF_MASK_BLOCK_SPARSE;
  // block-sparse: one workgroup per mask block (p.bs_block_m / _n set by the caller)
  const int bk = bs ? p.bs_block_n : kBwdF32Block, bq = bs ? p.bs_block_m : kBwdF32Block;
  p.n_kblocks = (a.seqlen_kv + bk - 1) / bk;
  p.n_qblocks = (a.seqlen_q + bq - 1) / bq;
  if (a.key.rope) {
    // q~ and k~ (fp32, contiguous) into the workspace copies p.qr / p.kr
    launch_rope_f32(static_cast<const float*>(a.q), reinterpret_cast<float*>(p.qr), static_cast<const float*>(a.cos),
                    static_cast<const float*>(a.sin), a.q_stride, a.rope_stride[0], a.heads_q, a.seqlen_q,
                    (int64_t)a.batch * a.heads_q * a.seqlen_q, D, s);
    launch_rope_f32(static_cast<const float*>(a.k), reinterpret_cast<float*>(p.kr), static_cast<const float*>(a.cos),
                    static_cast<const float*>(a.sin), a.k_stride, a.rope_stride[0], a.heads_kv, a.seqlen_kv,
                    (int64_t)a.batch * a.heads_kv * a.seqlen_kv, D, s);
  }
  const int wkv = bk / 32, wq = bq / 32;
  switch (D) {
    case 32: launch_bwd_f32_d<32>(p, a.key.mask, a.key.bias, a.key.rope, wkv, wq, s); return 0;
    case 64: launch_bwd_f32_d<64>(p, a.key.mask, a.key.bias, a.key.rope, wkv, wq, s); return 0;
    case 128: launch_bwd_f32_d<128>(p, a.key.mask, a.key.bias, a.key.rope, wkv, wq, s); return 0;
  }
  return -1;
}

}  // namespace af
