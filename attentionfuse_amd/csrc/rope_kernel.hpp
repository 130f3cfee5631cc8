// Rotate-half RoPE of whole rows, written once to a contiguous buffer.
//
// x~[d]       = x[d] cos[n][d]       - x[d + D/2] sin[n][d]
// x~[d + D/2] = x[d + D/2] cos[n][d + D/2] + x[d] sin[n][d + D/2]
// rounded to the input dtype (reference: attnfuse/compiler/codegen.py:126-135
// rotates the q and k tiles in registers and rounds them before Q K^T).
//
// The forward kernel rotates its query rows in registers (each is read once
// per workgroup), but every key row is read by all query blocks of its head:
// rotating it there repeats the rotation, and the cos/sin reads, once per
// query block.  rope_rows_kernel rotates each key row exactly once instead;
// the forward then streams k~ straight into LDS.
#pragma once

#include "af_common.hpp"

namespace af {

struct RopeRowsParams {
  const uint16_t* x;      // (B, H, N, D), unit d-stride
  uint16_t* out;          // (B, H, N, D) contiguous
  const uint16_t* cos;    // (>= N, D) tables, row stride rs
  const uint16_t* sin;
  int64_t xs[3];          // batch, head and row strides of x (elements)
  int64_t rs;
  int64_t rows;           // B * H * N
  int32_t H, N;
};

// Thread j of a row rotates the rotate-half pair (chunk j, chunk j + D/16).
template <class E, int D>
__device__ __forceinline__ void rope_row_chunk(const uint16_t* x, const uint16_t* cr, const uint16_t* sr,
                                               uint16_t* out, int j) {
  const int dl = 8 * j, dh = dl + D / 2;
  u32x4 lo = ld16(x + dl), hi = ld16(x + dh);
  rope_pair<E>(lo, hi, ld16(cr + dl), ld16(sr + dl), ld16(cr + dh), ld16(sr + dh));
  st16(out + dl, lo);
  st16(out + dh, hi);
}

// A workgroup covers RPB consecutive positions n of one batch entry b and the
// heads [h0, h0 + HG): thread j of a row rotates chunk pair j of position n
// for each of those heads, so one cos/sin read serves HG rows and HG rows'
// loads are in flight at once.  Workgroup index = (b * ceil(H/HG) + h0/HG) *
// ceil(N/RPB) + n/RPB.
template <class E, int D, int HG>
__global__ void __launch_bounds__(256) rope_rows_kernel(const RopeRowsParams p) {
  constexpr int TPR = D / 16;          // threads per row
  constexpr int RPB = 256 / TPR;       // positions per workgroup
  const int tid = threadIdx.x, j = tid % TPR;
  const int nblocks = (p.N + RPB - 1) / RPB, hgroups = (p.H + HG - 1) / HG;
  const int n = (int)(blockIdx.x % nblocks) * RPB + tid / TPR;
  if (n >= p.N) return;
  const int hb = (int)(blockIdx.x / nblocks);
  const int h0 = (hb % hgroups) * HG, b = hb / hgroups;
  const int dl = 8 * j, dh = dl + D / 2;
  const uint16_t* x = p.x + b * p.xs[0] + h0 * p.xs[1] + n * p.xs[2];
  uint16_t* out = p.out + (((int64_t)b * p.H + h0) * p.N + n) * D;
  u32x4 lo[HG], hi[HG];
#pragma unroll
  for (int g = 0; g < HG; ++g)
    if (h0 + g < p.H) {
      lo[g] = ld16(x + g * p.xs[1] + dl);
      hi[g] = ld16(x + g * p.xs[1] + dh);
    }
  const uint16_t* cr = p.cos + n * p.rs;
  const uint16_t* sr = p.sin + n * p.rs;
  const u32x4 clo = ld16(cr + dl), slo = ld16(sr + dl), chi = ld16(cr + dh), shi = ld16(sr + dh);
#pragma unroll
  for (int g = 0; g < HG; ++g)
    if (h0 + g < p.H) {
      rope_pair<E>(lo[g], hi[g], clo, slo, chi, shi);
      st16(out + (int64_t)g * p.N * D + dl, lo[g]);
      st16(out + (int64_t)g * p.N * D + dh, hi[g]);
    }
}

}  // namespace af
