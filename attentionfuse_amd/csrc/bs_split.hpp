// Split block-sparse walks: the combine kernels that merge the partial
// results of a row (or column) cut into pieces by af_blockmask_plan.
//
// A BigBird-style mask has a few lists as long as the whole grid (the global
// query block visits every key block; every query block visits the global
// key block) next to many short ones.  Walked by one workgroup each, those
// lists finish long after the rest of the grid.  The plan cuts them into
// near-equal pieces, each a workgroup of its own that writes fp32 partials:
//  * forward: unnormalised O and (running max m in log2 units, row sum l);
//    merged as O = sum_i 2^(m_i - M) O_i / sum_i 2^(m_i - M) l_i with
//    M = max_i m_i, LSE = (M + log2 sum_i 2^(m_i - M) l_i) ln 2;
//  * backward: dQ~ (dK~, dV) partial sums, which add linearly; the sum is
//    scaled and, with RoPE, rotated back like the unsplit kernels' epilogue.
#pragma once

#include <hip/hip_runtime.h>

#include "af_common.hpp"

namespace af {

struct BsFwdCombineParams {
  const int32_t* splits;  // (n_splits, 3): row block, first slot, slots
  const float* part_o;    // (slots, B*H, BM, D)
  const float* part_ml;   // (slots, B*H, BM, 2)
  uint16_t* o;
  float* lse;             // nullable
  int64_t os[4], ls[3];
  int32_t B, H, Nq, BM;
  int32_t softmax;        // 0: ReLU normalisation (no log-sum-exp)
};

// One gradient tensor whose split lists are summed: dQ (query rows) or dK,
// dV (key rows).
struct BsGradTarget {
  const int32_t* splits;  // (n_splits, 3): list, first slot, slots
  const float* part;      // (slots, B*H, BLK, D)
  uint16_t* out;          // rows (b, h, n) at os[0], os[1], os[2]
  int64_t os[3];
  int32_t H, N, BLK, n_splits;
  float scale;
  int32_t rope;           // rotate back with the RoPE tables (dQ, dK)
  int32_t wg0;            // first workgroup of this tensor in the grid
};

struct BsGradCombineParams {
  BsGradTarget t[3];
  int32_t n_targets, B;
  const uint16_t* cos;    // RoPE tables, row stride rs
  const uint16_t* sin;
  int64_t rs;
};

// Partial rows whose loads are issued together before any is used: the
// slots of a split are read in batches of this many, not one dependent load
// after another.
constexpr int kCombineBatch = 8;

// One thread per 8 dims of a row: forward pieces of split row blocks,
// merged batch by batch with the running (M, L, acc) rescaled like the
// online softmax.
template <class E, int D>
__global__ void __launch_bounds__(256) bs_fwd_combine_kernel(const BsFwdCombineParams p) {
  constexpr int TPR = D / 8;
  constexpr int RPB = 256 / TPR;
  constexpr int KB = kCombineBatch;
  const int BH = p.B * p.H;
  const int per = (p.BM + RPB - 1) / RPB;  // workgroups per (split, head)
  const int chunk = blockIdx.x % per;
  const int sbh = blockIdx.x / per;
  const int bh = sbh % BH, si = sbh / BH;
  const int tid = threadIdx.x, j = tid % TPR;
  const int rr = chunk * RPB + tid / TPR;
  const int32_t* sp = p.splits + 3 * si;
  const int mb = sp[0], s0 = sp[1], ns = sp[2];
  const int row = mb * p.BM + rr;
  if (rr >= p.BM || row >= p.Nq) return;
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int i0 = 0; i0 < ns; i0 += KB) {
    f32x2 ml[KB];
    f32x4 lo[KB], hi[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      if (i0 + k < ns) {
        const int64_t r = ((int64_t)(s0 + i0 + k) * BH + bh) * p.BM + rr;
        ml[k] = *reinterpret_cast<const f32x2*>(p.part_ml + 2 * r);
        lo[k] = *reinterpret_cast<const f32x4*>(p.part_o + r * D + 8 * j);
        hi[k] = *reinterpret_cast<const f32x4*>(p.part_o + r * D + 8 * j + 4);
      } else {
        ml[k] = f32x2{-INFINITY, 0.f};
        lo[k] = hi[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // pieces that saw no visible key carry m = -1e30, l = 0, O = 0; slot
    // i0 exists, so Mb is finite and the first rescale multiplies zeros
    float Mb = M;
#pragma unroll
    for (int k = 0; k < KB; ++k) Mb = fmaxf(Mb, ml[k][0]);
    const float r0 = exp2f(M - Mb);
    L *= r0;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= r0;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const float w = exp2f(ml[k][0] - Mb);
      L += w * ml[k][1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] += w * lo[k][e];
        acc[4 + e] += w * hi[k][e];
      }
    }
    M = Mb;
  }
  const float inv = (L == 0.f) ? 1.f : 1.f / L;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= inv;
  const int b = bh / p.H, h = bh - b * p.H;
  st16(p.o + b * p.os[0] + h * p.os[1] + (int64_t)row * p.os[2] + 8 * j, pack8<E>(acc));
  if (p.lse != nullptr && j == 0) {
    float lse = -INFINITY;
    if (p.softmax && L > 0.f) lse = (M + __log2f(L)) * kLn2;
    p.lse[b * p.ls[0] + h * p.ls[1] + (int64_t)row * p.ls[2]] = lse;
  }
}

// One thread per dims [8 j, 8 j + 8) and their rotate-half partners
// [8 j + D/2, ...) of a row: sum of a split list's gradient pieces, scaled
// and (RoPE) rotated back.  The grid holds the workgroups of up to three
// tensors (dQ, dK, dV) one after the other.
template <class E, int D>
__global__ void __launch_bounds__(256) bs_grad_combine_kernel(const BsGradCombineParams p) {
  constexpr int TPR = D / 16;
  constexpr int RPB = 256 / TPR;
  constexpr int KB = kCombineBatch / 2;
  int ti = 0;
  if (p.n_targets > 1 && (int)blockIdx.x >= p.t[1].wg0) ti = 1;
  if (p.n_targets > 2 && (int)blockIdx.x >= p.t[2].wg0) ti = 2;
  const BsGradTarget& T = p.t[ti];
  const int wg = blockIdx.x - T.wg0;
  const int BH = p.B * T.H;
  const int per = (T.BLK + RPB - 1) / RPB;
  const int chunk = wg % per;
  const int sbh = wg / per;
  const int bh = sbh % BH, si = sbh / BH;
  const int tid = threadIdx.x, j = tid % TPR;
  const int rr = chunk * RPB + tid / TPR;
  const int32_t* sp = T.splits + 3 * si;
  const int blk = sp[0], s0 = sp[1], ns = sp[2];
  const int n = blk * T.BLK + rr;
  if (rr >= T.BLK || n >= T.N) return;
  const int dl = 8 * j, dh = dl + D / 2;
  float lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) lo[e] = hi[e] = 0.f;
  for (int i0 = 0; i0 < ns; i0 += KB) {
    f32x4 x[KB][4];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      if (i0 + k < ns) {
        const float* r = T.part + (((int64_t)(s0 + i0 + k) * BH + bh) * T.BLK + rr) * D;
        x[k][0] = *reinterpret_cast<const f32x4*>(r + dl);
        x[k][1] = *reinterpret_cast<const f32x4*>(r + dl + 4);
        x[k][2] = *reinterpret_cast<const f32x4*>(r + dh);
        x[k][3] = *reinterpret_cast<const f32x4*>(r + dh + 4);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) x[k][q] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int k = 0; k < KB; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] += x[k][0][e];
        lo[4 + e] += x[k][1][e];
        hi[e] += x[k][2][e];
        hi[4 + e] += x[k][3][e];
      }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lo[e] *= T.scale;
    hi[e] *= T.scale;
  }
  if (T.rope) {
    float cl[8], sl[8], ch[8], sh[8];
    unpack8<E>(ld16(p.cos + n * p.rs + dl), cl);
    unpack8<E>(ld16(p.sin + n * p.rs + dl), sl);
    unpack8<E>(ld16(p.cos + n * p.rs + dh), ch);
    unpack8<E>(ld16(p.sin + n * p.rs + dh), sh);
#pragma unroll
    for (int e = 0; e < 8; ++e) rope_grad_pair(lo[e], hi[e], cl[e], sl[e], ch[e], sh[e]);
  }
  const int b = bh / T.H, h = bh - b * T.H;
  uint16_t* orow = T.out + b * T.os[0] + h * T.os[1] + (int64_t)n * T.os[2];
  st16(orow + dl, pack8<E>(lo));
  st16(orow + dh, pack8<E>(hi));
}

// Launches (bs_split.hip); dtype 0 = fp16, 1 = bf16.  Return -1 for a head
// dim or dtype without an instantiation.
int launch_bs_fwd_combine(const BsFwdCombineParams& p, int n_splits, int dtype, int head_dim, hipStream_t s);
// Fills the targets' wg0 and launches one grid over all of them.
int launch_bs_grad_combine(BsGradCombineParams& p, int dtype, int head_dim, hipStream_t s);

}  // namespace af
