// fp32 backward: dQ, dK, dV of softmax attention for fp32 inputs, every
// product in fp32 on the fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// The reference runs fp32 backward through Triton dots in TF32, with dQ's
// product cast to bf16 (attnfuse/compiler/codegen_backward.py:287-297), and
// tests it at 2e-2 (tests/test_backward.py:30-33).  The structure follows
// the fp32 forward (fwd_f32_kernel.hpp):
//
//   bwd_prep_f32_kernel  per query row: delta = sum_d dO O and L log2(e)
//                        (0 for a row that sees no key) into the workspace.
//   bwd_dkv_f32_kernel   a wave owns 32 keys.  For every query head of its
//                        group and 32-row query tile, staged once in LDS for
//                        the workgroup's four waves: S = q~ k~^T and
//                        dP = dO v^T with queries as
//                        the MFMA rows, P and dS from the saved L and delta,
//                        dV += P^T dO, dK += dS^T q~.  Register r of lane l
//                        holds query 8(r/4) + 4h + (r mod 4) of key l mod 32
//                        (h = l / 32), which is the query the A operand of
//                        the r-th dV / dK MFMA needs from that lane.
//   bwd_dq_f32_kernel    a wave owns 32 queries; its q~ and dO half rows sit
//                        in registers.  Per 32-key tile, staged once in LDS
//                        for the workgroup's four waves: S^T and dP^T with
//                        keys as the MFMA rows, dS^T, dQ^T += k~^T dS^T.
//
// With a block mask (reference: attnfuse/compiler/codegen_blocksparse_bwd.py:
// 29-233) a workgroup is one mask block (WAVES = block size / 32, 2 or 4):
// dK/dV walk the K-major list of their key block, dQ the Q-major lists of
// their query block, in 32-row tiles of the listed blocks, each visited whole.
//
// Output block c, row m of dV, dK and dQ^T holds d = (D/32) m + c, so a
// lane's operand reads and stores are D/32 consecutive floats.  With RoPE
// the rotated-space gradients are rotated back before the store:
// dx[d] = g[d] cos[d] + g[d + D/2] sin[d + D/2],
// dx[d + D/2] = g[d + D/2] cos[d + D/2] - g[d] sin[d].
#pragma once

#include "af_common.hpp"
#include "bwd_kernel.hpp"
#include "fwd_f32_kernel.hpp"

namespace af {

constexpr int kBwdF32Waves = 4;
constexpr int kBwdF32Block = 32 * kBwdF32Waves;

// One thread per query row r = (b H_q + h) N_q + n.
template <int D>
__global__ void __launch_bounds__(256) bwd_prep_f32_kernel(const BwdParams p) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Nq;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const int n = (int)(r % p.Nq);
  const int64_t bh = r / p.Nq;
  const int hq = (int)(bh % p.Hq), b = (int)(bh / p.Hq);
  const float* o = reinterpret_cast<const float*>(p.o) + b * p.os[0] + hq * p.os[1] + (int64_t)n * p.os[2];
  const float* g = reinterpret_cast<const float*>(p.dout) + b * p.dos[0] + hq * p.dos[1] + (int64_t)n * p.dos[2];
  float delta = 0.f;
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(o + d);
    const f32x4 c = *reinterpret_cast<const f32x4*>(g + d);
    delta += a[0] * c[0] + a[1] * c[1] + a[2] * c[2] + a[3] * c[3];
  }
  const float L = p.lse[b * p.ls[0] + hq * p.ls[1] + (int64_t)n * p.ls[2]];
  p.ld[2 * r] = L == -INFINITY ? 0.f : L * kLog2e;
  p.ld[2 * r + 1] = delta;
}

// Visibility of key j to query i under the dense / causal / windowed masks.
__device__ __forceinline__ bool f32_visible(int mask, int window, int i, int j) {
  if (mask == MASK_CAUSAL) return j <= i;
  if (mask == MASK_SW) return abs(i - j) < window;
  if (mask == MASK_CSW) return j <= i && j > i - window;
  return true;
}

// Rotate-back of a rotated-space gradient pair (lo = d < D/2, hi = d + D/2).
__device__ __forceinline__ void f32_rope_back(float& lo, float& hi, float clo, float slo, float chi, float shi) {
  const float a = lo * clo + hi * shi;
  const float b = hi * chi - lo * slo;
  lo = a;
  hi = b;
}

// LDS of either body: two (32 x (D + 4)) fp32 tiles (q~ and dO rows for
// dK/dV, k~ and v rows for dQ).
template <int D>
using F32Tile = float[32][D + 4];

// dK/dV body of workgroup wg; ql / gl: the two LDS tiles.
template <int D, int WAVES>
__device__ __forceinline__ void bwd_dkv_f32_body(const BwdParams& p, int mask, int bias, int rope, F32Tile<D>& ql,
                                                 F32Tile<D>& gl, int wg) {
  constexpr int DH = D / 2, DC = D / 32;
  constexpr int BLK = 32 * WAVES;
  typedef typename F32Vec<DC>::T VecC;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 31, h = lane >> 5;
  // workgroup = (key block, group split, b, h_kv), key block slowest; split
  // gsi takes query heads [gsi G/g_split, (gsi + 1) G/g_split) of the group
  const int nbh = p.B * p.Hkv;
  const int kb = wg / (nbh * p.g_split);
  const int gsi = (wg / nbh) % p.g_split;
  const int bh = wg % nbh;
  const int b = bh / p.Hkv, hk = bh % p.Hkv;
  const int kw0 = kb * BLK;  // first key of the workgroup
  const int gpw = p.G / p.g_split;
  const int k0 = kw0 + w * 32;

  // Query tiles that can see a key of the workgroup: one range for all four
  // waves (set by the workgroup index only), so every wave runs the same
  // loop and reaches every barrier; a wave whose keys start past N_kv
  // computes masked tiles and stores nothing.
  int q_lo = 0, q_hi = p.Nq;
  if (mask == MASK_CAUSAL) {
    q_lo = kw0;
  } else if (mask == MASK_SW) {
    q_lo = max(0, kw0 - p.window + 1);
    q_hi = min(q_hi, kw0 + BLK - 1 + p.window);
  } else if (mask == MASK_CSW) {
    q_lo = kw0;
    q_hi = min(q_hi, kw0 + BLK - 1 + p.window);
  }
  q_lo &= ~31;
  // query tiles: a range, or the K-major list of this key block (entries of
  // block_m queries, bs_sub tiles each)
  int ntq = q_hi > q_lo ? (q_hi - q_lo + 31) / 32 : 0, bs_sub = 1;
  const int32_t* bs_row = nullptr;
  if (mask == MASK_BS) {
    bs_sub = p.bs_block_m / 32;
    bs_row = p.bs_q_idx + kb * p.bs_q_rs;
    ntq = p.bs_q_num[kb] * bs_sub;
  }

  const float zc = p.scale * kLog2e;
  const int key = k0 + col;  // this lane's key in S and dP
  // k~ and v half rows of this lane's key (clamped; keys >= N_kv are masked)
  const float* krow = reinterpret_cast<const float*>(p.kt) + b * p.kts[0] + hk * p.kts[1] +
                      (int64_t)min(key, p.Nkv - 1) * p.kts[2] + h * DH;
  const float* vrow = reinterpret_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1] +
                      (int64_t)min(key, p.Nkv - 1) * p.vs[2] + h * DH;
  f32x16 dk[DC], dv[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[c][r] = dv[c][r] = 0.f;

  for (int gi = gsi * gpw; gi < (gsi + 1) * gpw; ++gi) {
    const int hq = hk * p.G + gi;
    const float slope = bias == BIAS_ALIBI ? p.slopes[hq] * kLog2e : 0.f;
    const float* qt = reinterpret_cast<const float*>(p.qt) + b * p.qts[0] + hq * p.qts[1];
    const float* dog = reinterpret_cast<const float*>(p.dout) + b * p.dos[0] + hq * p.dos[1];
    const float* ld = p.ld + 2 * ((int64_t)(b * p.Hq + hq) * p.Nq);
    for (int t = 0; t < ntq; ++t) {
      const int q0 = mask == MASK_BS ? bs_row_get(bs_row, ntq, bs_row, t / bs_sub) * p.bs_block_m + (t % bs_sub) * 32
                                     : q_lo + 32 * t;
      __syncthreads();  // every wave is done with the previous tile
      for (int idx = threadIdx.x; idx < 32 * (D / 4); idx += WAVES * 64) {
        const int r = idx / (D / 4), c4 = (idx % (D / 4)) * 4;
        const int n = q0 + r;
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, g = {0.f, 0.f, 0.f, 0.f};
        if (n < p.Nq) {
          a = *reinterpret_cast<const f32x4*>(qt + (int64_t)n * p.qts[2] + c4);
          g = *reinterpret_cast<const f32x4*>(dog + (int64_t)n * p.dos[2] + c4);
        }
        *reinterpret_cast<f32x4*>(&ql[r][c4]) = a;
        *reinterpret_cast<f32x4*>(&gl[r][c4]) = g;
      }
      __syncthreads();
      // S and dP: queries q0 + (l mod 32) as the A rows, d paired across halves
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int j = 0; j < DH / 4; ++j) {
        const f32x4 qa4 = *reinterpret_cast<const f32x4*>(&ql[col][h * DH + 4 * j]);
        const f32x4 ka4 = *reinterpret_cast<const f32x4*>(krow + 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa4[e], ka4[e], s, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < DH / 4; ++j) {
        const f32x4 ga4 = *reinterpret_cast<const f32x4*>(&gl[col][h * DH + 4 * j]);
        const f32x4 va4 = *reinterpret_cast<const f32x4*>(vrow + 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga4[e], va4[e], dp, 0, 0, 0);
      }
      // element mask of a partial block-sparse tile: bits of this lane's key
      // over the tile's 32 queries, shifted by 4 h (constant bit per element)
      uint32_t ebits = ~0u;
      if (mask == MASK_BS && p.bs_col_bits != nullptr) {
        const int e = t / bs_sub;
        if (p.bs_q_partial[kb * p.bs_q_rs + e] != 0) {
          const int sb = t - e * bs_sub;
          const int64_t word = (((int64_t)kb * p.bs_q_rs + e) * p.bs_block_n + (key - kw0)) *
                                   ((p.bs_block_m + 63) / 64) + (sb >> 1);
          ebits = key < p.Nkv ? (uint32_t)(p.bs_col_bits[word] >> (32 * (sb & 1))) >> (4 * h) : 0u;
        }
      }
      // P and dS of query q0 + 8(r/4) + 4h + (r mod 4), key k0 + col
      float pr[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = q0 + 8 * (r >> 2) + 4 * h + (r & 3);
        const f32x2 l2 = *reinterpret_cast<const f32x2*>(ld + 2 * min(qi, p.Nq - 1));
        float x = s[r] * zc - l2[0];
        if (bias == BIAS_ALIBI) x -= slope * (float)abs(qi - key);
        const bool vis = qi < p.Nq && key < p.Nkv && f32_visible(mask, p.window, qi, key) &&
                         (ebits & (1u << (8 * (r >> 2) + (r & 3))));
        pr[r] = vis ? __builtin_amdgcn_exp2f(x) : 0.f;
        ds[r] = pr[r] * (dp[r] - l2[1]);
      }
      // dV += P^T dO and dK += dS^T q~: B operands are the LDS rows of the
      // queries of register i, D/32 consecutive d per lane
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qi = 8 * (i >> 2) + 4 * h + (i & 3);
        const VecC gv = *reinterpret_cast<const VecC*>(&gl[qi][DC * col]);
        const VecC qv = *reinterpret_cast<const VecC*>(&ql[qi][DC * col]);
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          float gc, qc;
          if constexpr (DC == 1) {
            gc = gv;
            qc = qv;
          } else {
            gc = gv[c];
            qc = qv[c];
          }
          dv[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(pr[i], gc, dv[c], 0, 0, 0);
          dk[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[i], qc, dk[c], 0, 0, 0);
        }
      }
    }
  }
  if (k0 >= p.Nkv) return;

  // dK (scaled, rotated back with RoPE) and dV rows k0 + 8(r/4) + 4h + (r mod 4)
#pragma unroll
  for (int c = 0; c < DC; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[c][r] *= p.scale;
  if (rope) {
    // d = DC col + c; its rotate-half partner d +- D/2 is lane col ^ 16
    const bool lo = col < 16;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = min(k0 + 8 * (r >> 2) + 4 * h + (r & 3), p.Nkv - 1);
      const float* cr = reinterpret_cast<const float*>(p.cos) + (int64_t)kr * p.rs[0];
      const float* sr = reinterpret_cast<const float*>(p.sin) + (int64_t)kr * p.rs[0];
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const float g = dk[c][r];
        const float gp = __shfl_xor(g, 16, 64);
        const int dl = lo ? DC * col + c : DC * col + c - DH;
        float l = lo ? g : gp, hh = lo ? gp : g;
        f32_rope_back(l, hh, cr[dl], sr[dl], cr[dl + DH], sr[dl + DH]);
        dk[c][r] = lo ? l : hh;
      }
    }
  }
  // one split: final dK / dV; several: this split's partial sums (already
  // scaled and rotated back, both linear) in (g_split, B, Hkv, Nkv, D)
  float* dkg = reinterpret_cast<float*>(p.dk) + b * p.dks[0] + hk * p.dks[1];
  float* dvg = reinterpret_cast<float*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1];
  int64_t dks2 = p.dks[2], dvs2 = p.dvs[2];
  if (p.g_split > 1) {
    const int64_t off = (((int64_t)gsi * p.B + b) * p.Hkv + hk) * p.Nkv * D;
    dkg = p.dkp + off;
    dvg = p.dvp + off;
    dks2 = dvs2 = D;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kr = k0 + 8 * (r >> 2) + 4 * h + (r & 3);
    if (kr >= p.Nkv) continue;
    VecC a, v;
    if constexpr (DC == 1) {
      a = dk[0][r];
      v = dv[0][r];
    } else {
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        a[c] = dk[c][r];
        v[c] = dv[c][r];
      }
    }
    *reinterpret_cast<VecC*>(dkg + (int64_t)kr * dks2 + DC * col) = a;
    *reinterpret_cast<VecC*>(dvg + (int64_t)kr * dvs2 + DC * col) = v;
  }
}

// dK, dV row = the sum of the g_split partial rows, in split order (the
// result does not depend on which workgroup finished first).  One thread per
// (row r = (b Hkv + h) Nkv + n, 4 consecutive d).
template <int D>
__global__ void __launch_bounds__(256) bwd_dkv_combine_f32_kernel(const BwdParams p) {
  const int64_t rows = (int64_t)p.B * p.Hkv * p.Nkv;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = t / (D / 4);
  if (r >= rows) return;
  const int d = (int)(t % (D / 4)) * 4;
  const int n = (int)(r % p.Nkv);
  const int64_t bh = r / p.Nkv;
  const int hk = (int)(bh % p.Hkv), b = (int)(bh / p.Hkv);
  f32x4 sk = *reinterpret_cast<const f32x4*>(p.dkp + r * D + d);
  f32x4 sv = *reinterpret_cast<const f32x4*>(p.dvp + r * D + d);
  for (int sp = 1; sp < p.g_split; ++sp) {
    sk += *reinterpret_cast<const f32x4*>(p.dkp + (sp * rows + r) * D + d);
    sv += *reinterpret_cast<const f32x4*>(p.dvp + (sp * rows + r) * D + d);
  }
  *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.dk) + b * p.dks[0] + hk * p.dks[1] + (int64_t)n * p.dks[2] +
                            d) = sk;
  *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1] + (int64_t)n * p.dvs[2] +
                            d) = sv;
}

// dQ body of workgroup wg; kl / vl: the two LDS tiles.
template <int D, int WAVES>
__device__ __forceinline__ void bwd_dq_f32_body(const BwdParams& p, int mask, int bias, int rope, F32Tile<D>& kl,
                                                F32Tile<D>& vl, int wg) {
  constexpr int DH = D / 2, DC = D / 32;
  constexpr int BLK = 32 * WAVES;
  typedef typename F32Vec<DC>::T VecC;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 31, h = lane >> 5;
  const int nbh = p.B * p.Hq;
  int mb = wg / nbh;
  const int bh = wg % nbh;
  if (mask == MASK_CAUSAL || mask == MASK_CSW) mb = p.n_qblocks - 1 - mb;
  const int b = bh / p.Hq, hq = bh % p.Hq, hk = hq / p.G;
  const int qw0 = mb * BLK;  // first query of the workgroup
  const int q0 = qw0 + w * 32;
  const int qrow = q0 + col;
  const int qc = min(qrow, p.Nq - 1);  // clamped: rows >= N_q compute, store nothing

  // this lane's q~ and dO half rows: the B operands of S^T and dP^T
  const float* qt = reinterpret_cast<const float*>(p.qt) + b * p.qts[0] + hq * p.qts[1] + (int64_t)qc * p.qts[2];
  const float* dog = reinterpret_cast<const float*>(p.dout) + b * p.dos[0] + hq * p.dos[1] + (int64_t)qc * p.dos[2];
  f32x4 qh[DH / 4], gh[DH / 4];
#pragma unroll
  for (int j = 0; j < DH / 4; ++j) {
    qh[j] = *reinterpret_cast<const f32x4*>(qt + h * DH + 4 * j);
    gh[j] = *reinterpret_cast<const f32x4*>(dog + h * DH + 4 * j);
  }

  // Key tiles one of the workgroup's queries can see: one range for all four
  // waves (set by the workgroup index only), so every wave runs the same
  // loop and reaches every barrier.
  int n_lo = 0, n_hi = p.Nkv;
  if (mask == MASK_CAUSAL) {
    n_hi = min(n_hi, qw0 + BLK);
  } else if (mask == MASK_SW) {
    n_lo = max(0, qw0 - p.window + 1);
    n_hi = min(n_hi, qw0 + BLK - 1 + p.window);
  } else if (mask == MASK_CSW) {
    n_lo = max(0, qw0 - p.window + 1);
    n_hi = min(n_hi, qw0 + BLK);
  }
  n_lo &= ~31;
  // key tiles: a range, or the Q-major lists of this query block (full, then
  // partial; entries of block_n keys, bs_sub tiles each)
  int ntk = n_hi > n_lo ? (n_hi - n_lo + 31) / 32 : 0, bs_sub = 1, bs_nfull = 0;
  const int32_t* bs_full = nullptr;
  const int32_t* bs_part = nullptr;
  if (mask == MASK_BS) {
    bs_sub = p.bs_block_n / 32;
    bs_nfull = p.bs_full_num[mb];
    bs_full = p.bs_full_idx + mb * p.bs_full_rs;
    bs_part = p.bs_part_idx + mb * p.bs_part_rs;
    ntk = (bs_nfull + p.bs_part_num[mb]) * bs_sub;
  }

  const float zc = p.scale * kLog2e;
  const float slope = bias == BIAS_ALIBI ? p.slopes[hq] * kLog2e : 0.f;
  const f32x2 l2 = *reinterpret_cast<const f32x2*>(p.ld + 2 * ((int64_t)(b * p.Hq + hq) * p.Nq + qc));
  const float* kt = reinterpret_cast<const float*>(p.kt) + b * p.kts[0] + hk * p.kts[1];
  const float* vg = reinterpret_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1];

  f32x16 dq[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[c][r] = 0.f;

  for (int t = 0; t < ntk; ++t) {
    const int n0 = mask == MASK_BS ? bs_row_get(bs_full, bs_nfull, bs_part, t / bs_sub) * p.bs_block_n + (t % bs_sub) * 32
                                   : n_lo + 32 * t;
    __syncthreads();  // every wave is done with the previous tile
    for (int idx = threadIdx.x; idx < 32 * (D / 4); idx += WAVES * 64) {
      const int r = idx / (D / 4), c4 = (idx % (D / 4)) * 4;
      const int n = n0 + r;
      f32x4 a = {0.f, 0.f, 0.f, 0.f}, v = {0.f, 0.f, 0.f, 0.f};
      if (n < p.Nkv) {
        a = *reinterpret_cast<const f32x4*>(kt + (int64_t)n * p.kts[2] + c4);
        v = *reinterpret_cast<const f32x4*>(vg + (int64_t)n * p.vs[2] + c4);
      }
      *reinterpret_cast<f32x4*>(&kl[r][c4]) = a;
      *reinterpret_cast<f32x4*>(&vl[r][c4]) = v;
    }
    __syncthreads();
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
    for (int j = 0; j < DH / 4; ++j) {
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(&kl[col][h * DH + 4 * j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(k4[e], qh[j][e], s, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < DH / 4; ++j) {
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(&vl[col][h * DH + 4 * j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dp = __builtin_amdgcn_mfma_f32_32x32x2f32(v4[e], gh[j][e], dp, 0, 0, 0);
    }
    // element mask of a partial block-sparse tile (partial entries follow
    // the full ones): bits of this lane's query row over the tile's 32 keys,
    // shifted by 4 h (constant bit per element)
    uint32_t ebits = ~0u;
    if (mask == MASK_BS && p.bs_row_bits != nullptr) {
      const int e = t / bs_sub;
      if (e >= bs_nfull) {
        const int sb = t - e * bs_sub;
        const int64_t word = (((int64_t)mb * p.bs_part_rs + (e - bs_nfull)) * p.bs_block_m + (qrow - qw0)) *
                                 (p.bs_block_n / 64) + (sb >> 1);
        ebits = qrow < p.Nq ? (uint32_t)(p.bs_row_bits[word] >> (32 * (sb & 1))) >> (4 * h) : 0u;
      }
    }
    // dS^T of key n0 + 8(r/4) + 4h + (r mod 4), query qrow
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kj = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
      float x = s[r] * zc - l2[0];
      if (bias == BIAS_ALIBI) x -= slope * (float)abs(qrow - kj);
      const bool vis = qrow < p.Nq && kj < p.Nkv && f32_visible(mask, p.window, qrow, kj) &&
                       (ebits & (1u << (8 * (r >> 2) + (r & 3))));
      const float pr = vis ? __builtin_amdgcn_exp2f(x) : 0.f;
      ds[r] = pr * (dp[r] - l2[1]);
    }
    // dQ^T += k~^T dS^T, k~ rows of the keys of register i from LDS
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = 8 * (i >> 2) + 4 * h + (i & 3);
      const VecC kv = *reinterpret_cast<const VecC*>(&kl[kj][DC * col]);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        float kc;
        if constexpr (DC == 1) kc = kv;
        else kc = kv[c];
        dq[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(kc, ds[i], dq[c], 0, 0, 0);
      }
    }
  }

  if (qrow >= p.Nq) return;
#pragma unroll
  for (int c = 0; c < DC; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[c][r] *= p.scale;
  if (rope) {
    // d = DC (8(r/4) + 4h + (r mod 4)) + c: registers r < 8 hold d < D/2,
    // and register r + 8 holds the partner d + D/2
    const float* cr = reinterpret_cast<const float*>(p.cos) + (int64_t)qrow * p.rs[0];
    const float* sr = reinterpret_cast<const float*>(p.sin) + (int64_t)qrow * p.rs[0];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const int d = DC * (8 * (r >> 2) + 4 * h + (r & 3)) + c;
        float l = dq[c][r], hh = dq[c][r + 8];
        f32_rope_back(l, hh, cr[d], sr[d], cr[d + DH], sr[d + DH]);
        dq[c][r] = l;
        dq[c][r + 8] = hh;
      }
  }
  float* dqr = reinterpret_cast<float*>(p.dq) + b * p.dqs[0] + hq * p.dqs[1] + (int64_t)qrow * p.dqs[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d0 = DC * (8 * (r >> 2) + 4 * h + (r & 3));
    VecC st;
    if constexpr (DC == 1) {
      st = dq[0][r];
    } else {
#pragma unroll
      for (int c = 0; c < DC; ++c) st[c] = dq[c][r];
    }
    *reinterpret_cast<VecC*>(dqr + d0) = st;
  }
}

// The dK/dV and dQ kernels, one launch each, and both in one launch: its
// first n_dkv_wg workgroups run the dK/dV body (heaviest key blocks first
// under a causal mask), the rest the dQ body, whose workgroups fill the
// slots the short causal dK/dV workgroups free at the end of the first.
template <int D, int WAVES = kBwdF32Waves>
__global__ void __launch_bounds__(WAVES * 64) bwd_dkv_f32_kernel(const BwdParams p, int mask, int bias, int rope) {
  __shared__ __attribute__((aligned(16))) F32Tile<D> ql, gl;
  bwd_dkv_f32_body<D, WAVES>(p, mask, bias, rope, ql, gl, (int)blockIdx.x);
}

template <int D, int WAVES = kBwdF32Waves>
__global__ void __launch_bounds__(WAVES * 64) bwd_dq_f32_kernel(const BwdParams p, int mask, int bias, int rope) {
  __shared__ __attribute__((aligned(16))) F32Tile<D> kl, vl;
  bwd_dq_f32_body<D, WAVES>(p, mask, bias, rope, kl, vl, (int)blockIdx.x);
}

template <int D, int WAVES = kBwdF32Waves>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2)))
    bwd_dkvdq_f32_kernel(const BwdParams p, int mask, int bias, int rope) {
  __shared__ __attribute__((aligned(16))) F32Tile<D> ta, tb;
  if ((int)blockIdx.x < p.n_dkv_wg)
    bwd_dkv_f32_body<D, WAVES>(p, mask, bias, rope, ta, tb, (int)blockIdx.x);
  else
    bwd_dq_f32_body<D, WAVES>(p, mask, bias, rope, ta, tb, (int)blockIdx.x - p.n_dkv_wg);
}

}  // namespace af
