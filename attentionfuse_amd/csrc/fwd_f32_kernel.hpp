// fp32 forward: fp32 inputs, scores, softmax and P V all in fp32 on the
// fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// The reference accepts fp32 tensors (tests/test_correctness.py:28 and
// test_backward.py:63 run them) and its Triton dots then compute in TF32
// (10-bit mantissa); here every product is a full fp32 product, so the
// results sit closer to the fp32 oracle than the reference's do.
//
// Structure.  One wave owns 32 query rows; a workgroup is four independent
// waves (128 rows of one (b, h_q)), with no barrier after the query rows
// are staged.  Per 32-key tile a wave computes
//   S^T (32 keys x 32 queries) = K Q^T   in D/2 MFMAs (K-dim 2 each), and
//   O^T (D x 32 queries) += V^T P^T      in 16 * D/32 MFMAs.
// The dot-product order is free, so MFMA i pairs d = i (lanes 0-31) with
// d = D/2 + i (lanes 32-63): lane l reads one contiguous half row of its
// key (l mod 32) and of its query.  Accumulator register r of lane l holds
// key 8(r/4) + 4h + (r mod 4) of query l mod 32 (h = l / 32), which is the
// key the B operand of the r-th P V MFMA needs from that lane, so P goes
// from the softmax straight into the P V MFMAs.  Output block c, row m
// holds d = (D/32) m + c: a lane's V operands of one key, and its O stores,
// are D/32 consecutive floats.  Every lane owns one query of O^T, so the
// online-softmax rescale needs no cross-lane traffic.
//
// Masks (block-sparse: the BlockMask row of each wave's 32 queries lists its
// key blocks), bias kind, normalisation and RoPE are uniform runtime switches:
// the mask test and bias add are a few VALU instructions per score against
// 64 cycles per MFMA.  Keys are rotated once per call (rope_f32_kernel) and
// the query rows once per workgroup, as the 16-bit path does.
#pragma once

#include "af_common.hpp"
#include "fwd_kernel.hpp"

namespace af {

struct FwdF32Params {
  FwdParams f;   // pointers address fp32 data; strides are in elements
  int32_t mask, bias, norm, rope;
};

#ifndef AF_F32_TWO_K
#define AF_F32_TWO_K(D) ((D) >= 128)
#endif

constexpr int kF32Waves = 4;          // waves (32 query rows each) per workgroup
constexpr int kF32BlockM = 32 * kF32Waves;

// Rotate-half RoPE of fp32 rows (B, H, N, D) into a contiguous buffer; one
// thread per (row, d < D/2) pair.
template <int D>
__global__ void __launch_bounds__(256) rope_f32_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                       const float* __restrict__ cs, const float* __restrict__ sn,
                                                       int64_t xs0, int64_t xs1, int64_t xs2, int64_t rs, int H,
                                                       int N, int64_t rows) {
  constexpr int DH = D / 2;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = t / DH;
  if (r >= rows) return;
  const int d = (int)(t % DH);
  const int n = (int)(r % N);
  const int64_t bh = r / N;
  const int hh = (int)(bh % H), b = (int)(bh / H);
  const float* xr = x + b * xs0 + hh * xs1 + n * xs2;
  const float lo = xr[d], hi = xr[d + DH];
  const float* cr = cs + n * rs;
  const float* sr = sn + n * rs;
  out[r * D + d] = lo * cr[d] - hi * sr[d];
  out[r * D + d + DH] = hi * cr[d + DH] + lo * sr[d + DH];
}

template <int N>
struct F32Vec;
template <>
struct F32Vec<1> {
  typedef float T;
};
template <>
struct F32Vec<2> {
  typedef f32x2 T;
};
template <>
struct F32Vec<4> {
  typedef f32x4 T;
};

template <int D>
__global__ void __launch_bounds__(kF32Waves * 64) fwd_f32_kernel(const FwdF32Params P) {
  constexpr int DH = D / 2;   // d per lane half in the score MFMAs
  constexpr int DC = D / 32;  // output column blocks
  constexpr int QP = D + 4;   // LDS row pitch in floats: rows 16 bytes apart in bank order
  typedef typename F32Vec<DC>::T VecC;
  __shared__ __attribute__((aligned(16))) float qs[kF32Waves][32][QP];

  const FwdParams& p = P.f;
  const int mask = P.mask, bias = P.bias, norm = P.norm;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 31, h = lane >> 5;
  const int nbh = p.B * p.Hq;
  int mb = (int)(blockIdx.x / nbh);
  const int bh = (int)(blockIdx.x % nbh);
  // causal-type masks: the longest key ranges first
  if (mask == MASK_CAUSAL || mask == MASK_CSW) mb = p.n_mblocks - 1 - mb;
  const int b = bh / p.Hq, hq = bh % p.Hq, hk = hq / p.G;
  const int q0 = mb * kF32BlockM + w * 32;
  const int qrow = q0 + col;

  // ---- query rows (rotated with RoPE) into this wave's LDS rows ------------
  const float* qg = reinterpret_cast<const float*>(p.q) + b * p.qs[0] + hq * p.qs[1];
  for (int idx = lane; idx < 32 * (D / 4); idx += 64) {
    const int r = idx / (D / 4), c4 = (idx % (D / 4)) * 4;
    const int n = q0 + r;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (n < p.Nq) {
      const float* qr = qg + (int64_t)n * p.qs[2];
      v = *reinterpret_cast<const f32x4*>(qr + c4);
      if (P.rope) {
        const bool lo = c4 < DH;
        const f32x4 pv = *reinterpret_cast<const f32x4*>(qr + (lo ? c4 + DH : c4 - DH));
        const f32x4 c = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.cos) + n * p.rs[0] + c4);
        const f32x4 s = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.sin) + n * p.rs[0] + c4);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = lo ? v[j] * c[j] - pv[j] * s[j] : v[j] * c[j] + pv[j] * s[j];
      }
    }
    *reinterpret_cast<f32x4*>(&qs[w][r][c4]) = v;
  }
  __syncthreads();
  if (q0 >= p.Nq) return;

  // ---- key range of this wave ------------------------------------------------
  int n_lo = 0, n_hi = p.Nkv;
  if (mask == MASK_CAUSAL) {
    n_hi = min(n_hi, q0 + 32);
  } else if (mask == MASK_SW) {
    n_lo = max(0, q0 - p.window + 1);
    n_hi = min(n_hi, q0 + 31 + p.window);
  } else if (mask == MASK_CSW) {
    n_lo = max(0, q0 - p.window + 1);
    n_hi = min(n_hi, q0 + 32);
  }
  n_lo &= ~31;
  // 32-key tiles: a range, or with a block mask the tiles of the listed key
  // blocks of this wave's mask row (32-row waves never straddle two rows)
  int ntiles = n_hi > n_lo ? (n_hi - n_lo + 31) / 32 : 0;
  int bs_sub = 1, bs_nfull = 0, mr = 0;
  const int32_t* bs_full_row = nullptr;
  const int32_t* bs_part_row = nullptr;
  if (mask == MASK_BS) {
    mr = q0 / p.bs_block_m;
    bs_sub = p.bs_block_n / 32;
    bs_nfull = p.bs_full_num[mr];
    bs_full_row = p.bs_full_idx + mr * p.bs_full_rs;
    bs_part_row = p.bs_part_idx + mr * p.bs_part_rs;
    ntiles = (bs_nfull + p.bs_part_num[mr]) * bs_sub;
  }
  auto tile_n0 = [&](int t) -> int {
    if (mask == MASK_BS) {
      const int e = t / bs_sub;
      return bs_row_get(bs_full_row, bs_nfull, bs_part_row, e) * p.bs_block_n + 32 * (t - e * bs_sub);
    }
    return n_lo + 32 * t;
  };

  const float* kg = reinterpret_cast<const float*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const float* vg = reinterpret_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  // logits in log2 units for softmax (exp2), natural units for ReLU
  const float unit = norm == NORM_SOFTMAX ? kLog2e : 1.f;
  const float zc = p.scale * unit;
  const float slope = bias == BIAS_ALIBI ? p.slopes[hq] * unit : 0.f;
  const float* brow = nullptr;
  if (bias == BIAS_ADD)
    brow = reinterpret_cast<const float*>(p.bias) + b * p.bs[0] + hq * p.bs[1] + (int64_t)min(qrow, p.Nq - 1) * p.bs[2];

  f32x16 o[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.f;
  float m_run = -1e30f, lsum = 0.f;

  // K rows are clamped to the last key: loads stay in bounds and every
  // score of a key >= N_kv is masked below.  With two K buffers (head dims
  // whose kernel runs one wave per SIMD anyway) tile t + 2's rows are
  // loaded while tiles t + 1 and t are computed: one tile of compute did not
  // cover the load latency, the score MFMAs of each tile waited for their K
  // rows.  One buffer: tile t + 1's rows load while tile t computes.
  constexpr bool kTwoK = AF_F32_TWO_K(D);
  constexpr int kKAhead = kTwoK ? 2 : 1;
  f32x4 kva[DH / 4], kvb[kTwoK ? DH / 4 : 1];
  auto load_k = [&](f32x4 (&kv)[DH / 4], int n0) {
    const float* kr = kg + (int64_t)min(n0 + col, p.Nkv - 1) * p.ks[2] + h * DH;
#pragma unroll
    for (int i = 0; i < DH / 4; ++i) kv[i] = *reinterpret_cast<const f32x4*>(kr + 4 * i);
  };
  if (ntiles > 0) load_k(kva, tile_n0(0));
  if constexpr (kTwoK) {
    if (ntiles > 1) load_k(kvb, tile_n0(1));
  }

  auto tile = [&](int t, f32x4 (&kv)[DH / 4]) __attribute__((always_inline)) {
    const int n0 = tile_n0(t);
    VecC vv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = min(n0 + 8 * (i >> 2) + 4 * h + (i & 3), p.Nkv - 1);
      vv[i] = *reinterpret_cast<const VecC*>(vg + (int64_t)key * p.vs[2] + DC * col);
    }
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int j = 0; j < DH / 4; ++j) {
      const f32x4 qv = *reinterpret_cast<const f32x4*>(&qs[w][col][h * DH + 4 * j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[j][e], qv[e], s, 0, 0, 0);
    }
    if (t + kKAhead < ntiles) load_k(kv, tile_n0(t + kKAhead));  // rows clamped, so in bounds

    // element mask of a partial block-sparse tile: bits of this lane's
    // query row over the tile's 32 keys (partial entries follow the full
    // ones), shifted by 4 h so that every element tests a constant bit
    uint32_t ebits = ~0u;
    if (mask == MASK_BS && p.bs_row_bits != nullptr) {
      const int e = t / bs_sub;
      if (e >= bs_nfull) {
        const int sb = t - e * bs_sub;
        const int64_t word =
            (((int64_t)mr * p.bs_part_rs + (e - bs_nfull)) * p.bs_block_m + (qrow - mr * p.bs_block_m)) *
                (p.bs_block_n / 64) + (sb >> 1);
        ebits = qrow < p.Nq ? (uint32_t)(p.bs_row_bits[word] >> (32 * (sb & 1))) >> (4 * h) : 0u;
      }
    }
    float x[16];
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
      float v = s[r] * zc;
      if (bias == BIAS_ALIBI) v -= slope * (float)abs(qrow - key);
      if (bias == BIAS_ADD) v += (key < p.Nkv ? brow[key] : 0.f) * unit;
      bool vis = key < p.Nkv;
      if (mask == MASK_CAUSAL) vis = vis && key <= qrow;
      else if (mask == MASK_SW) vis = vis && abs(qrow - key) < p.window;
      else if (mask == MASK_CSW) vis = vis && key <= qrow && key > qrow - p.window;
      vis = vis && (ebits & (1u << (8 * (r >> 2) + (r & 3))));
      x[r] = vis ? v : -INFINITY;
      mt = fmaxf(mt, x[r]);
    }
    if (norm == NORM_SOFTMAX) {
      const float m_new = fmaxf(m_run, max_xor32(mt));
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      lsum *= alpha;
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[c][r] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = __builtin_amdgcn_exp2f(x[r] - m_new);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = fmaxf(x[r], 0.f);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) lsum += x[r];

#pragma unroll
    for (int c = 0; c < DC; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float a;
        if constexpr (DC == 1) a = vv[i];
        else a = vv[i][c];
        o[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, x[i], o[c], 0, 0, 0);
      }
  };
  if constexpr (kTwoK) {
    for (int t = 0; t < ntiles; t += 2) {
      tile(t, kva);
      if (t + 1 < ntiles) tile(t + 1, kvb);
    }
  } else {
    for (int t = 0; t < ntiles; ++t) tile(t, kva);
  }

  // ---- epilogue: this lane's half of the keys plus its partner's ------------
  const float lt = lsum + xor32(lsum);
  const float inv = (lt == 0.f) ? 1.f : 1.f / lt;
  if (qrow < p.Nq) {
    float* orow = reinterpret_cast<float*>(p.o) + b * p.os[0] + hq * p.os[1] + (int64_t)qrow * p.os[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d0 = DC * (8 * (r >> 2) + 4 * h + (r & 3));
      VecC st;
      if constexpr (DC == 1) {
        st = o[0][r] * inv;
      } else {
#pragma unroll
        for (int c = 0; c < DC; ++c) st[c] = o[c][r] * inv;
      }
      *reinterpret_cast<VecC*>(orow + d0) = st;
    }
    if (p.lse != nullptr && h == 0) {
      float L = -INFINITY;
      if (norm == NORM_SOFTMAX && lt > 0.f) L = (m_run + __log2f(lt)) * kLn2;
      p.lse[b * p.ls[0] + hq * p.ls[1] + (int64_t)qrow * p.ls[2]] = L;
    }
  }
}

}  // namespace af
