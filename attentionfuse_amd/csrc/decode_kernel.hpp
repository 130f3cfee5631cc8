// Flash-decoding for gfx950 (piece (b)): one query row per head, the KV
// cache split over workgroups, then a log-sum-exp combine.
//
// Semantics follow the reference decode kernels
// (reference: attnfuse/compiler/codegen_decode.py:46-211): per split, an
// online softmax over its keys gives (m, l, acc); the combine kernel merges
// m* = max m_s, l* = sum e^(m_s - m*) l_s, O = sum e^(m_s - m*) acc_s / l*.
// ALiBi uses the query position N_kv - 1: bias = -slope_h |(N_kv-1) - j|
// (codegen_decode.py:142-145).  Unlike the reference, split boundaries are
// exact: every key is counted once whatever N_kv is.
//
// Work decomposition:
//  * one workgroup = (split, batch, kv head, chunk of up to 16 query heads
//    of that kv head's GQA group): the group shares every K/V byte read, so
//    the cache is streamed once per (batch, kv head) whatever the group size;
//  * the four waves interleave 32-key steps inside the split; each wave
//    keeps its own (m, l, O^T) and the waves merge through LDS at the end;
//  * S^T = K Q^T on the 16x16x32 MFMA with K read straight from HBM into the
//    A operand (16-byte loads, no LDS); O^T += V^T P^T on the same MFMA with
//    V^T written to a per-wave LDS tile; P^T feeds the MFMA from registers.
#pragma once

#include "af_common.hpp"

namespace af {

struct DecodeParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  const float* slopes;
  float* ws_ml;    // (S, B, Hq, 2) fp32: m (log2 units), l
  float* ws_acc;   // (S, B, Hq, D) fp32: unnormalised accumulator
  int64_t qs[4], ks[4], vs[4], os[4];
  int32_t B, Hq, Hkv, Nkv, G, nqc, nsplit, split_len;
  float scale;
};

// 16x16x32 MFMA layouts (lane l, group g = l / 16):
//   A (16 x 32): row l%16, k-slots 8g..8g+7     B (32 x 16): column l%16
//   C (16 x 16, 4 fp32): register r holds row 4g + r, column l%16.
// Two 16-key score blocks give lane (g, q) keys {4g + r} and {16 + 4g + r};
// those eight values are the B operand of the P*V MFMA over 32 keys when the
// V^T A operand uses the same key slots: slot e < 4 -> key 4g + e,
// slot e >= 4 -> key 16 + 4g + (e - 4).

template <class E, int D, int BIAS>
__global__ void __launch_bounds__(256) decode_split_kernel(const DecodeParams p) {
  constexpr int KSD = D / 32;      // 32-deep k-steps of K Q^T
  constexpr int DB = D / 16;       // 16-row blocks of O^T
  constexpr int VTP = 32 + 8;      // V^T tile pitch (elements)
  constexpr int VT_ELEMS = D * VTP;
  __shared__ __attribute__((aligned(16))) uint16_t lds[4 * VT_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int split = blockIdx.x;
  int rest = blockIdx.y;
  const int qc = rest % p.nqc; rest /= p.nqc;
  const int hk = rest % p.Hkv;
  const int b = rest / p.Hkv;
  const int hq0 = hk * p.G + 16 * qc;
  const int nq = min(16, p.G - 16 * qc);   // real query heads in this chunk
  const int hq = hq0 + c;                  // this lane's query column
  const bool qreal = c < nq;

  const uint16_t* __restrict__ kbase = p.k + b * p.ks[0] + hk * p.ks[1];
  const uint16_t* __restrict__ vbase = p.v + b * p.vs[0] + hk * p.vs[1];
  const int64_t kstr = p.ks[2], vstr = p.vs[2];

  // Q^T as B operand: lane (g, q = c) holds Q[q][32 ks + 8 g .. +7].
  u32x4 qf[KSD];
  {
    const uint16_t* qrow = p.q + b * p.qs[0] + (int64_t)(qreal ? hq : hq0) * p.qs[1];
#pragma unroll
    for (int ks = 0; ks < KSD; ++ks)
      qf[ks] = qreal ? ld16(qrow + 32 * ks + 8 * g) : u32x4{0, 0, 0, 0};
  }
  const float c2 = p.scale * kLog2e;
  float slope2 = 0.f;
  if constexpr (BIAS == 1) slope2 = qreal ? p.slopes[hq] * kLog2e : 0.f;

  const int s_lo = split * p.split_len;
  const int s_hi = min(s_lo + p.split_len, p.Nkv);
  const int nsteps = s_hi > s_lo ? (s_hi - s_lo + 31) / 32 : 0;

  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{};
  float m_run = -INFINITY, l_run = 0.f;
  uint16_t* vt = lds + w * VT_ELEMS;
  uint32_t* vt32 = reinterpret_cast<uint32_t*>(vt);

  // One 32-key step of this wave: K rows (A operand of S^T, keys k0 + 16 kb
  // + c) and V rows (lane owns keys k0 + 2c, 2c + 1 and 16-byte chunks
  // g + 4 i) come straight from HBM into registers.
  struct StepRegs {
    u32x4 ka[2][KSD];
    u32x4 va[D / 32][2];
  };
  auto load_step = [&](int st, StepRegs& r) {
    const int k0 = s_lo + 32 * st;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int n = k0 + 16 * kb + c;
      const bool ok = n < s_hi;
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks)
        r.ka[kb][ks] = ok ? ld16(kbase + n * kstr + 32 * ks + 8 * g) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int dc = g + 4 * i;
      const int n = k0 + 2 * c;
      r.va[i][0] = (n < s_hi) ? ld16(vbase + n * vstr + 8 * dc) : u32x4{0, 0, 0, 0};
      r.va[i][1] = (n + 1 < s_hi) ? ld16(vbase + (n + 1) * vstr + 8 * dc) : u32x4{0, 0, 0, 0};
    }
  };
  auto compute_step = [&](int st, const StepRegs& r) {
    const int k0 = s_lo + 32 * st;
    // S^T blocks.
    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x4{};
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks) s[kb] = E::mfma16(r.ka[kb][ks], qf[ks], s[kb]);
    }
    // V^T into this wave's LDS tile: row d, column = key - k0.
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int dc = g + 4 * i;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t a = r.va[i][0][e >> 1], bq = r.va[i][1][e >> 1];
        const uint32_t word = (e & 1) ? ((a >> 16) | (bq & 0xffff0000u))
                                      : ((a & 0xffffu) | (bq << 16));
        vt32[((8 * dc + e) * VTP + 2 * c) >> 1] = word;
      }
    }
    // Online softmax on this lane's eight keys of query c.
    float x[8];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int key = k0 + 16 * kb + 4 * g + rr;
        float v = s[kb][rr] * c2;
        if constexpr (BIAS == 1) v -= slope2 * (float)abs((p.Nkv - 1) - key);
        v = key < s_hi ? v : -INFINITY;
        x[4 * kb + rr] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
      ls += x[i];
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
    u32x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = E::pack(x[2 * i], x[2 * i + 1]);

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const uint16_t* row = vt + (16 * db + c) * VTP + 4 * g;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(row);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 16);
      const u32x4 va4 = {lo[0], lo[1], hi[0], hi[1]};
      o[db] = o[db] * alpha;
      o[db] = E::mfma16(va4, pb, o[db]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // The loads of step st + 4 are issued before step st is computed, so each
  // wave keeps two steps (16 KB at D = 128) of K/V in flight.
  StepRegs ra, rb;
  if (w < nsteps) load_step(w, ra);
  for (int st = w; st < nsteps; st += 8) {
    if (st + 4 < nsteps) load_step(st + 4, rb);
    compute_step(st, ra);
    if (st + 4 >= nsteps) break;
    if (st + 8 < nsteps) load_step(st + 8, ra);
    compute_step(st + 4, rb);
  }

  // ---- merge the four waves through LDS ------------------------------------
  // Per wave: l summed over the four lane groups; m is already uniform.
  float lw = l_run + __shfl_xor(l_run, 16, 64);
  lw += __shfl_xor(lw, 32, 64);
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  float* red_m = red;              // [4][16]
  float* red_l = red + 64;         // [4][16]
  float* red_o = red + 128;        // [4][16][D]  (q-major)
  if (g == 0) {
    red_m[w * 16 + c] = m_run;
    red_l[w * 16 + c] = lw;
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) red_o[(w * 16 + c) * D + 16 * db + 4 * g + r] = o[db][r];
  __syncthreads();
  // 256 threads merge 16 x D outputs.
  for (int idx = tid; idx < 16 * D; idx += 256) {
    const int qq = idx / D, d = idx - qq * D;
    if (qq >= nq) continue;
    float mstar = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) mstar = fmaxf(mstar, red_m[ww * 16 + qq]);
    const float mu = (mstar == -INFINITY) ? 0.f : mstar;
    float acc = 0.f, lsum = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float f = __builtin_amdgcn_exp2f(red_m[ww * 16 + qq] - mu);
      acc += f * red_o[(ww * 16 + qq) * D + d];
      lsum += f * red_l[ww * 16 + qq];
    }
    const int64_t row = ((int64_t)split * p.B + b) * p.Hq + hq0 + qq;
    p.ws_acc[row * D + d] = acc;
    if (d == 0) {
      p.ws_ml[2 * row] = mstar;
      p.ws_ml[2 * row + 1] = lsum;
    }
  }
}

// Combine: one 256-thread workgroup per (batch, query head).  Thread t owns
// output dim t % D and the splits s = t / D (mod 256 / D); the partial sums
// of the split groups meet in LDS.  All loads of a thread are independent,
// so the kernel is bound by the (L2-resident) workspace reads, not latency.
template <class E, int D, bool F32OUT = false>
__global__ void __launch_bounds__(256) decode_combine_kernel(const DecodeParams p) {
  constexpr int NG = 256 / D;
  __shared__ float red_acc[NG][D];
  __shared__ float red_l[NG];
  const int t = threadIdx.x;
  const int d = t % D, grp = t / D;
  const int row = blockIdx.x;                 // b * Hq + hq
  const int b = row / p.Hq, hq = row - b * p.Hq;
  const int S = p.nsplit;
  const int64_t plane = (int64_t)p.B * p.Hq;
  float mstar = -INFINITY;
  for (int s = 0; s < S; ++s) mstar = fmaxf(mstar, p.ws_ml[2 * (s * plane + row)]);
  const float mu = (mstar == -INFINITY) ? 0.f : mstar;
  float acc = 0.f, lsum = 0.f;
#pragma unroll 4
  for (int s = grp; s < S; s += NG) {
    const int64_t r = s * plane + row;
    const float f = __builtin_amdgcn_exp2f(p.ws_ml[2 * r] - mu);
    lsum += f * p.ws_ml[2 * r + 1];
    acc += f * p.ws_acc[r * D + d];
  }
  red_acc[grp][d] = acc;
  if (d == 0) red_l[grp] = lsum;
  __syncthreads();
  if (grp == 0) {
    float a = 0.f, l = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) {
      a += red_acc[g2][d];
      l += red_l[g2];
    }
    const float inv = (l == 0.f) ? 1.f : 1.f / l;
    if constexpr (F32OUT)
      reinterpret_cast<float*>(p.o)[b * p.os[0] + hq * p.os[1] + d] = a * inv;
    else
      p.o[b * p.os[0] + hq * p.os[1] + d] = E::one(a * inv);
  }
}

// ---------------------------------------------------------------------------
// fp32 split kernel.  Decode reads every K/V byte once and does 4 FLOP per
// 4 bytes read, so fp32 FMAs on the VALU keep up with HBM and no fp32 MFMA
// is needed.  Lane (k, c) = (lane / 8, lane % 8) holds dims [c D/8, (c+1)
// D/8) of key slot k: a wave covers 8 keys per step, the dot products are
// finished with three xor shuffles inside each group of 8 lanes, and the
// running max of a query head is wave-uniform after three more.  A
// workgroup serves up to kF32DecHeads(D) query heads of one key/value head,
// so each K/V row is read once for all of them; each wave keeps the K/V rows
// of its next step in flight while it computes the current one.  The
// partials (m in log2 units, l, acc) use the 16-bit kernel's workspace
// layout, so the combine kernel is the same.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int f32_decode_heads(int D) { return 64 / (D / 8) < 16 ? 64 / (D / 8) : 16; }
template <int D>
constexpr int kF32DecHeads() { return f32_decode_heads(D); }

template <int D, int BIAS>
__global__ void __launch_bounds__(256) decode_split_f32_kernel(const DecodeParams p) {
  constexpr int CH = D / 8;                 // dims per lane
  constexpr int GQ = kF32DecHeads<D>();     // query heads per workgroup
  __shared__ float red[4][GQ][2 + D];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int kk = lane >> 3, c = lane & 7;
  const int split = blockIdx.x;
  int rest = blockIdx.y;
  const int qc = rest % p.nqc;
  rest /= p.nqc;
  const int hk = rest % p.Hkv;
  const int b = rest / p.Hkv;
  const int hq0 = hk * p.G + GQ * qc;
  const int nq = min(GQ, p.G - GQ * qc);    // real query heads in this chunk

  const float* kbase = reinterpret_cast<const float*>(p.k) + b * p.ks[0] + hk * p.ks[1] + CH * c;
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1] + CH * c;
  // this lane's dims of every query head of the chunk, pre-scaled to log2
  // units (the scale multiplies the fp32 dot product; no rounding involved)
  const float c2 = p.scale * kLog2e;
  float q[GQ][CH];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    const float* qr = reinterpret_cast<const float*>(p.q) + b * p.qs[0] + (int64_t)(hq0 + min(g, nq - 1)) * p.qs[1] +
                      CH * c;
#pragma unroll
    for (int e = 0; e < CH; e += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(qr + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) q[g][e + j] = v[j];
    }
  }
  float slope2[GQ];
#pragma unroll
  for (int g = 0; g < GQ; ++g) slope2[g] = BIAS == 1 ? p.slopes[hq0 + min(g, nq - 1)] * kLog2e : 0.f;

  const int s_lo = split * p.split_len;
  const int s_hi = min(s_lo + p.split_len, p.Nkv);
  const int nsteps = s_hi > s_lo ? (s_hi - s_lo + 7) / 8 : 0;

  float m[GQ], l[GQ], acc[GQ][CH];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < CH; ++e) acc[g][e] = 0.f;
  }

  // rows of key slot kk of step st (clamped to the last key: every load is
  // in bounds, and scores of keys >= s_hi are masked)
  auto load = [&](int st, float (&kr)[CH], float (&vr)[CH]) {
    const int key = min(s_lo + 8 * st + kk, s_hi - 1);
#pragma unroll
    for (int e = 0; e < CH; e += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(kbase + (int64_t)key * p.ks[2] + e);
      const f32x4 v = *reinterpret_cast<const f32x4*>(vbase + (int64_t)key * p.vs[2] + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kr[e + j] = a[j];
        vr[e + j] = v[j];
      }
    }
  };
  auto compute = [&](int st, const float (&kr)[CH], const float (&vr)[CH]) {
    const int key = s_lo + 8 * st + kk;
    const bool ok = key < s_hi;
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < CH; ++e) d = __builtin_fmaf(q[g][e], kr[e], d);
      d += __shfl_xor(d, 1, 64);
      d += __shfl_xor(d, 2, 64);
      d += __shfl_xor(d, 4, 64);
      float x = d * c2;
      if constexpr (BIAS == 1) x -= slope2[g] * (float)abs((p.Nkv - 1) - key);
      x = ok ? x : -INFINITY;
      float mx = fmaxf(x, __shfl_xor(x, 8, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m[g], mx);   // wave-uniform
      if (m_new > m[g]) {
        const float alpha = __builtin_amdgcn_exp2f(m[g] - m_new);   // 0 while m = -inf
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < CH; ++e) acc[g][e] *= alpha;
        m[g] = m_new;
      }
      const float pr = (m[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x - m[g]);
      l[g] += pr;
#pragma unroll
      for (int e = 0; e < CH; ++e) acc[g][e] = __builtin_fmaf(pr, vr[e], acc[g][e]);
    }
  };
  float ka[CH], va[CH], kb2[CH], vb[CH];
  if (w < nsteps) load(w, ka, va);
  for (int st = w; st < nsteps; st += 8) {
    if (st + 4 < nsteps) load(st + 4, kb2, vb);
    compute(st, ka, va);
    if (st + 4 >= nsteps) break;
    if (st + 8 < nsteps) load(st + 8, ka, va);
    compute(st + 4, kb2, vb);
  }

  // ---- per wave: sums over the 8 key slots, then the 4 waves through LDS --
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    l[g] += __shfl_xor(l[g], 8, 64);
    l[g] += __shfl_xor(l[g], 16, 64);
    l[g] += __shfl_xor(l[g], 32, 64);
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      float a = acc[g][e];
      a += __shfl_xor(a, 8, 64);
      a += __shfl_xor(a, 16, 64);
      a += __shfl_xor(a, 32, 64);
      acc[g][e] = a;
    }
  }
  if (kk == 0) {
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      if (c == 0) {
        red[w][g][0] = m[g];
        red[w][g][1] = l[g];
      }
#pragma unroll
      for (int e = 0; e < CH; ++e) red[w][g][2 + CH * c + e] = acc[g][e];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < GQ * D; idx += 256) {
    const int g = idx / D, d = idx - g * D;
    if (g >= nq) continue;
    float mstar = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) mstar = fmaxf(mstar, red[ww][g][0]);
    const float mu = (mstar == -INFINITY) ? 0.f : mstar;
    float a = 0.f, ls = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float f = __builtin_amdgcn_exp2f(red[ww][g][0] - mu);
      a += f * red[ww][g][2 + d];
      ls += f * red[ww][g][1];
    }
    const int64_t row = ((int64_t)split * p.B + b) * p.Hq + hq0 + g;
    p.ws_acc[row * D + d] = a;
    if (d == 0) {
      p.ws_ml[2 * row] = mstar;
      p.ws_ml[2 * row + 1] = ls;
    }
  }
}

}  // namespace af
