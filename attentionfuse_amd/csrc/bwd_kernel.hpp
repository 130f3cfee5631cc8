// Attention backward for gfx950 (piece (c), with the block-sparse walk of
// piece (d)).
//
// Math (FA2; reference: attnfuse/compiler/codegen_backward.py:45-302):
//   delta_i = sum_d dO_id O_id                          (bwd_delta_kernel)
//   P_ij    = exp(S_ij - L_i),  S = scale * q~ k~^T + bias,  masked -> 0
//   dV_j    = sum_i P_ij dO_i
//   dP_ij   = dO_i . v_j,   dS_ij = P_ij (dP_ij - delta_i)
//   dK~_j   = scale * sum_i dS_ij q~_i,   dQ~_i = scale * sum_j dS_ij k~_j
// with q~ = rope(q), k~ = rope(k).  With fused RoPE the kernels return the
// gradient with respect to the un-rotated inputs, dx = R^T dx~, where
//   dx[d] = g[d] cos[d] + g[d+D/2] sin[d+D/2],
//   dx[d+D/2] = g[d+D/2] cos[d+D/2] - g[d] sin[d]
// (the transpose of rotate-half; the reference has no RoPE backward,
// attnfuse/runtime/backward.py:77-79).
//
// Decomposition:
//  * bwd_dkv_kernel: a workgroup owns 32*WAVES keys of one (batch, kv head);
//    each wave owns 32 keys with k~ and v held in registers as MFMA B
//    operands.  It walks the query tiles (32 rows) of every query head of
//    the GQA group, so dK/dV come out group-summed with no atomics.  Score
//    tiles are S (queries x keys) with the query rows permuted (kperm) so
//    that P and dS feed the dV^T and dK^T MFMAs straight from registers.
//  * bwd_dq_kernel: a workgroup owns 32*WAVES query rows of one (batch,
//    head); q~ and dO stay in registers; key tiles (32 keys) stream through
//    LDS as k~, k~^T and v.  Scores are S^T (keys x queries) so dS^T is the
//    B operand of the dQ^T MFMA.
//  * Both kernels stage 32-row tiles into LDS double-buffered (global loads
//    of tile t+1 in flight during the MFMAs of tile t), writing rows and,
//    where an MFMA needs the contraction index contiguous, the transpose.
#pragma once

#include "af_common.hpp"
#include "fwd_kernel.hpp"

namespace af {

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  float* delta;            // (B, Hq, Nq) fp32 workspace
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  const uint16_t* cos;
  const uint16_t* sin;
  const float* slopes;
  const int32_t* bs_full_num;
  const int32_t* bs_full_idx;
  const int32_t* bs_part_num;
  const int32_t* bs_part_idx;
  const int32_t* bs_q_num;
  const int32_t* bs_q_idx;
  int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4], ls[3], rs[2];
  int64_t bs_full_rs, bs_part_rs, bs_q_rs;
  int32_t B, Hq, Hkv, Nq, Nkv, G, window;
  int32_t bs_block_m, bs_block_n;
  int32_t n_qblocks, n_kblocks;   // workgroup tiling of the two kernels
  int32_t rope_len;               // rows of the RoPE tables
  float scale;
};

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O), fp32.
// ---------------------------------------------------------------------------
template <class E, int D>
__global__ void __launch_bounds__(256) bwd_delta_kernel(const BwdParams p) {
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int RPB = 256 / CPR;      // rows per workgroup
  const int tid = threadIdx.x;
  const int64_t r = (int64_t)blockIdx.x * RPB + tid / CPR;
  const int ch = tid % CPR;
  const int64_t total = (int64_t)p.B * p.Hq * p.Nq;
  float acc = 0.f;
  if (r < total) {
    const int i = (int)(r % p.Nq);
    const int64_t bh = r / p.Nq;
    const int hq = (int)(bh % p.Hq), b = (int)(bh / p.Hq);
    float fo[8], fd[8];
    unpack8<E>(ld16(p.o + b * p.os[0] + hq * p.os[1] + i * p.os[2] + 8 * ch), fo);
    unpack8<E>(ld16(p.dout + b * p.dos[0] + hq * p.dos[1] + i * p.dos[2] + 8 * ch), fd);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += fo[e] * fd[e];
  }
#pragma unroll
  for (int off = 1; off < CPR; off <<= 1) acc += __shfl_xor(acc, off, 64);
  if (r < total && ch == 0) p.delta[r] = acc;
}

// ---------------------------------------------------------------------------
// 32-row tile staging.  A unit is (row pair rp, rotate-half pair j): rows
// 2rp, 2rp+1 and the 16-byte chunks j and j + D/16 of each.  The tile is
// written row-major (pitch D+8) and, when TRANS, transposed (pitch 40) as
// packed (row 2rp, row 2rp+1) words.
// ---------------------------------------------------------------------------
template <class E, int D, bool ROPE, bool TRANS>
struct Tile32 {
  static constexpr int UNITS = 16 * (D / 16);
  static constexpr int RP = D + 8;     // row-major pitch
  static constexpr int TP = 32 + 8;    // transposed pitch
  u32x4 x[2][2];                        // [row][lo/hi]
  u32x4 cs[ROPE ? 2 : 1][2], sn[ROPE ? 2 : 1][2];
  int unit = -1;

  // Rows past the end of the tensor (or of the RoPE tables) fall outside the
  // buffer resource and load as zeros.
  __device__ void load(int u, __amdgpu_buffer_rsrc_t xr, int64_t rstride, int r0,
                       __amdgpu_buffer_rsrc_t cr, __amdgpu_buffer_rsrc_t sr, int64_t cstride) {
    unit = u;
    const int rp = u / (D / 16), j = u % (D / 16);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = r0 + 2 * rp + t;
      const uint32_t off = (uint32_t)((row * rstride + 8 * j) * 2);
      x[t][0] = buf_ld16(xr, off);
      x[t][1] = buf_ld16(xr, off + D);
      if constexpr (ROPE) {
        const uint32_t co = (uint32_t)((row * cstride + 8 * j) * 2);
        cs[t][0] = buf_ld16(cr, co);
        cs[t][1] = buf_ld16(cr, co + D);
        sn[t][0] = buf_ld16(sr, co);
        sn[t][1] = buf_ld16(sr, co + D);
      }
    }
  }

  __device__ void store(uint16_t* rows, uint16_t* trans) {
    const int rp = unit / (D / 16), j = unit % (D / 16);
    if constexpr (ROPE) {
#pragma unroll
      for (int t = 0; t < 2; ++t) rope_pair<E>(x[t][0], x[t][1], cs[t][0], sn[t][0], cs[t][1], sn[t][1]);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      st16(rows + (2 * rp + t) * RP + 8 * j, x[t][0]);
      st16(rows + (2 * rp + t) * RP + 8 * j + D / 2, x[t][1]);
    }
    if constexpr (TRANS) {
      uint32_t* t32 = reinterpret_cast<uint32_t*>(trans);
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t a = x[0][half][e >> 1], bq = x[1][half][e >> 1];
          const uint32_t word = (e & 1) ? ((a >> 16) | (bq & 0xffff0000u)) : ((a & 0xffffu) | (bq << 16));
          const int d = 8 * j + half * (D / 2) + e;
          t32[(d * TP + 2 * rp) >> 1] = word;
        }
    }
  }
};

// Registers of a 32-row operand held by a wave: lane (h, c) holds row c,
// dims 16 ks + 8 h .. +7, rotated when ROPE.
template <class E, int D, bool ROPE>
__device__ inline void load_operand_rows(u32x4* f, const uint16_t* base, int64_t rstride, int row, int nvalid,
                                         const uint16_t* cos, const uint16_t* sin, int64_t cstride, int h) {
  constexpr int KS = D / 16;
  const bool ok = row < nvalid;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) f[ks] = ok ? ld16(base + row * rstride + 16 * ks + 8 * h) : u32x4{0, 0, 0, 0};
  if constexpr (ROPE) {
    if (ok) {
      const uint16_t* cr = cos + row * cstride;
      const uint16_t* sr = sin + row * cstride;
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks) {
        const int dl = 16 * ks + 8 * h, dh = dl + D / 2;
        rope_pair<E>(f[ks], f[ks + KS / 2], ld16(cr + dl), ld16(sr + dl), ld16(cr + dh), ld16(sr + dh));
      }
    }
  }
}

// Store a transposed 32x32-block gradient accumulator (rows = dims,
// column = this lane's row `row`) as out[row][d], applying the scale and,
// with ROPE, the inverse rotation R^T at position `row`.
template <class E, int D, bool ROPE>
__device__ inline void store_grad_rows(f32x16* acc, uint16_t* out, int64_t rstride, int row, int nvalid,
                                       float scale, const uint16_t* cos, const uint16_t* sin, int64_t cstride,
                                       int h) {
  constexpr int DB = D / 32;
  if (row >= nvalid) return;
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] *= scale;
  if constexpr (ROPE) {
    const uint16_t* cr = cos + row * cstride;
    const uint16_t* sr = sin + row * cstride;
    // register group (db, g) holds dims 32 db + 8 g + 4 h + e; its rotate-half
    // partner d + D/2 is group (dbh, gh) of the same lane.
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (32 * db + 8 * g >= D / 2) continue;
        const int dbh = (32 * db + 8 * g + D / 2) / 32, gh = ((8 * g + D / 2) % 32) / 8;
        const int dl = 32 * db + 8 * g + 4 * h, dh = dl + D / 2;
        const u32x2 cl = *reinterpret_cast<const u32x2*>(cr + dl);
        const u32x2 sl = *reinterpret_cast<const u32x2*>(sr + dl);
        const u32x2 ch = *reinterpret_cast<const u32x2*>(cr + dh);
        const u32x2 sh = *reinterpret_cast<const u32x2*>(sr + dh);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t wcl = cl[e >> 1], wsl = sl[e >> 1], wch = ch[e >> 1], wsh = sh[e >> 1];
          const float fcl = (e & 1) ? E::hi(wcl) : E::lo(wcl);
          const float fsl = (e & 1) ? E::hi(wsl) : E::lo(wsl);
          const float fch = (e & 1) ? E::hi(wch) : E::lo(wch);
          const float fsh = (e & 1) ? E::hi(wsh) : E::lo(wsh);
          float glo = acc[db][4 * g + e], ghi = acc[dbh][4 * gh + e];
          rope_grad_pair(glo, ghi, fcl, fsl, fch, fsh);
          acc[db][4 * g + e] = glo;
          acc[dbh][4 * gh + e] = ghi;
        }
      }
  }
  uint16_t* orow = out + row * rstride;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + 8 * g + 4 * h;
      u32x2 w2;
      w2[0] = E::pack(acc[db][4 * g], acc[db][4 * g + 1]);
      w2[1] = E::pack(acc[db][4 * g + 2], acc[db][4 * g + 3]);
      *reinterpret_cast<u32x2*>(orow + d0) = w2;
    }
}

// Masking of one score element (query i, key j); the range logic of the
// forward kernel decides which tiles are visited at all.
template <int MASK>
__device__ __forceinline__ bool visible(int i, int j, int Nq, int Nkv, int W) {
  bool ok = i < Nq && j < Nkv;
  if constexpr (MASK == MASK_CAUSAL) ok = ok && j <= i;
  if constexpr (MASK == MASK_SW) ok = ok && abs(i - j) < W;
  if constexpr (MASK == MASK_CSW) ok = ok && j <= i && i - j < W;
  return ok;
}

// Byte range of `rows` rows of D elements at `rstride` elements apart.
template <int D>
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t rstride) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * rstride + D) * 2) : 0u;
}

// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) bwd_dkv_kernel(const BwdParams p) {
  constexpr int NT = WAVES * 64;
  constexpr int BK = 32 * WAVES;
  constexpr int KS = D / 16, DB = D / 32;
  using QT = Tile32<E, D, ROPE, true>;
  using OT = Tile32<E, D, false, true>;
  constexpr int RP = QT::RP, TP = QT::TP;
  constexpr int ROWS = 32 * RP, TRS = D * TP;
  constexpr int STAGE = 2 * ROWS + 2 * TRS + 2 * 2 * 32;   // halves; 64 floats at the end
  constexpr int UPT = (2 * QT::UNITS + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  // key block outermost: under a causal mask the first key blocks see the
  // most query tiles, so they are dispatched first.
  // no keys: nothing to write (the launch still has one workgroup)
  if (p.n_kblocks <= 0) return;
  // key block outermost: under a causal mask the first key blocks see the
  // most query tiles, so they are dispatched first.
  const int BHK = p.B * p.Hkv;
  const int kb = blockIdx.x / BHK;
  const int bhk = blockIdx.x % BHK;
  const int hk = bhk % p.Hkv, b = bhk / p.Hkv;
  const int n0 = kb * BK;
  const int n0w = n0 + 32 * w;
  const int key = n0w + c;

  // k~ and v for this wave's 32 keys, as B operands (lane: row c).
  u32x4 kf[KS], vf[KS];
  load_operand_rows<E, D, ROPE>(kf, p.k + b * p.ks[0] + hk * p.ks[1], p.ks[2], key, p.Nkv, p.cos, p.sin,
                                p.rs[0], h);
  load_operand_rows<E, D, false>(vf, p.v + b * p.vs[0] + hk * p.vs[1], p.vs[2], key, p.Nkv, nullptr, nullptr, 0,
                                 h);

  // query-tile schedule (tiles of 32 rows) for one head
  int m_lo = 0, m_hi = p.Nq, ntq;
  int bs_sub = 1, bs_n = 0;
  const int32_t* bs_row = nullptr;
  if constexpr (MASK == MASK_CAUSAL) {
    m_lo = n0 & ~31;
  } else if constexpr (MASK == MASK_SW) {
    m_lo = max(n0 - p.window + 1, 0) & ~31;
    m_hi = min(n0 + BK - 1 + p.window, p.Nq);
  } else if constexpr (MASK == MASK_CSW) {
    m_lo = n0 & ~31;
    m_hi = min(n0 + BK - 1 + p.window, p.Nq);
  }
  if constexpr (MASK == MASK_BS) {
    bs_sub = p.bs_block_m / 32;
    bs_n = p.bs_q_num[kb];
    bs_row = p.bs_q_idx + kb * p.bs_q_rs;
    ntq = bs_n * bs_sub;
  } else {
    ntq = m_hi > m_lo ? (m_hi - m_lo + 31) / 32 : 0;
  }
  auto tile_m0 = [&](int t) -> int {
    if constexpr (MASK == MASK_BS) {
      const int e = t / bs_sub;
      return bs_row[e] * p.bs_block_m + (t - e * bs_sub) * 32;
    } else {
      return m_lo + 32 * t;
    }
  };
  const int ntiles = ntq * p.G;

  QT qt[UPT];
  OT ot[UPT];
  float lreg = 0.f, dreg = 0.f;
  const uint32_t rope_bytes = ROPE ? span_bytes<D>(p.rope_len, p.rs[0]) : 0u;
  const auto crs = make_rsrc(p.cos, rope_bytes);
  const auto srs = make_rsrc(p.sin, rope_bytes);
  auto stage_load = [&](int t) {
    const int gi = t / ntq, hq = hk * p.G + gi;
    const int m0 = tile_m0(t - gi * ntq);
    const auto qrs = make_rsrc(p.q + b * p.qs[0] + hq * p.qs[1], span_bytes<D>(p.Nq, p.qs[2]));
    const auto ors = make_rsrc(p.dout + b * p.dos[0] + hq * p.dos[1], span_bytes<D>(p.Nq, p.dos[2]));
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * NT;
      if (u < QT::UNITS)
        qt[i].load(u, qrs, p.qs[2], m0, crs, srs, p.rs[0]);
      else if (u < 2 * QT::UNITS)
        ot[i].load(u - QT::UNITS, ors, p.dos[2], m0, crs, srs, 0);
    }
    if (tid < 32) {
      const int row = m0 + tid;
      const bool ok = row >= 0 && row < p.Nq;
      const float L = ok ? p.lse[b * p.ls[0] + hq * p.ls[1] + row * p.ls[2]] : 0.f;
      lreg = (L == -INFINITY) ? 0.f : L * kLog2e;
      dreg = ok ? p.delta[((int64_t)b * p.Hq + hq) * p.Nq + row] : 0.f;
    }
  };
  auto stage_store = [&](uint16_t* buf) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * NT;
      if (u < QT::UNITS) qt[i].store(buf, buf + 2 * ROWS);
      else if (u < 2 * QT::UNITS) ot[i].store(buf + ROWS, buf + 2 * ROWS + TRS);
    }
    float* f = reinterpret_cast<float*>(buf + 2 * ROWS + 2 * TRS);
    if (tid < 32) {
      f[tid] = lreg;
      f[32 + tid] = dreg;
    }
  };

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  const float c2 = p.scale * kLog2e;
  constexpr bool kAlibiOneSided = BIAS == BIAS_ALIBI && (MASK == MASK_CAUSAL || MASK == MASK_CSW);

  if (ntiles > 0) {
    stage_load(0);
    stage_store(lds);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const bool more = t + 1 < ntiles;
    if (more) stage_load(t + 1);
    const int gi = t / ntq, hq = hk * p.G + gi;
    const int m0 = tile_m0(t - gi * ntq);
    const uint16_t* buf = lds + (t & 1) * STAGE;
    const uint16_t* Qs = buf;
    const uint16_t* dOs = buf + ROWS;
    const uint16_t* Qt = buf + 2 * ROWS;
    const uint16_t* dOt = buf + 2 * ROWS + TRS;
    const float* Ls = reinterpret_cast<const float*>(buf + 2 * ROWS + 2 * TRS);
    const float* Dl = Ls + 32;

    bool active = n0w < p.Nkv && m0 < p.Nq;
    if constexpr (MASK == MASK_CAUSAL) active = active && m0 + 31 >= n0w;
    if constexpr (MASK == MASK_SW) active = active && m0 + 31 > n0w - p.window && m0 < n0w + 31 + p.window;
    if constexpr (MASK == MASK_CSW) active = active && m0 + 31 >= n0w && m0 < n0w + 31 + p.window;
    if (active) {
      // S and dP (queries x keys), query rows permuted.
      f32x16 s = f32x16{}, dp = f32x16{};
      const uint16_t* qrow = Qs + kperm(c) * RP + 8 * h;
      const uint16_t* orow = dOs + kperm(c) * RP + 8 * h;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s = E::mfma32(ld16(qrow + 16 * ks), kf[ks], s);
        dp = E::mfma32(ld16(orow + 16 * ks), vf[ks], dp);
      }
      float slope2 = 0.f;
      if constexpr (BIAS == BIAS_ALIBI) slope2 = p.slopes[hq] * kLog2e;
      // only tiles that cross the diagonal / window edge or run past an
      // end need the per-element test
      bool need_mask = m0 + 32 > p.Nq || n0w + 32 > p.Nkv;
      if constexpr (MASK == MASK_CAUSAL) need_mask = need_mask || n0w + 31 > m0;
      if constexpr (MASK == MASK_SW)
        need_mask = need_mask || m0 + 31 - n0w >= p.window || n0w + 31 - m0 >= p.window;
      if constexpr (MASK == MASK_CSW) need_mask = need_mask || n0w + 31 > m0 || m0 + 31 - n0w >= p.window;
      // logits in log2 units: register r holds query m0 + 16 (r/8) + 8h + r%8
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // causal-type masks see only j <= i, where -slope |i - j| is linear
        // in the query index (one add per element)
        float abias = 0.f;
        if constexpr (kAlibiOneSided) abias = slope2 * (float)(key - (m0 + 16 * j + 8 * h));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          float x = s[r] * c2;
          if constexpr (kAlibiOneSided) {
            x += abias;
            abias -= slope2;
          } else if constexpr (BIAS == BIAS_ALIBI) {
            x -= slope2 * (float)abs(m0 + 16 * j + 8 * h + e - key);
          }
          s[r] = x;
        }
      }
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = m0 + 16 * (r >> 3) + 8 * h + (r & 7);
          s[r] = visible<MASK>(qi, key, p.Nq, p.Nkv, p.window) ? s[r] : -INFINITY;
        }
      }
      u32x4 pp[2], pd[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4 l4a = *reinterpret_cast<const f32x4*>(Ls + 16 * j + 8 * h);
        const f32x4 l4b = *reinterpret_cast<const f32x4*>(Ls + 16 * j + 8 * h + 4);
        const f32x4 d4a = *reinterpret_cast<const f32x4*>(Dl + 16 * j + 8 * h);
        const f32x4 d4b = *reinterpret_cast<const f32x4*>(Dl + 16 * j + 8 * h + 4);
        float pv[8], dsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          const float L2 = e < 4 ? l4a[e] : l4b[e - 4];
          const float dl = e < 4 ? d4a[e] : d4b[e - 4];
          const float pr = __builtin_amdgcn_exp2f(s[r] - L2);
          pv[e] = pr;
          dsv[e] = pr * (dp[r] - dl);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pp[j][i] = E::pack(pv[2 * i], pv[2 * i + 1]);
          pd[j][i] = E::pack(dsv[2 * i], dsv[2 * i + 1]);
        }
      }
      // dV^T += dO^T P,  dK~^T += Q~^T dS   (contraction over 32 queries)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t* otr = dOt + (32 * db + c) * TP + 8 * h;
        const uint16_t* qtr = Qt + (32 * db + c) * TP + 8 * h;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          dv[db] = E::mfma32(ld16(otr + 16 * j), pp[j], dv[db]);
          dk[db] = E::mfma32(ld16(qtr + 16 * j), pd[j], dk[db]);
        }
      }
    }
    if (more) stage_store(lds + ((t + 1) & 1) * STAGE);
    __syncthreads();
  }

  uint16_t* dkb = p.dk + b * p.dks[0] + hk * p.dks[1];
  uint16_t* dvb = p.dv + b * p.dvs[0] + hk * p.dvs[1];
  store_grad_rows<E, D, false>(dv, dvb, p.dvs[2], key, p.Nkv, 1.f, nullptr, nullptr, 0, h);
  store_grad_rows<E, D, ROPE>(dk, dkb, p.dks[2], key, p.Nkv, p.scale, p.cos, p.sin, p.rs[0], h);
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) bwd_dq_kernel(const BwdParams p) {
  constexpr int NT = WAVES * 64;
  constexpr int BMq = 32 * WAVES;
  constexpr int KS = D / 16, DB = D / 32;
  using KT = Tile32<E, D, ROPE, true>;
  using VT = Tile32<E, D, false, false>;
  constexpr int RP = KT::RP, TP = KT::TP;
  constexpr int ROWS = 32 * RP, TRS = D * TP;
  constexpr int STAGE = 2 * ROWS + TRS;
  constexpr int UPT = (2 * KT::UNITS + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  // no queries: nothing to write (the launch still has one workgroup)
  if (p.n_qblocks <= 0) return;
  const int BH = p.B * p.Hq;
  const int bh = blockIdx.x % BH;
  const int mbi = blockIdx.x / BH;
  const bool heavy_last = MASK == MASK_CAUSAL || MASK == MASK_CSW;
  const int mb = heavy_last ? (p.n_qblocks - 1 - mbi) : mbi;
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.G;
  const int m0 = mb * BMq, q0w = m0 + 32 * w, qrow = q0w + c;

  u32x4 qf[KS], of[KS];
  load_operand_rows<E, D, ROPE>(qf, p.q + b * p.qs[0] + hq * p.qs[1], p.qs[2], qrow, p.Nq, p.cos, p.sin, p.rs[0],
                                h);
  load_operand_rows<E, D, false>(of, p.dout + b * p.dos[0] + hq * p.dos[1], p.dos[2], qrow, p.Nq, nullptr,
                                 nullptr, 0, h);
  float L2 = 0.f, dl = 0.f;
  if (qrow < p.Nq) {
    const float L = p.lse[b * p.ls[0] + hq * p.ls[1] + qrow * p.ls[2]];
    L2 = (L == -INFINITY) ? 0.f : L * kLog2e;
    dl = p.delta[((int64_t)b * p.Hq + hq) * p.Nq + qrow];
  }

  int n_lo = 0, n_hi = p.Nkv, ntiles;
  int bs_nfull = 0, bs_sub = 1;
  const int32_t* bs_full_row = nullptr;
  const int32_t* bs_part_row = nullptr;
  if constexpr (MASK == MASK_CAUSAL) {
    n_hi = min(m0 + BMq, p.Nkv);
  } else if constexpr (MASK == MASK_SW) {
    n_lo = max(m0 - p.window + 1, 0) & ~31;
    n_hi = min(m0 + BMq - 1 + p.window, p.Nkv);
  } else if constexpr (MASK == MASK_CSW) {
    n_lo = max(m0 - p.window + 1, 0) & ~31;
    n_hi = min(m0 + BMq, p.Nkv);
  }
  if constexpr (MASK == MASK_BS) {
    bs_sub = p.bs_block_n / 32;
    bs_nfull = p.bs_full_num[mb];
    bs_full_row = p.bs_full_idx + mb * p.bs_full_rs;
    bs_part_row = p.bs_part_idx + mb * p.bs_part_rs;
    ntiles = (bs_nfull + p.bs_part_num[mb]) * bs_sub;
  } else {
    ntiles = n_hi > n_lo ? (n_hi - n_lo + 31) / 32 : 0;
  }
  auto tile_n0 = [&](int t) -> int {
    if constexpr (MASK == MASK_BS) {
      const int e = t / bs_sub;
      const int blk = e < bs_nfull ? bs_full_row[e] : bs_part_row[e - bs_nfull];
      return blk * p.bs_block_n + (t - e * bs_sub) * 32;
    } else {
      return n_lo + 32 * t;
    }
  };

  const uint16_t* kbase = p.k + b * p.ks[0] + hk * p.ks[1];
  const uint16_t* vbase = p.v + b * p.vs[0] + hk * p.vs[1];
  KT kt[UPT];
  VT vt[UPT];
  const auto krs = make_rsrc(kbase, span_bytes<D>(p.Nkv, p.ks[2]));
  const auto vrs = make_rsrc(vbase, span_bytes<D>(p.Nkv, p.vs[2]));
  const uint32_t rope_bytes = ROPE ? span_bytes<D>(p.rope_len, p.rs[0]) : 0u;
  const auto crs = make_rsrc(p.cos, rope_bytes);
  const auto srs = make_rsrc(p.sin, rope_bytes);
  auto stage_load = [&](int t) {
    const int n0 = tile_n0(t);
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * NT;
      if (u < KT::UNITS)
        kt[i].load(u, krs, p.ks[2], n0, crs, srs, p.rs[0]);
      else if (u < 2 * KT::UNITS)
        vt[i].load(u - KT::UNITS, vrs, p.vs[2], n0, crs, srs, 0);
    }
  };
  auto stage_store = [&](uint16_t* buf) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * NT;
      if (u < KT::UNITS) kt[i].store(buf, buf + 2 * ROWS);
      else if (u < 2 * KT::UNITS) vt[i].store(buf + ROWS, nullptr);
    }
  };

  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = f32x16{};
  const float c2 = p.scale * kLog2e;
  float slope2 = 0.f;
  if constexpr (BIAS == BIAS_ALIBI) slope2 = p.slopes[hq] * kLog2e;
  constexpr bool kAlibiOneSided = BIAS == BIAS_ALIBI && (MASK == MASK_CAUSAL || MASK == MASK_CSW);

  if (ntiles > 0) {
    stage_load(0);
    stage_store(lds);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const bool more = t + 1 < ntiles;
    if (more) stage_load(t + 1);
    const int n0 = tile_n0(t);
    const uint16_t* buf = lds + (t & 1) * STAGE;
    const uint16_t* Ks = buf;
    const uint16_t* Vs = buf + ROWS;
    const uint16_t* Kt = buf + 2 * ROWS;

    bool active = q0w < p.Nq && n0 >= 0 && n0 < p.Nkv;
    if constexpr (MASK == MASK_CAUSAL) active = active && n0 <= q0w + 31;
    if constexpr (MASK == MASK_SW) active = active && n0 + 31 > q0w - p.window && n0 < q0w + 31 + p.window;
    if constexpr (MASK == MASK_CSW) active = active && n0 + 31 > q0w - p.window && n0 <= q0w + 31;
    if (active) {
      f32x16 s = f32x16{}, dp = f32x16{};
      const uint16_t* krow = Ks + kperm(c) * RP + 8 * h;
      const uint16_t* vrow = Vs + kperm(c) * RP + 8 * h;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s = E::mfma32(ld16(krow + 16 * ks), qf[ks], s);
        dp = E::mfma32(ld16(vrow + 16 * ks), of[ks], dp);
      }
      bool need_mask = q0w + 32 > p.Nq || n0 + 32 > p.Nkv;
      if constexpr (MASK == MASK_CAUSAL) need_mask = need_mask || n0 + 31 > q0w;
      if constexpr (MASK == MASK_SW)
        need_mask = need_mask || q0w + 31 - n0 >= p.window || n0 + 31 - q0w >= p.window;
      if constexpr (MASK == MASK_CSW) need_mask = need_mask || n0 + 31 > q0w || q0w + 31 - n0 >= p.window;
      // logits in log2 units: register r holds key n0 + 16 (r/8) + 8h + r%8
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float abias = 0.f;
        if constexpr (kAlibiOneSided) abias = slope2 * (float)(n0 + 16 * j + 8 * h - qrow);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          float x = s[r] * c2;
          if constexpr (kAlibiOneSided) {
            x += abias;
            abias += slope2;
          } else if constexpr (BIAS == BIAS_ALIBI) {
            x -= slope2 * (float)abs(qrow - (n0 + 16 * j + 8 * h + e));
          }
          s[r] = x;
        }
      }
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kj = n0 + 16 * (r >> 3) + 8 * h + (r & 7);
          s[r] = visible<MASK>(qrow, kj, p.Nq, p.Nkv, p.window) ? s[r] : -INFINITY;
        }
      }
      u32x4 pd[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float dsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          const float pr = __builtin_amdgcn_exp2f(s[r] - L2);
          dsv[e] = pr * (dp[r] - dl);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) pd[j][i] = E::pack(dsv[2 * i], dsv[2 * i + 1]);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t* ktr = Kt + (32 * db + c) * TP + 8 * h;
#pragma unroll
        for (int j = 0; j < 2; ++j) dq[db] = E::mfma32(ld16(ktr + 16 * j), pd[j], dq[db]);
      }
    }
    if (more) stage_store(lds + ((t + 1) & 1) * STAGE);
    __syncthreads();
  }

  store_grad_rows<E, D, ROPE>(dq, p.dq + b * p.dqs[0] + hq * p.dqs[1], p.dqs[2], qrow, p.Nq, p.scale, p.cos,
                              p.sin, p.rs[0], h);
}

}  // namespace af
