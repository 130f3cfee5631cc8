// Attention backward for gfx950 (piece (c), with the block-sparse walk of
// piece (d)).
//
// Math (FA2; reference: attnfuse/compiler/codegen_backward.py:45-302):
//   delta_i = sum_d dO_id O_id
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
//  * bwd_prep_kernel: delta and L log2(e) per query row (one 8-byte pair,
//    streamed into LDS with the query tiles), and with RoPE the rotated q~ and
//    k~ written once to the workspace, rounded to the input dtype exactly as
//    the forward rounds them in registers.  Every query tile is read by all
//    key blocks (and every key tile by all query blocks), so rotating once
//    replaces one rotation (and one cos/sin read) per visit.
//  * dK/dV body (bwd_dkv_body): a workgroup owns 32*WAVES keys of one
//    (batch, kv head);
//    each wave owns 32 keys, k~ in registers (and v too for D <= 64; for
//    D = 128 the workgroup's V block sits in LDS so that the dK/dV
//    accumulators, k~ and the score tiles fit two waves per SIMD).  It walks
//    the 32-row query tiles of every query head of the GQA group, so dK/dV
//    come out group-summed with no atomics.  Scores are S (queries x keys)
//    with the query rows permuted (kperm), so P and dS feed the dV^T and dK^T
//    MFMAs straight from registers.
//  * dQ body (bwd_dq_body): a workgroup owns 32*WAVES query rows of one
//    (batch, head); q~ and dO stay in registers; 32-key tiles of k~ and v
//    stream through LDS.  Scores are S^T (keys x queries) so dS^T is the B
//    operand of the dQ^T MFMA.
//  * bwd_dkvdq_kernel runs both bodies in one launch, dK/dV workgroups
//    first (bwd_dkv_kernel / bwd_dq_kernel run them alone where the two
//    bodies want different widths or registers).  The heavy key blocks of a
//    causal mask split their GQA group over g_split workgroups that write
//    fp32 partials, summed by bwd_dkv_combine_kernel.
//  * In the 128-dim bodies every MFMA operand read from LDS is issued a few
//    MFMAs (or k-steps) ahead of its MFMA (AF_*_AHEAD), so the MFMAs do not
//    each wait out an LDS round trip.
//  * LDS tiles are row-major with no padding and an XOR swizzle of their
//    16-byte chunks (lds_swz): the row reads of the score MFMAs and the
//    transposing reads (ds_read_b64_tr_b16) of the gradient MFMAs both hit
//    64 distinct banks, so no transposed copy of any tile is stored.
//  * Tiles are staged in a ring of two or three LDS slots: buffer loads
//    (rows past the end load as zeros) of the next tiles are in flight while
//    tile t is on the MFMA pipes.
#pragma once

#include "af_common.hpp"
#include "fwd_kernel.hpp"
#include "rope_kernel.hpp"

namespace af {

#ifndef AF_DKV_TR_AHEAD
#define AF_DKV_TR_AHEAD(D) ((D) == 128 ? 4 : 0)
#endif
#ifndef AF_DQ_TR_AHEAD
#define AF_DQ_TR_AHEAD(D) ((D) == 128 ? 4 : 0)
#endif
#ifndef AF_DKV_S_AHEAD
#define AF_DKV_S_AHEAD(D) ((D) == 128 ? 2 : 0)
#endif
#ifndef AF_DQ_S_AHEAD
#define AF_DQ_S_AHEAD(D) ((D) == 128 ? 2 : 0)
#endif

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  // (B, Hq, Nq) fp32 pairs {L log2(e) (0 for a row that sees no key),
  // delta}, workspace: one row's pair is 8 contiguous bytes, so a query
  // tile's 32 pairs load into LDS with one wave instruction
  float* ld;
  uint16_t* qr;            // RoPE: q~ workspace, (B, Hq, Nq, D) contiguous
  uint16_t* kr;            // RoPE: k~ workspace, (B, Hkv, Nkv, D) contiguous
  const uint16_t* qt;      // q~ as the score kernels read it (qr, or q)
  const uint16_t* kt;      // k~ likewise (kr, or k)
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
  // Element masks of partial tiles (all three NULL, or none): row bits of
  // the Q-major partial entries, (n_q_blocks, bs_part_rs, BLOCK_M,
  // BLOCK_N / 64) words over keys; column bits of the K-major entries,
  // (n_kv_blocks, bs_q_rs, BLOCK_N, ceil(BLOCK_M / 64)) words over queries;
  // and which K-major entries are partial, (n_kv_blocks, bs_q_rs).
  const uint64_t* bs_row_bits;
  const uint64_t* bs_col_bits;
  const int32_t* bs_q_partial;
  int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4], ls[3], rs[2];
  int64_t qts[4], kts[4];  // strides of qt, kt
  int64_t bs_full_rs, bs_part_rs, bs_q_rs;
  int32_t B, Hq, Hkv, Nq, Nkv, G, window;
  int32_t bs_block_m, bs_block_n;
  int32_t n_qblocks, n_kblocks;   // workgroup tiling of the two kernels
  int32_t rope_len;               // rows of the RoPE tables
  // dK/dV: the G query heads of a key/value head are split over g_split
  // workgroups per key block; with g_split > 1 each writes fp32 partial sums
  // (unscaled, rotated space) to dkp / dvp, (g_split, B, Hkv, Nkv, D), and
  // bwd_dkv_combine_kernel adds them up.
  int32_t g_split;
  // Only key blocks [0, n_split_kb) are split (their workgroups come first);
  // the last, lightest ones of a causal mask run all G heads in one
  // workgroup and store dK/dV directly.  split_keys = the key rows of the
  // split blocks (min(n_split_kb * BLOCK_N, N_kv)), the rows the combine sums.
  int32_t n_split_kb, split_keys;
  float* dkp;
  float* dvp;
  // Block-sparse work plans (nullable): grid row i of the dQ kernel is item
  // i of bs_q_items, of the dK/dV kernel item i of bs_kv_items (list, first
  // entry, entries, slot); slot >= 0 writes fp32 partial sums (unscaled,
  // rotated space) to part_dq (slot, B*Hq, BLOCK_M, D) or part_dk / part_dv
  // (slot, B*Hkv, BLOCK_N, D) for bs_grad_combine_kernel.  The K-major plan
  // is used with g_split == 1 only.
  const int32_t* bs_q_items;
  const int32_t* bs_kv_items;
  float* part_dq;
  float* part_dk;
  float* part_dv;
  // bwd_dkvdq_kernel: workgroups [0, n_dkv_wg) run dK/dV, the rest dQ
  int32_t n_dkv_wg;
  // block-sparse walks: rows of the dQ grid (plan items or query blocks),
  // and heads per XCD group of the dQ and the dK/dV grids
  // (xcd_head_groups), 0 = off
  int32_t bs_q_rows, bs_xcd_heads_q, bs_xcd_heads_kv;
  float scale;
};

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) and L log2(e), fp32; with RoPE also q~ and k~ into
// the workspace.
// A row is handled by D/16 threads, thread j holding the rotate-half pair of
// chunks j and j + D/16.  Rows [0, B*Hq*Nq) are query rows, the next
// B*Hkv*Nkv (RoPE only) key rows.
// ---------------------------------------------------------------------------
template <class E, int D, bool ROPE>
__global__ void __launch_bounds__(256) bwd_prep_kernel(const BwdParams p) {
  constexpr int TPR = D / 16;          // threads per row
  constexpr int RPB = 256 / TPR;       // rows per workgroup
  const int tid = threadIdx.x;
  const int64_t r = (int64_t)blockIdx.x * RPB + tid / TPR;
  const int j = tid % TPR;
  const int64_t nq = (int64_t)p.B * p.Hq * p.Nq;
  const int64_t nk = ROPE ? (int64_t)p.B * p.Hkv * p.Nkv : 0;
  if (r < nq) {
    const int i = (int)(r % p.Nq);
    const int64_t bh = r / p.Nq;
    const int hq = (int)(bh % p.Hq), b = (int)(bh / p.Hq);
    const uint16_t* orow = p.o + b * p.os[0] + hq * p.os[1] + i * p.os[2];
    const uint16_t* drow = p.dout + b * p.dos[0] + hq * p.dos[1] + i * p.dos[2];
    float fo[8], fd[8], acc = 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      unpack8<E>(ld16(orow + 8 * j + half * (D / 2)), fo);
      unpack8<E>(ld16(drow + 8 * j + half * (D / 2)), fd);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += fo[e] * fd[e];
    }
#pragma unroll
    for (int off = 1; off < TPR; off <<= 1) acc += __shfl_xor(acc, off, 64);
    if (j == 0) {
      const float L = p.lse[b * p.ls[0] + hq * p.ls[1] + i * p.ls[2]];
      *reinterpret_cast<f32x2*>(p.ld + 2 * r) = f32x2{(L == -INFINITY) ? 0.f : L * kLog2e, acc};
    }
    if constexpr (ROPE) {
      rope_row_chunk<E, D>(p.q + b * p.qs[0] + hq * p.qs[1] + i * p.qs[2], p.cos + i * p.rs[0],
                           p.sin + i * p.rs[0], p.qr + r * D, j);
    }
  } else if (ROPE && r < nq + nk) {
    const int64_t rk = r - nq;
    const int n = (int)(rk % p.Nkv);
    const int64_t bh = rk / p.Nkv;
    const int hk = (int)(bh % p.Hkv), b = (int)(bh / p.Hkv);
    rope_row_chunk<E, D>(p.k + b * p.ks[0] + hk * p.ks[1] + n * p.ks[2], p.cos + n * p.rs[0],
                         p.sin + n * p.rs[0], p.kr + rk * D, j);
  }
}

// Registers of a 32-row operand held by a wave: lane (h, c) holds row c,
// dims 16 ks + 8 h .. +7 (rows past nvalid are zero).
template <int D>
__device__ inline void load_operand_rows(u32x4* f, const uint16_t* base, int64_t rstride, int row, int nvalid,
                                         int h) {
  constexpr int KS = D / 16;
  const bool ok = row < nvalid;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) f[ks] = ok ? ld16(base + row * rstride + 16 * ks + 8 * h) : u32x4{0, 0, 0, 0};
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

// fp32 row of a transposed 32x32-block accumulator (rows = dims, column =
// this lane's row): register 4g + e of block db is dim 32 db + 8 g + 4 h + e.
template <int D>
__device__ inline void store_partial_row(const f32x16* acc, float* out, int h) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + 8 * g + 4 * h;
      *reinterpret_cast<f32x4*>(out + d0) =
          f32x4{acc[db][4 * g], acc[db][4 * g + 1], acc[db][4 * g + 2], acc[db][4 * g + 3]};
    }
}

// dK, dV of key row n = the sum of the g_split partial rows; dK is scaled and,
// with RoPE, rotated back to the input space (the transpose of rotate-half).
// Thread j of a row handles dims [8 j, 8 j + 8) and their rotate-half
// partners [8 j + D/2, ...).
template <class E, int D, bool ROPE>
__global__ void __launch_bounds__(256) bwd_dkv_combine_kernel(const BwdParams p) {
  constexpr int TPR = D / 16;
  constexpr int RPB = 256 / TPR;
  const int tid = threadIdx.x;
  // rows of the split key blocks only: (b, hk, n < split_keys)
  const int64_t rs = (int64_t)blockIdx.x * RPB + tid / TPR;
  if (rs >= (int64_t)p.B * p.Hkv * p.split_keys) return;
  const int64_t rows = (int64_t)p.B * p.Hkv * p.Nkv;
  const int j = tid % TPR;
  const int n = (int)(rs % p.split_keys);
  const int64_t bh = rs / p.split_keys;
  const int64_t r = bh * p.Nkv + n;
  const int hk = (int)(bh % p.Hkv), b = (int)(bh / p.Hkv);
  const int dl = 8 * j, dh = dl + D / 2;
  float vlo[8], vhi[8], klo[8], khi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) vlo[e] = vhi[e] = klo[e] = khi[e] = 0.f;
  for (int sp = 0; sp < p.g_split; ++sp) {
    const int64_t off = (sp * rows + r) * D;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p.dvp + off + dl + 4 * q);
      const f32x4 c = *reinterpret_cast<const f32x4*>(p.dvp + off + dh + 4 * q);
      const f32x4 x = *reinterpret_cast<const f32x4*>(p.dkp + off + dl + 4 * q);
      const f32x4 y = *reinterpret_cast<const f32x4*>(p.dkp + off + dh + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vlo[4 * q + e] += a[e];
        vhi[4 * q + e] += c[e];
        klo[4 * q + e] += x[e];
        khi[4 * q + e] += y[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    klo[e] *= p.scale;
    khi[e] *= p.scale;
  }
  if constexpr (ROPE) {
    float cl[8], sl[8], ch[8], sh[8];
    unpack8<E>(ld16(p.cos + n * p.rs[0] + dl), cl);
    unpack8<E>(ld16(p.sin + n * p.rs[0] + dl), sl);
    unpack8<E>(ld16(p.cos + n * p.rs[0] + dh), ch);
    unpack8<E>(ld16(p.sin + n * p.rs[0] + dh), sh);
#pragma unroll
    for (int e = 0; e < 8; ++e) rope_grad_pair(klo[e], khi[e], cl[e], sl[e], ch[e], sh[e]);
  }
  uint16_t* dvrow = p.dv + b * p.dvs[0] + hk * p.dvs[1] + n * p.dvs[2];
  uint16_t* dkrow = p.dk + b * p.dks[0] + hk * p.dks[1] + n * p.dks[2];
  st16(dvrow + dl, pack8<E>(vlo));
  st16(dvrow + dh, pack8<E>(vhi));
  st16(dkrow + dl, pack8<E>(klo));
  st16(dkrow + dh, pack8<E>(khi));
}

// Masking of one score element (query i, key j); the range logic of each
// kernel decides which tiles are visited at all and which need this test.
template <int MASK>
__device__ __forceinline__ bool visible(int i, int j, int Nq, int Nkv, int W) {
  bool ok = i < Nq && j < Nkv;
  if constexpr (MASK == MASK_CAUSAL) ok = ok && j <= i;
  if constexpr (MASK == MASK_SW) ok = ok && abs(i - j) < W;
  if constexpr (MASK == MASK_CSW) ok = ok && j <= i && i - j < W;
  return ok;
}


// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------
// Head dims up to 64: three waves per SIMD (168 VGPRs), which the 4-wave
// workgroups meet by themselves and the 2-wave block-sparse ones miss by a
// register.
template <int D>
constexpr int bwd_dkv_waves_per_eu() {
  return D <= 64 ? 3 : 1;
}

// LDS of a dK/dV workgroup (16-bit elements): NS stages of the q~ tile, the
// dO tile and 32 (L log2 e, delta) pairs, and for D > 64 the V block.  The
// loads of stage t + NS - 1 are issued while stage t computes.  Head dims
// from 128 on keep two stages: with the V block a third would leave room for
// one 4-wave workgroup per CU (D = 128), or none (D = 256).
template <int D, int WAVES>
struct DkvLds {
  static constexpr int TILE = 32 * D;
  static constexpr int STAGE = 2 * TILE + 128;
  static constexpr int VBLK = D > 64 ? 32 * WAVES * D : 0;
  static constexpr int NS = D >= 128 ? 2 : 3;
  static constexpr int ELEMS = NS * STAGE + VBLK;
};

// One dK/dV workgroup, index wg of the dK/dV grid, with its LDS at lds.
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__device__ __forceinline__ void bwd_dkv_body(const BwdParams& p, uint16_t* lds, int wg) {
  constexpr int NT = WAVES * 64;
  constexpr int BK = 32 * WAVES;
  constexpr int KS = D / 16, DB = D / 32;
  constexpr bool VLDS = D > 64;            // V block in LDS instead of registers
  // transposed operands of the dV/dK MFMAs read this many MFMAs ahead (0:
  // read next to each MFMA); the 128-dim body has the registers to spare
  constexpr int kTrAhead = AF_DKV_TR_AHEAD(D);
  // k-steps of the S and dP MFMAs whose operands are read ahead
  constexpr int kSAhead = AF_DKV_S_AHEAD(D);
  constexpr int TILE = DkvLds<D, WAVES>::TILE;    // one 32-row tile (elements)
  constexpr int STAGE = DkvLds<D, WAVES>::STAGE;
  constexpr int NS = DkvLds<D, WAVES>::NS;

  // no keys: nothing to write (the launch still has one workgroup)
  if (p.n_kblocks <= 0) return;
  // the wave index is made provably uniform: it selects buffer resources and
  // LDS bases of the loads into LDS, which must be scalar
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // key block outermost: under a causal mask the first key blocks see the
  // most query tiles, so they are dispatched first.  Then the head-group
  // split, then (batch, key/value head).
  const int BHK = p.B * p.Hkv;
  // split key blocks first (g_split workgroups each), then unsplit ones
  const int heavy_wg = p.n_split_kb * BHK * p.g_split;
  int kbi, rem, gsplit = p.g_split;
  if (kIsBs<MASK> && p.g_split == 1 && p.bs_xcd_heads_kv > 0) {
    // every key-block row unsplit: grid n_split_kb x BHK
    xcd_head_groups(wg, BHK, p.n_split_kb, p.bs_xcd_heads_kv, kbi, rem);
  } else if (wg < heavy_wg) {
    kbi = wg / (BHK * p.g_split);
    rem = wg - kbi * (BHK * p.g_split);
  } else {
    kbi = p.n_split_kb + (wg - heavy_wg) / BHK;
    rem = (wg - heavy_wg) % BHK;
    gsplit = 1;
  }
  // block-sparse plan item: a piece [e0, e0 + ne) of column kb's list
  int kb = kbi, bs_e0 = 0, bs_ne = -1, bs_slot = -1;
  if constexpr (kIsBs<MASK>) {
    if (p.bs_kv_items != nullptr) {
      const int32_t* it = p.bs_kv_items + 4 * kbi;
      kb = it[0];
      bs_e0 = it[1];
      bs_slot = it[3];
      // a whole list (slot -1) is walked to its current count on the
      // device, so lists edited in place keep their plan valid
      bs_ne = bs_slot >= 0 ? it[2] : -1;
    }
  }
  const int split = rem / BHK;
  const int bhk = rem - split * BHK;
  const int hk = bhk % p.Hkv, b = bhk / p.Hkv;
  const int gper = p.G / gsplit;          // query heads of this workgroup
  const int hq0 = hk * p.G + split * gper;
  const int n0 = kb * BK;
  const int n0w = n0 + 32 * w;
  const int key = n0w + c;

  // k~ (and v) for this wave's 32 keys, as B operands (lane: row c).
  u32x4 kf[KS], vf[VLDS ? 1 : KS];
  load_operand_rows<D>(kf, p.kt + b * p.kts[0] + hk * p.kts[1], p.kts[2], key, p.Nkv, h);
  const uint16_t* vbase = p.v + b * p.vs[0] + hk * p.vs[1];
  uint16_t* const vblk = lds + NS * STAGE;
  if constexpr (VLDS) {
    const auto vrs = make_rsrc(vbase, span_bytes<D>(p.Nkv, p.vs[2]));
    // key row r is stored at block row kperm(r), so a wave's V operand reads
    // use the same per-lane offsets as its (permuted) query-row reads
    constexpr int VCH = BK * D / 8;
#pragma unroll
    for (int i = 0; i < VCH / NT; ++i) {
      const int g = tid + i * NT, row = g / (D / 8), kc = g % (D / 8);
      st16(vblk + lds_at<D>(kperm(row), 8 * kc), buf_ld16(vrs, (uint32_t)(((n0 + row) * p.vs[2] + 8 * kc) * 2)));
    }
  } else {
    load_operand_rows<D>(vf, vbase, p.vs[2], key, p.Nkv, h);
  }

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
  if constexpr (kIsBs<MASK>) {
    bs_sub = p.bs_block_m / 32;
    bs_n = p.bs_q_num[kb];
    bs_row = p.bs_q_idx + kb * p.bs_q_rs;
    // a piece of a split list stops at the list's current end
    ntq = (bs_ne >= 0 ? min(bs_ne, max(bs_n - bs_e0, 0)) : bs_n) * bs_sub;
  } else {
    ntq = m_hi > m_lo ? (m_hi - m_lo + 31) / 32 : 0;
  }
  BsTiles bst;
  if constexpr (kIsBs<MASK>)
    bst.init(bs_row, bs_n, bs_row, bs_e0, bs_sub, p.bs_block_m, 32, ntq, lane, p.bs_q_rs,
             MASK == MASK_BSE ? 2 : 0,
             p.bs_q_partial != nullptr ? p.bs_q_partial + kb * p.bs_q_rs : nullptr);
  auto tile_m0 = [&](int t) -> int {
    if constexpr (kIsBs<MASK>) {
      return bst(t);
    } else {
      return m_lo + 32 * t;
    }
  };
  const int ntiles = ntq * gper;

  TileDma<D, NT> dma;
  dma.init(w, lane, p.qts[2], p.dos[2]);
  // issue the loads of stage t into LDS slot `slot`: the q~ and dO tiles,
  // and (wave 0) the tile's 32 (L log2 e, delta) pairs; rows past N_q load
  // as zeros
  // stage t is query tile tl of head hq0 + gi, t = gi * ntq + tl; the loop
  // steps (gi, tl) along instead of dividing t by ntq twice per stage
  auto stage_load = [&](int gi, int tl, int slot) {
    const int hq = hq0 + gi;
    const int m0 = tile_m0(tl);
    dma.load(lds, slot * STAGE, w, p.qt + b * p.qts[0] + hq * p.qts[1], p.qts[2], p.Nq,
             p.dout + b * p.dos[0] + hq * p.dos[1], p.dos[2], p.Nq, m0);
    if (w == 0) {
      const int64_t row0 = ((int64_t)b * p.Hq + hq) * p.Nq + m0;
      const auto rs = make_rsrc(p.ld + 2 * row0, (uint32_t)max(p.Nq - m0, 0) * 8u);
      buf_ld4_lds(rs, lds + slot * STAGE + 2 * TILE, (uint32_t)lane * 4u);
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
  const int qr_row = kperm(c);   // tile row of this lane's (permuted) query

  // (head, query tile) of the stage computed (gi, tl) and of the next one to
  // load (gl, ll)
  auto adv = [&](int& g, int& l) {
    if (++l == ntq) {
      l = 0;
      ++g;
    }
  };
  int gi = 0, tl = 0, gl = 0, ll = 0;
  auto load_next = [&](int slot) {
    stage_load(gl, ll, slot);
    adv(gl, ll);
  };
  // a stage is IPW loads per wave, plus the (L, delta) pairs on wave 0;
  // waiting for all but the newest stage leaves that many in flight
  static_assert(decltype(dma)::INSTR % WAVES == 0, "equal loads per wave");
  constexpr int kStageLoads = decltype(dma)::IPW;
  auto wait_all_but_newest = [&]() {
    if (w == 0) wait_vmcnt<kStageLoads + 1>();
    else wait_vmcnt<kStageLoads>();
  };
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (i < ntiles) load_next(i);
  if (NS > 2 && ntiles > 1) wait_all_but_newest();
  else wait_lds_dma();
  lds_barrier();
  int slot = 0;
  for (int t = 0; t < ntiles; ++t) {
    // stage t + NS - 1 goes to the slot stage t - 1 used; the barrier
    // closing step t - 1 ended its reads
    const bool ahead = t + NS - 1 < ntiles;
    if (ahead) load_next(slot == 0 ? NS - 1 : slot - 1);
    const int hq = hq0 + gi;
    const int m0 = tile_m0(tl);
    // a partial block-sparse tile whose element mask applies: its K-major
    // entry and 32-row sub-tile
    bool epart = false;
    int ee = 0, esb = 0;
    if constexpr (MASK == MASK_BSE) {
      epart = bst.partial(tl);
      if (epart) {
        ee = bst.entry(tl);
        esb = bst.sub_of(tl);
      }
    }
    adv(gi, tl);
    const uint16_t* buf = lds + slot * STAGE;
    const uint16_t* Qs = buf;
    const uint16_t* Os = buf + TILE;
    const float* LD = reinterpret_cast<const float*>(buf + 2 * TILE);

    bool active = n0w < p.Nkv && m0 < p.Nq;
    if constexpr (MASK == MASK_CAUSAL) active = active && m0 + 31 >= n0w;
    if constexpr (MASK == MASK_SW) active = active && m0 + 31 > n0w - p.window && m0 < n0w + 31 + p.window;
    if constexpr (MASK == MASK_CSW) active = active && m0 + 31 >= n0w && m0 < n0w + 31 + p.window;
    if (active) {
      // S and dP (queries x keys), query rows permuted.
      f32x16 s = f32x16{}, dp = f32x16{};
      if constexpr (kSAhead > 0) {
        // the q~, dO (and V) operands of k-step ks read kSAhead k-steps
        // earlier
        u32x4 qop[KS], oop[KS], vop[KS];
        auto read_qo = [&](int ks) {
          const int off = lds_at<D>(qr_row, 16 * ks + 8 * h);
          qop[ks] = ld16(Qs + off);
          oop[ks] = ld16(Os + off);
          if constexpr (VLDS) vop[ks] = ld16(vblk + 32 * w * D + off);
          else vop[ks] = vf[ks];
        };
#pragma unroll
        for (int ks = 0; ks < kSAhead; ++ks) read_qo(ks);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = E::mfma32(qop[ks], kf[ks], s);
          dp = E::mfma32(oop[ks], vop[ks], dp);
          if (ks + kSAhead < KS) read_qo(ks + kSAhead);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = lds_at<D>(qr_row, 16 * ks + 8 * h);
          s = E::mfma32(ld16(Qs + off), kf[ks], s);
          u32x4 vb;
          if constexpr (VLDS) vb = ld16(vblk + 32 * w * D + off);
          else vb = vf[ks];
          dp = E::mfma32(ld16(Os + off), vb, dp);
        }
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
      // logits in log2 units (register r holds query m0 + 16 (r/8) + 8h +
      // r%8); without a bias the raw scores go through the mask (-inf stays
      // -inf under the positive scale) and the exponent below takes s c2 - L
      // in one fma
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (BIAS == BIAS_ALIBI) {
          // causal-type masks see only j <= i, where -slope |i - j| is
          // linear in the query index (one add per element)
          float abias = 0.f;
          if constexpr (kAlibiOneSided) abias = slope2 * (float)(key - (m0 + 16 * j + 8 * h));
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int r = 8 * j + e;
            float x = s[r] * c2;
            if constexpr (kAlibiOneSided) {
              x += abias;
              abias -= slope2;
            } else {
              x -= slope2 * (float)abs(m0 + 16 * j + 8 * h + e - key);
            }
            s[r] = x;
          }
        }
      }
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = m0 + 16 * (r >> 3) + 8 * h + (r & 7);
          s[r] = visible<MASK>(qi, key, p.Nq, p.Nkv, p.window) ? s[r] : -INFINITY;
        }
      }
      if constexpr (MASK == MASK_BSE) {
        if (epart) {
          // bits of this lane's key over the tile's 32 query rows, shifted
          // by 8 h once so that every element tests a constant bit
          const int wc = (p.bs_block_m + 63) / 64;
          const int64_t word = (((int64_t)kb * p.bs_q_rs + ee) * p.bs_block_n + (key - n0)) * wc + (esb >> 1);
          const uint32_t bits = key < p.Nkv ? (uint32_t)(p.bs_col_bits[word] >> (32 * (esb & 1))) >> (8 * h) : 0u;
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = (bits & (1u << (16 * (r >> 3) + (r & 7)))) ? s[r] : -INFINITY;
        }
      }
      u32x4 pp[2], pd[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // (L log2 e, delta) pairs of tile rows 16 j + 8 h .. + 7
        f32x4 ld4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ld4[i] = *reinterpret_cast<const f32x4*>(LD + 2 * (16 * j + 8 * h) + 4 * i);
        float pv[8], dsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          const float L2 = ld4[e >> 1][2 * (e & 1)];
          const float dl = ld4[e >> 1][2 * (e & 1) + 1];
          const float x = BIAS == BIAS_ALIBI ? s[r] - L2 : __builtin_fmaf(s[r], c2, -L2);
          const float pr = __builtin_amdgcn_exp2f(x);
          pv[e] = pr;
          dsv[e] = pr * (dp[r] - dl);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pp[j][i] = E::pack(pv[2 * i], pv[2 * i + 1]);
          pd[j][i] = E::pack(dsv[2 * i], dsv[2 * i + 1]);
        }
      }
      // dV^T += dO^T P,  dK~^T += Q~^T dS   (contraction over 32 queries;
      // the transposed operands come from transposing LDS reads)
      if constexpr (kTrAhead > 0) {
        // MFMA i = (db, j, dV or dK) with its operand read kTrAhead MFMAs
        // earlier; the scheduling barriers keep the compiler from sinking
        // each read back next to its MFMA, which then waited out a whole
        // LDS round trip (16 serialised read -> wait -> MFMA triples)
        constexpr int NOPS = DB * 4;
        auto read_op = [&](int i) -> u32x4 {
          const int db = i >> 2, j = (i >> 1) & 1;
          const uint16_t* base = ((i & 1) ? Qs : Os) + 16 * j * D;
          const u32x2 lo = lds_read_tr16(base + tr_at<D>(lane, 0, db));
          const u32x2 hi = lds_read_tr16(base + tr_at<D>(lane, 1, db));
          return u32x4{lo[0], lo[1], hi[0], hi[1]};
        };
        u32x4 op[NOPS];
#pragma unroll
        for (int i = 0; i < kTrAhead; ++i) op[i] = read_op(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NOPS; ++i) {
          const int db = i >> 2, j = (i >> 1) & 1;
          if (i & 1) dk[db] = E::mfma32(op[i], pd[j], dk[db]);
          else dv[db] = E::mfma32(op[i], pp[j], dv[db]);
          if (i + kTrAhead < NOPS) op[i + kTrAhead] = read_op(i + kTrAhead);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int t0 = tr_at<D>(lane, 0, db), t1 = tr_at<D>(lane, 1, db);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const u32x2 olo = lds_read_tr16(Os + 16 * j * D + t0);
            const u32x2 ohi = lds_read_tr16(Os + 16 * j * D + t1);
            dv[db] = E::mfma32(u32x4{olo[0], olo[1], ohi[0], ohi[1]}, pp[j], dv[db]);
            const u32x2 qlo = lds_read_tr16(Qs + 16 * j * D + t0);
            const u32x2 qhi = lds_read_tr16(Qs + 16 * j * D + t1);
            dk[db] = E::mfma32(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, pd[j], dk[db]);
          }
        }
      }
    }
    // stage t + 1 has landed in every wave (stage t + 2 may be in flight)
    if (NS > 2 && ahead) wait_all_but_newest();
    else wait_lds_dma();
    lds_barrier();
    slot = slot + 1 == NS ? 0 : slot + 1;
  }

  uint16_t* dkb = p.dk + b * p.dks[0] + hk * p.dks[1];
  uint16_t* dvb = p.dv + b * p.dvs[0] + hk * p.dvs[1];
  if (kIsBs<MASK> && bs_slot >= 0) {
    // a piece of a split column
    if (key < p.Nkv) {
      const int64_t row = ((int64_t)bs_slot * BHK + bhk) * BK + (key - n0);
      store_partial_row<D>(dv, p.part_dv + row * D, h);
      store_partial_row<D>(dk, p.part_dk + row * D, h);
    }
    return;
  }
  if (gsplit > 1) {
    if (key < p.Nkv) {
      const int64_t row = (((int64_t)split * p.B + b) * p.Hkv + hk) * p.Nkv + key;
      store_partial_row<D>(dv, p.dvp + row * D, h);
      store_partial_row<D>(dk, p.dkp + row * D, h);
    }
    return;
  }
  store_grad_rows<E, D, false>(dv, dvb, p.dvs[2], key, p.Nkv, 1.f, nullptr, nullptr, 0, h);
  store_grad_rows<E, D, ROPE>(dk, dkb, p.dks[2], key, p.Nkv, p.scale, p.cos, p.sin, p.rs[0], h);
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
// LDS of a dQ workgroup (16-bit elements): three stages of the k~ and v
// tiles; the loads of stage t + 2 are issued while stage t computes.
template <int D>
struct DqLds {
  static constexpr int TILE = 32 * D;
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NS = 3;
  static constexpr int ELEMS = NS * STAGE;
};

// One dQ workgroup, index wg of the dQ grid, with its LDS at lds.
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__device__ __forceinline__ void bwd_dq_body(const BwdParams& p, uint16_t* lds, int wg) {
  constexpr int NT = WAVES * 64;
  constexpr int BMq = 32 * WAVES;
  constexpr int KS = D / 16, DB = D / 32;
  constexpr int TILE = DqLds<D>::TILE;
  constexpr int STAGE = DqLds<D>::STAGE;
  constexpr int NS = DqLds<D>::NS;
  // transposed K~ operands of the dQ MFMAs read this many MFMAs ahead (0:
  // next to each MFMA)
  constexpr int kTrAhead = AF_DQ_TR_AHEAD(D);
  // k-steps of the score MFMAs whose K~ / V operands are read ahead
  constexpr int kSAhead = AF_DQ_S_AHEAD(D);

  // no queries: nothing to write (the launch still has one workgroup)
  if (p.n_qblocks <= 0) return;
  // the wave index is made provably uniform: it selects buffer resources and
  // LDS bases of the loads into LDS, which must be scalar
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BH = p.B * p.Hq;
  int bh = wg % BH;
  int mbi = wg / BH;
  if constexpr (kIsBs<MASK>) xcd_head_groups(wg, BH, p.bs_q_rows, p.bs_xcd_heads_q, mbi, bh);
  const bool heavy_last = MASK == MASK_CAUSAL || MASK == MASK_CSW;
  // block-sparse plan item: a piece [e0, e0 + ne) of row mb's list
  int mb = heavy_last ? (p.n_qblocks - 1 - mbi) : mbi;
  int bs_e0 = 0, bs_ne = -1, bs_slot = -1;
  if constexpr (kIsBs<MASK>) {
    if (p.bs_q_items != nullptr) {
      const int32_t* it = p.bs_q_items + 4 * mbi;
      mb = it[0];
      bs_e0 = it[1];
      bs_slot = it[3];
      bs_ne = bs_slot >= 0 ? it[2] : -1;
    }
  }
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.G;
  const int m0 = mb * BMq, q0w = m0 + 32 * w, qrow = q0w + c;

  u32x4 qf[KS], of[KS];
  load_operand_rows<D>(qf, p.qt + b * p.qts[0] + hq * p.qts[1], p.qts[2], qrow, p.Nq, h);
  load_operand_rows<D>(of, p.dout + b * p.dos[0] + hq * p.dos[1], p.dos[2], qrow, p.Nq, h);
  float L2 = 0.f, dl = 0.f;
  if (qrow < p.Nq) {
    const f32x2 ld = *reinterpret_cast<const f32x2*>(p.ld + 2 * (((int64_t)b * p.Hq + hq) * p.Nq + qrow));
    L2 = ld[0];
    dl = ld[1];
  }

  int n_lo = 0, n_hi = p.Nkv, ntiles;
  int bs_nfull = 0, bs_npart = 0, bs_sub = 1;
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
  if constexpr (kIsBs<MASK>) {
    bs_sub = p.bs_block_n / 32;
    bs_nfull = p.bs_full_num[mb];
    bs_npart = p.bs_part_num[mb];
    bs_full_row = p.bs_full_idx + mb * p.bs_full_rs;
    bs_part_row = p.bs_part_idx + mb * p.bs_part_rs;
    ntiles = (bs_ne >= 0 ? min(bs_ne, max(bs_nfull + bs_npart - bs_e0, 0)) : bs_nfull + bs_npart) * bs_sub;
  } else {
    ntiles = n_hi > n_lo ? (n_hi - n_lo + 31) / 32 : 0;
  }
  BsTiles bst;
  if constexpr (kIsBs<MASK>)
    bst.init(bs_full_row, bs_nfull, bs_part_row, bs_e0, bs_sub, p.bs_block_n, 32, ntiles, lane, p.bs_full_rs,
             MASK == MASK_BSE ? 1 : 0);
  auto tile_n0 = [&](int t) -> int {
    if constexpr (kIsBs<MASK>) {
      return bst(t);
    } else {
      return n_lo + 32 * t;
    }
  };

  TileDma<D, NT> dma;
  dma.init(w, lane, p.kts[2], p.vs[2]);
  const uint16_t* kbase = p.kt + b * p.kts[0] + hk * p.kts[1];
  const uint16_t* vbase = p.v + b * p.vs[0] + hk * p.vs[1];
  auto stage_load = [&](int t, int slot) {
    dma.load(lds, slot * STAGE, w, kbase, p.kts[2], p.Nkv, vbase, p.vs[2], p.Nkv, tile_n0(t));
  };

  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = f32x16{};
  const float c2 = p.scale * kLog2e;
  float slope2 = 0.f;
  if constexpr (BIAS == BIAS_ALIBI) slope2 = p.slopes[hq] * kLog2e;
  constexpr bool kAlibiOneSided = BIAS == BIAS_ALIBI && (MASK == MASK_CAUSAL || MASK == MASK_CSW);
  const int kr_row = kperm(c);   // tile row of this lane's (permuted) key

  static_assert(decltype(dma)::INSTR % WAVES == 0, "equal loads per wave");
  constexpr int kStageLoads = decltype(dma)::IPW;
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (i < ntiles) stage_load(i, i);
  if (ntiles > 1) wait_vmcnt<kStageLoads>();
  else wait_lds_dma();
  lds_barrier();
  int slot = 0;
  for (int t = 0; t < ntiles; ++t) {
    // stage t + 2 goes to the slot stage t - 1 used; the barrier closing
    // step t - 1 ended its reads
    const bool ahead = t + NS - 1 < ntiles;
    if (ahead) stage_load(t + NS - 1, slot == 0 ? NS - 1 : slot - 1);
    const int n0 = tile_n0(t);
    const uint16_t* Ks = lds + slot * STAGE;
    const uint16_t* Vs = Ks + TILE;

    bool active = q0w < p.Nq && n0 >= 0 && n0 < p.Nkv;
    if constexpr (MASK == MASK_CAUSAL) active = active && n0 <= q0w + 31;
    if constexpr (MASK == MASK_SW) active = active && n0 + 31 > q0w - p.window && n0 < q0w + 31 + p.window;
    if constexpr (MASK == MASK_CSW) active = active && n0 + 31 > q0w - p.window && n0 <= q0w + 31;
    if (active) {
      f32x16 s = f32x16{}, dp = f32x16{};
      if constexpr (kSAhead > 0) {
        // the K~ and V operands of k-step ks read kSAhead k-steps earlier
        u32x4 kop[KS], vop[KS];
        auto read_kv = [&](int ks) {
          const int off = lds_at<D>(kr_row, 16 * ks + 8 * h);
          kop[ks] = ld16(Ks + off);
          vop[ks] = ld16(Vs + off);
        };
#pragma unroll
        for (int ks = 0; ks < kSAhead; ++ks) read_kv(ks);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = E::mfma32(kop[ks], qf[ks], s);
          dp = E::mfma32(vop[ks], of[ks], dp);
          if (ks + kSAhead < KS) read_kv(ks + kSAhead);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = lds_at<D>(kr_row, 16 * ks + 8 * h);
          s = E::mfma32(ld16(Ks + off), qf[ks], s);
          dp = E::mfma32(ld16(Vs + off), of[ks], dp);
        }
      }
      bool need_mask = q0w + 32 > p.Nq || n0 + 32 > p.Nkv;
      if constexpr (MASK == MASK_CAUSAL) need_mask = need_mask || n0 + 31 > q0w;
      if constexpr (MASK == MASK_SW)
        need_mask = need_mask || q0w + 31 - n0 >= p.window || n0 + 31 - q0w >= p.window;
      if constexpr (MASK == MASK_CSW) need_mask = need_mask || n0 + 31 > q0w || q0w + 31 - n0 >= p.window;
      // logits minus L in log2 units (one fma per element without a bias):
      // register r holds key n0 + 16 (r/8) + 8h + r%8
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float abias = 0.f;
        if constexpr (kAlibiOneSided) abias = slope2 * (float)(n0 + 16 * j + 8 * h - qrow) - L2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          float x;
          if constexpr (kAlibiOneSided) {
            x = __builtin_fmaf(s[r], c2, abias);
            abias += slope2;
          } else if constexpr (BIAS == BIAS_ALIBI) {
            x = __builtin_fmaf(s[r], c2, -L2) - slope2 * (float)abs(qrow - (n0 + 16 * j + 8 * h + e));
          } else {
            x = __builtin_fmaf(s[r], c2, -L2);
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
      if constexpr (MASK == MASK_BSE) {
        if (bst.partial(t)) {
          // element mask of a partial tile: bits of this lane's query row
          // over the tile's 32 keys, shifted by 8 h once so that every
          // element tests a constant bit
          const int e = bst.entry(t), sb = bst.sub_of(t);
          const int64_t word = (((int64_t)mb * p.bs_part_rs + (e - bs_nfull)) * p.bs_block_m + (qrow - m0)) *
                                   (p.bs_block_n / 64) + (sb >> 1);
          const uint32_t bits = qrow < p.Nq ? (uint32_t)(p.bs_row_bits[word] >> (32 * (sb & 1))) >> (8 * h) : 0u;
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = (bits & (1u << (16 * (r >> 3) + (r & 7)))) ? s[r] : -INFINITY;
        }
      }
      u32x4 pd[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float dsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * j + e;
          const float pr = __builtin_amdgcn_exp2f(s[r]);
          dsv[e] = pr * (dp[r] - dl);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) pd[j][i] = E::pack(dsv[2 * i], dsv[2 * i + 1]);
      }
      // dQ~^T += K~^T dS^T (contraction over 32 keys, K~^T by transposing
      // reads), each MFMA's operand read kTrAhead MFMAs earlier as in the
      // dK/dV body
      if constexpr (kTrAhead > 0) {
        constexpr int NOPS = DB * 2;
        auto read_op = [&](int i) -> u32x4 {
          const int db = i >> 1, j = i & 1;
          const u32x2 lo = lds_read_tr16(Ks + 16 * j * D + tr_at<D>(lane, 0, db));
          const u32x2 hi = lds_read_tr16(Ks + 16 * j * D + tr_at<D>(lane, 1, db));
          return u32x4{lo[0], lo[1], hi[0], hi[1]};
        };
        u32x4 op[NOPS];
#pragma unroll
        for (int i = 0; i < kTrAhead; ++i) op[i] = read_op(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NOPS; ++i) {
          dq[i >> 1] = E::mfma32(op[i], pd[i & 1], dq[i >> 1]);
          if (i + kTrAhead < NOPS) op[i + kTrAhead] = read_op(i + kTrAhead);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int t0 = tr_at<D>(lane, 0, db), t1 = tr_at<D>(lane, 1, db);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const u32x2 klo = lds_read_tr16(Ks + 16 * j * D + t0);
            const u32x2 khi = lds_read_tr16(Ks + 16 * j * D + t1);
            dq[db] = E::mfma32(u32x4{klo[0], klo[1], khi[0], khi[1]}, pd[j], dq[db]);
          }
        }
      }
    }
    // stage t + 1 has landed in every wave (stage t + 2 may be in flight)
    if (ahead) wait_vmcnt<kStageLoads>();
    else wait_lds_dma();
    lds_barrier();
    slot = slot + 1 == NS ? 0 : slot + 1;
  }

  if (kIsBs<MASK> && bs_slot >= 0) {
    // a piece of a split row
    if (qrow < p.Nq) store_partial_row<D>(dq, p.part_dq + (((int64_t)bs_slot * BH + bh) * BMq + (qrow - m0)) * D, h);
    return;
  }
  store_grad_rows<E, D, ROPE>(dq, p.dq + b * p.dqs[0] + hq * p.dqs[1], p.dqs[2], qrow, p.Nq, p.scale, p.cos,
                              p.sin, p.rs[0], h);
}

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(bwd_dkv_waves_per_eu<D>())))
    bwd_dkv_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[DkvLds<D, WAVES>::ELEMS];
  bwd_dkv_body<E, D, MASK, BIAS, ROPE, WAVES>(p, lds, blockIdx.x);
}

template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) bwd_dq_kernel(const BwdParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[DqLds<D>::ELEMS];
  bwd_dq_body<E, D, MASK, BIAS, ROPE, WAVES>(p, lds, blockIdx.x);
}

// dK/dV and dQ in one launch: workgroups [0, n_dkv_wg) are the dK/dV grid,
// the rest the dQ grid.  Both read only the prep kernel's output, and the
// dispatcher starts workgroups in index order, so dQ workgroups take the
// slots that short dK/dV workgroups free (under a causal mask the first key
// blocks walk every query tile and the last almost none).
template <class E, int D, int MASK, int BIAS, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(bwd_dkv_waves_per_eu<D>())))
    bwd_dkvdq_kernel(const BwdParams p) {
  constexpr int EK = DkvLds<D, WAVES>::ELEMS, EQ = DqLds<D>::ELEMS;
  __shared__ __attribute__((aligned(16))) uint16_t lds[EK > EQ ? EK : EQ];
  if ((int)blockIdx.x < p.n_dkv_wg)
    bwd_dkv_body<E, D, MASK, BIAS, ROPE, WAVES>(p, lds, blockIdx.x);
  else
    bwd_dq_body<E, D, MASK, BIAS, ROPE, WAVES>(p, lds, (int)blockIdx.x - p.n_dkv_wg);
}

}  // namespace af
