// Fused attention forward for gfx950 (piece (a) + the block-sparse walk of
// piece (d)).
//
// Semantics follow the reference forward kernel
// (reference: attnfuse/compiler/codegen.py:67-381): S = (rope(q) . rope(k)) *
// scale, plus ALiBi -slope*|i-j| or an additive bias tile, causal / sliding
// window / bounds masks, online softmax in fp32 (or ReLU normalised by its
// row sum), P rounded to the input dtype before P*V, O = acc / l with l == 0
// treated as 1, optional L = m + ln(l).
//
// Work decomposition (MI355X-first, not a translation):
//  * a workgroup owns BM = 32*WAVES query rows of one (batch, head); each
//    wave64 owns 32 rows: one 32x32 MFMA output block.
//  * K and V stream through LDS in 64-key stages, two slots each, loaded
//    global -> LDS by buffer_load ... lds while earlier stages are on the
//    MFMA pipes.  The loads go through raw buffer resources, so rows past
//    N_kv come back as zeros from the hardware bounds check (no clamps, no
//    branches).  With RoPE, K arrives already rotated (rope_rows_kernel
//    writes k~ once per call); V is written row-major and read back
//    transposed by ds_read_b64_tr_b16.
//  * scores are computed transposed (S^T = K Q^T): each lane then holds 32
//    keys of one query, so the row max is in-register plus one
//    v_permlane32_swap, and P^T is the B operand of the P*V MFMA without any
//    register shuffle (see af_common.hpp).  Row sums add the rounded P on
//    the VALU in fp32.
//  * the softmax max is lazy: the running max only moves when a score
//    exceeds it by more than 2^kTau, so the O rescale is rare.
//  * Q stays in registers for the whole kernel, rotated once.
//  * causal grids run the longest query blocks first.
//  * kernels with no bias or ALiBi at head dims up to 64 (block masks
//    aside) run each tile's scores, P and P V in one unpipelined step
//    (fwd_unpipelined), and the registers that saves buy a fourth (ALiBi:
//    third) wave per SIMD;
//    other kernels compute the scores of tile t+1 while P of tile t is on
//    the VALU.  Block-sparse kernels defer P V by one step (fwd_defer): the
//    score MFMAs of tile t+1 and the P V MFMAs of tile t-1 alternate, one
//    per chunk, with the softmax VALU work of tile t in one basic block.
#pragma once

#include "af_common.hpp"

namespace af {

// MASK_BSE (no af_mask value of its own): a block-sparse walk whose partial
// tiles carry element masks (af_blockmask.part_row_bits ...); its kernels
// are instantiated apart, so that plain block-sparse walks keep no state for
// them.  Head dims up to 128.
enum { MASK_FULL = 0, MASK_CAUSAL = 1, MASK_SW = 2, MASK_BS = 3, MASK_CSW = 4, MASK_BSE = 5 };
template <int MASK>
inline constexpr bool kIsBs = MASK == MASK_BS || MASK == MASK_BSE;
enum { BIAS_NONE = 0, BIAS_ALIBI = 1, BIAS_ADD = 2 };
enum { NORM_SOFTMAX = 0, NORM_RELU = 1 };

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  const uint16_t* cos;
  const uint16_t* sin;
  const float* slopes;
  const uint16_t* bias;
  uint32_t* coverage;
  const int32_t* bs_full_num;
  const int32_t* bs_full_idx;
  const int32_t* bs_part_num;
  const int32_t* bs_part_idx;
  // Block-sparse work plan (nullable): item i of (row block, first entry,
  // entries, slot) is grid row i; slot >= 0 writes the piece's unnormalised
  // O to part_o and its (running max, row sum) to part_ml, both indexed
  // (slot, B*Hq, BLOCK_M), for the combine kernel.
  const int32_t* bs_items;
  // Element masks of the partial tiles (nullable): (n_q_blocks,
  // bs_part_rs, BLOCK_M, BLOCK_N / 64) words, bit k of word w of row r set
  // when query r of the block sees key 64 w + k of the entry's key block.
  const uint64_t* bs_row_bits;
  float* part_o;
  float* part_ml;
  int64_t qs[4], ks[4], vs[4], os[4], ls[3], rs[2], bs[4];
  int64_t bs_full_rs, bs_part_rs;
  int32_t B, Hq, Hkv, Nq, Nkv, G;
  int32_t n_mblocks, bs_block_m, bs_block_n;
  // block-sparse walks: heads per XCD group (xcd_head_groups), 0 = off
  int32_t bs_xcd_heads;
  int32_t cov_nq, cov_nk;
  int32_t rope_len;
  float scale;
  int32_t window;
};

// Whether a forward instantiation runs the unpipelined step (see the
// kernel): softmax or ReLU with no bias or ALiBi over a dense, causal or
// windowed walk at head dims up to 64.  It holds one score tile instead of
// two, so the kernels without a bias hold 110-115 VGPRs and run four waves
// per SIMD, the ALiBi kernels (whose initial score accumulator takes 16
// more) 123-168 and three or four.  Same-box A/B against the pipelined
// steps: config 2 1.5-2 %, the dense and windowed forwards 3.5-6 % faster
// (three waves before, outputs bit-identical); config 2 with ALiBi 7 %,
// dense ALiBi 10 % and windowed ALiBi 3 % faster (the first two against the
// deferred P V pipeline at two waves); causal ReLU 7-10 % and causal ReLU
// with ALiBi 8-11 % faster (bit-identical).  At head dim 128 the step saved
// too few registers for a third wave (186 VGPRs) and was 1-2 % slower; with
// an additive bias it spilled 384-776 bytes; on block-sparse walks (31 KB
// of LDS per 2-wave workgroup caps them at five per CU) it was neutral.
template <int D, int MASK, int BIAS, int NORM>
constexpr bool fwd_unpipelined() {
  return D <= 64 && (BIAS == BIAS_NONE || BIAS == BIAS_ALIBI) &&
         (MASK == MASK_FULL || MASK == MASK_CAUSAL || MASK == MASK_SW || MASK == MASK_CSW);
}

// Whether a forward instantiation runs the deferred P V pipeline (see the
// kernel): the block-sparse softmax walks without ALiBi at head dims up to
// 64 (two waves per SIMD; the BigBird forward 2-3 % faster than the
// pipelined step).
#ifndef AF_FWD_DEFER
#define AF_FWD_DEFER 1
#endif
template <int D, int MASK, int BIAS, int NORM>
constexpr bool fwd_defer() {
  if (!AF_FWD_DEFER || D > 64 || NORM != NORM_SOFTMAX) return false;
  return (MASK == MASK_BS || MASK == MASK_BSE) && BIAS != BIAS_ALIBI;
}

// Waves per SIMD the register budget is set for: the unpipelined step four
// without a bias or with windowed ALiBi (123-125 VGPRs; scheduled for three,
// the same registers ran 5 % slower), three with the other ALiBi kinds (a
// causal-type kind rebuilding its initial accumulator from 16 multiplies per
// tile to free the registers for a fourth wave ran 3.5 % slower).  The other
// kernels with head dims up to 64 fit 168 VGPRs (three waves), except the
// deferred pipeline, which keeps two score tiles and two P tiles live, and
// additive biases (two waves); D = 128 takes one.
template <int D, int MASK, int BIAS, int NORM>
constexpr int fwd_waves_per_eu() {
  if (fwd_unpipelined<D, MASK, BIAS, NORM>()) return (BIAS == BIAS_NONE || MASK == MASK_SW) ? 4 : 3;
  if (D > 64) return 1;
  if (fwd_defer<D, MASK, BIAS, NORM>()) return 2;
  // an additive bias tile takes 8 loaded values per score block: at three
  // waves these kernels spilled 18-36 registers, with ReLU about 300
  if (BIAS == BIAS_ADD) return 2;
  return 3;
}

// Head dims up to 64 run three or four waves per SIMD (three or four 4-wave
// workgroups per CU, 32 KB of LDS each).
template <class E, int D, int MASK, int BIAS, int NORM, bool ROPE, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(fwd_waves_per_eu<D, MASK, BIAS, NORM>())))
    fwd_kernel(const FwdParams p) {
  constexpr int NT = WAVES * 64;
  constexpr int BM = 32 * WAVES;
  constexpr int BN = 64;
  constexpr int KS = D / 16;         // 16-deep k-steps of Q K^T
  constexpr int DB = D / 32;         // 32-row blocks of O^T
  constexpr int TILE = BN * D;       // one swizzled (BN x D) tile, no padding

  // two K slots, then two V slots
  constexpr bool kDefer = fwd_defer<D, MASK, BIAS, NORM>();
  constexpr int kSlots = 2;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kSlots * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // provably wave-uniform: it selects the LDS bases of the loads into LDS
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int c = lane & 31;

  const int BH = p.B * p.Hq;
  // m-block-major order: the heaviest query blocks of every head first.
  // Workgroup g runs on XCD g % 8, so when B*H is a multiple of 8 each XCD
  // works on a fixed eighth of the heads, whose K/V stay in its L2.
  int bh = blockIdx.x % BH;
  int mbi = blockIdx.x / BH;
  if constexpr (kIsBs<MASK>) xcd_head_groups(blockIdx.x, BH, p.n_mblocks, p.bs_xcd_heads, mbi, bh);
  const bool heavy_last = MASK == MASK_CAUSAL || MASK == MASK_CSW;
  // block-sparse plan item: a piece [e0, e0 + ne) of row mb's list
  int mb = heavy_last ? (p.n_mblocks - 1 - mbi) : mbi;
  int bs_e0 = 0, bs_ne = -1, bs_slot = -1;
  if constexpr (kIsBs<MASK>) {
    if (p.bs_items != nullptr) {
      const int32_t* it = p.bs_items + 4 * mbi;
      mb = it[0];
      bs_e0 = it[1];
      bs_slot = it[3];
      // a whole list (slot -1) is walked to its current count on the
      // device, so lists edited in place keep their plan valid
      bs_ne = bs_slot >= 0 ? it[2] : -1;
    }
  }
  const int b = bh / p.Hq;
  const int hq = bh - b * p.Hq;
  const int hk = hq / p.G;
  const int m0 = mb * BM;
  const int q0w = m0 + 32 * w;
  const int qrow = q0w + c;

  const uint16_t* __restrict__ qbase = p.q + b * p.qs[0] + hq * p.qs[1];
  const uint16_t* kbase = p.k + b * p.ks[0] + hk * p.ks[1];
  const uint16_t* vbase = p.v + b * p.vs[0] + hk * p.vs[1];
  const int64_t kstr = p.ks[2], vstr = p.vs[2];
  const int64_t rstr = p.rs[0];

  const float c2 = p.scale * kLog2e;

  // ---- Q fragment (B operand of S^T = K Q^T), rotated once -------------
  // The rotated q~ is rounded to 16 bits unscaled, as the reference kernel
  // rounds it (attnfuse/compiler/codegen.py:126-135); the softmax scale is
  // applied to the fp32 scores.
  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = (qrow < p.Nq) ? ld16(qbase + qrow * p.qs[2] + 16 * ks + 8 * h)
                           : u32x4{0, 0, 0, 0};
  }
  if constexpr (ROPE) {
    if (qrow < p.Nq) {
      const uint16_t* cr = p.cos + qrow * rstr;
      const uint16_t* sr = p.sin + qrow * rstr;
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks) {
        const int dl = 16 * ks + 8 * h, dh = dl + D / 2;
        rope_pair<E>(qf[ks], qf[ks + KS / 2], ld16(cr + dl), ld16(sr + dl),
                     ld16(cr + dh), ld16(sr + dh));
      }
    }
  }

  // ---- key-tile schedule ------------------------------------------------
  int n_lo = 0, n_hi = p.Nkv, ntiles;
  int bs_nfull = 0, bs_npart = 0, bs_sub = 1;
  const int32_t* bs_full_row = nullptr;
  const int32_t* bs_part_row = nullptr;
  if constexpr (MASK == MASK_CAUSAL) {
    n_hi = min(m0 + BM, p.Nkv);
  } else if constexpr (MASK == MASK_SW) {
    n_lo = max(m0 - p.window + 1, 0) & ~(BN - 1);
    n_hi = min(m0 + BM - 1 + p.window, p.Nkv);
  } else if constexpr (MASK == MASK_CSW) {
    n_lo = max(m0 - p.window + 1, 0) & ~(BN - 1);
    n_hi = min(m0 + BM, p.Nkv);
  }
  if constexpr (kIsBs<MASK>) {
    bs_sub = p.bs_block_n / BN;
    bs_nfull = p.bs_full_num[mb];
    bs_npart = p.bs_part_num[mb];
    bs_full_row = p.bs_full_idx + mb * p.bs_full_rs;
    bs_part_row = p.bs_part_idx + mb * p.bs_part_rs;
    // a piece of a split list stops at the list's current end
    ntiles = (bs_ne >= 0 ? min(bs_ne, max(bs_nfull + bs_npart - bs_e0, 0)) : bs_nfull + bs_npart) * bs_sub;
  } else {
    ntiles = n_hi > n_lo ? (n_hi - n_lo + BN - 1) / BN : 0;
  }
  BsTiles bst;
  if constexpr (kIsBs<MASK>)
    bst.init(bs_full_row, bs_nfull, bs_part_row, bs_e0, bs_sub, p.bs_block_n, BN, ntiles, lane, p.bs_full_rs,
             MASK == MASK_BSE ? 1 : 0);
  // Causal-type ALiBi walks the key tiles from the diagonal down: its bias
  // -slope (i - j) then only falls from tile to tile, so the running max set
  // by the first (diagonal) tile holds and the later tiles take the lazy
  // softmax step.  Walked upwards the max rose by slope * 64 per tile and
  // every step had to compute it.
  constexpr bool kDescend =
      BIAS == BIAS_ALIBI && NORM == NORM_SOFTMAX && (MASK == MASK_CAUSAL || MASK == MASK_CSW);
  // Dense two-sided ALiBi (-slope |i - j|) walks outwards from the tile of
  // the block's first query, alternating right and left, so the bias falls
  // on both sides of it in the same way.  (Windowed, the same walk with two
  // waves per SIMD measured 3 % slower than exact steps at three, 0.177 vs
  // 0.171 ms at config 2's shape, window 1024; dense 0.412 -> 0.383 ms.)
  constexpr bool kOutward = BIAS == BIAS_ALIBI && NORM == NORM_SOFTMAX && MASK == MASK_FULL;
  const int kc = kOutward ? min(max((m0 - n_lo) / BN, 0), max(ntiles - 1, 0)) : 0;
  const int kside = kOutward ? min(kc, ntiles - 1 - kc) : 0;
  auto tile_n0 = [&](int t) -> int {
    if constexpr (kIsBs<MASK>) {
      return bst(t);
    } else if constexpr (kDescend) {
      return n_lo + (ntiles - 1 - t) * BN;
    } else if constexpr (kOutward) {
      int k;
      if (t <= 2 * kside) k = (t & 1) ? kc + ((t + 1) >> 1) : kc - (t >> 1);
      else k = (ntiles - 1 - kc > kc) ? kc + (t - kside) : kc - (t - kside);
      return n_lo + k * BN;
    } else {
      return n_lo + t * BN;
    }
  };

  // ---- K / V staging: buffer loads straight into swizzled LDS tiles ----------
  // Rows past N_kv fall outside the buffer resources and load as zeros (their
  // scores are masked anyway).  With RoPE the K given here is already
  // rotated (k~, written once per key by rope_rows_kernel).  Two K slots and
  // two V slots: K runs one tile ahead of V (see the pipeline below).
  RowsDma<D, NT, BN> kdma, vdma;
  kdma.init(w, lane, kstr);
  vdma.init(w, lane, vstr);
  // slot parity t & 1 is passed as a literal by the unrolled pipeline so
  // that every LDS address is a register plus an immediate offset
  auto load_k = [&](int t, int par) { kdma.load(lds, par * TILE, w, kbase, kstr, p.Nkv, tile_n0(t)); };
  auto load_v = [&](int t, int par) { vdma.load(lds, (kSlots + par) * TILE, w, vbase, vstr, p.Nkv, tile_n0(t)); };
  // per-lane LDS offsets: the K rows of the S^T MFMA (key block 0; block 1 is
  // 32 rows on, same swizzle) and the transposed V reads of the P V MFMA
  int koff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = lds_at<D>(kperm(c), 16 * ks + 8 * h);
  int voff[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    voff[db][0] = tr_at<D>(lane, 0, db);
    voff[db][1] = tr_at<D>(lane, 1, db);
  }

  // ---- online-softmax state ------------------------------------------------
  // Softmax runs in log2 units with a *lazy* running max: a row's m only
  // moves when a new score exceeds it by more than kTau, so P = 2^(x - m)
  // stays <= 2^kTau (exact in fp16/bf16 up to rounding) and the O rescale
  // (a multiply of every accumulator) is skipped on almost every tile.  Row
  // sums add the rounded P that the P V MFMA uses, in fp32, so O = sum P V /
  // sum P stays a weighted mean of V even for one dominant key (the reference
  // sums the unrounded p, attnfuse/compiler/codegen.py:227, which is further
  // from exact attention).  One v_dot2_f32_{f16,bf16} against (1, 1) adds
  // a packed pair exactly (f16 denormals kept) and co-issues with the MFMAs
  // of other waves: 16 per tile, where v_fma_mix took 32 (f16) and
  // shift/mask + add 64 (bf16).
  constexpr float kTau = 8.f;
  constexpr float kNegBig = -1.0e30f;
  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  float lsum[2] = {0.f, 0.f};
  float m_run = kNegBig;
  float slope2 = 0.f;
  if constexpr (BIAS == BIAS_ALIBI) slope2 = p.slopes[hq] * kLog2e;
  // Causal-type masks: every visible key has j <= i, so -slope |i - j| =
  // slope (j - i) is linear in the key index.  Register r of a 32-key block
  // holds key j0 + k_r (j0 = block start + 8h, k_r = 16 (r/8) + r%8), so the
  // logit is (s + u k_r) * zc + slope (j0 - i) with u = slope / zc: the
  // u k_r part is the initial accumulator of the score MFMAs (the same for
  // every tile and lane) and slope (j0 - i) is one offset per block.
  constexpr bool kAlibiOneSided = BIAS == BIAS_ALIBI && (MASK == MASK_CAUSAL || MASK == MASK_CSW);
  const float zc0 = (NORM == NORM_SOFTMAX) ? c2 : p.scale;            // score -> logit scale
  const float aslope = (NORM == NORM_SOFTMAX) ? slope2 : slope2 * kLn2;  // slope in logit units
  f32x16 sinit = f32x16{};
  if constexpr (kAlibiOneSided) {
    const float u = aslope / zc0;
#pragma unroll
    for (int r = 0; r < 16; ++r) sinit[r] = u * (float)(16 * (r >> 3) + (r & 7));
  }
  const uint16_t* brow = nullptr;
  if constexpr (BIAS == BIAS_ADD) brow = p.bias + b * p.bs[0] + hq * p.bs[1] + (int64_t)qrow * p.bs[2];

  // S^T = K Q^T of tile t (two 32-key blocks), K from its LDS slot.
  auto scores = [&](int par, f32x16* s) {
    const uint16_t* Ks = lds + par * TILE;
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      s[kb] = sinit;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s[kb] = E::mfma32(ld16(Ks + 32 * kb * D + koff[ks]), qf[ks], s[kb]);
    }
  };
  // The same in two parts, for head dims whose operands fit in registers
  // next to the scores: every K operand of a tile is read from LDS first, so
  // that the MFMAs, issued later, find them landed instead of each waiting
  // out one LDS round trip.
  constexpr bool kBatchK = D <= 64;
  constexpr bool kBatchV = D <= 128;
  // The first key block's operands are read up front; the second block's
  // are read as the first block's MFMAs issue.
  auto read_k = [&](int par, u32x4 (&kop)[KS]) {
    const uint16_t* Ks = lds + par * TILE;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kop[ks] = ld16(Ks + koff[ks]);
  };
  auto scores_k = [&](int par, const u32x4 (&kop)[KS], f32x16* s) {
    const uint16_t* Ks = lds + par * TILE;
    s[0] = sinit;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s[0] = E::mfma32(kop[ks], qf[ks], s[0]);
#pragma unroll
    for (int kb = 1; kb < BN / 32; ++kb) {
      s[kb] = sinit;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s[kb] = E::mfma32(ld16(Ks + 32 * kb * D + koff[ks]), qf[ks], s[kb]);
    }
  };

  // S^T of tile t recomputed from K in global memory, for the rare step that
  // must move the running max after its K slot has been refilled.  Same
  // operand layout as the LDS reads above; keys past N_kv read as zeros
  // (their scores are masked).
  auto scores_global = [&](int t, f32x16* s) {
    const int n0 = tile_n0(t);
    const auto kr = make_rsrc(kbase + (int64_t)n0 * kstr, span_bytes<D>(p.Nkv - n0, kstr));
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      const uint32_t row = (uint32_t)((32 * kb + kperm(c)) * kstr + 8 * h) * 2u;
      s[kb] = sinit;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s[kb] = E::mfma32(buf_ld16(kr, row + 32u * ks), qf[ks], s[kb]);
    }
  };

  // Affine map (zc, off[kb]) from a score of key block kb to its logit minus
  // the running max (log2 units for softmax, natural units for relu).
  struct Logit {
    float zc, off[BN / 32];
  };
  // Bias and mask of tile t's scores s; returns the map without the running
  // max.  `count` adds the tile to the coverage counters (once per tile).
  auto bias_mask = [&](int t, f32x16* s, bool count) -> Logit {
    const int n0 = tile_n0(t);
    bool active = q0w < p.Nq && n0 >= 0 && n0 < p.Nkv;
    if constexpr (MASK == MASK_CAUSAL) active = active && n0 <= q0w + 31;
    if constexpr (MASK == MASK_SW)
      active = active && n0 + BN - 1 > q0w - p.window && n0 < q0w + 31 + p.window;
    if constexpr (MASK == MASK_CSW)
      active = active && n0 + BN - 1 > q0w - p.window && n0 <= q0w + 31;

    // A wave whose rows see nothing of this stage still runs it (all its
    // scores are masked, so P = 0 and O, l are unchanged): a branch around
    // the MFMAs would force the accumulators through copies every iteration.
    if (count && active && p.coverage != nullptr && lane == 0) {
      const int64_t ci = ((int64_t)(b * p.Hq + hq) * p.cov_nq + (q0w >> 5)) * p.cov_nk + (n0 >> 6);
      atomicAdd(p.coverage + ci, 1u);
    }
    bool need_mask = !active || n0 + BN > p.Nkv;
    if constexpr (MASK == MASK_CAUSAL) need_mask = need_mask || n0 + BN - 1 > q0w;
    if constexpr (MASK == MASK_SW)
      need_mask = need_mask || (q0w + 31 - n0 >= p.window) || (n0 + BN - 1 - q0w >= p.window);
    if constexpr (MASK == MASK_CSW)
      need_mask = need_mask || (q0w + 31 - n0 >= p.window) || n0 + BN - 1 > q0w;

    Logit lg;
    lg.zc = zc0;
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb)
      lg.off[kb] = kAlibiOneSided ? aslope * (float)(n0 + 32 * kb + 8 * h - qrow) : 0.f;
    if constexpr (BIAS == BIAS_ADD) {
      const float bscale = (NORM == NORM_SOFTMAX) ? kLog2e : 1.f;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int key0 = n0 + 32 * kb + 16 * j + 8 * h;
          float bv[8];
          if (qrow < p.Nq && key0 + 8 <= p.Nkv) {
            unpack8<E>(ld16(brow + key0 * p.bs[3]), bv);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint16_t raw = (qrow < p.Nq && key0 + e < p.Nkv) ? brow[(key0 + e) * p.bs[3]] : 0;
              bv[e] = E::lo(raw);
            }
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) s[kb][8 * j + e] = __builtin_fmaf(s[kb][8 * j + e], lg.zc, bv[e] * bscale);
        }
      lg.zc = 1.f;
    } else if constexpr (BIAS == BIAS_ALIBI) {
      if constexpr (!kAlibiOneSided) {
        // two-sided windows: -slope |i - j| per element
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = n0 + 32 * kb + acc_key(r, h);
            s[kb][r] = __builtin_fmaf(s[kb][r], lg.zc, -aslope * (float)abs(qrow - key));
          }
        lg.zc = 1.f;
      }
    }
    if (need_mask) {
      // Register r of key block kb holds key base + kr(r), base = n0 + 32 kb
      // + 8h, kr(r) = 16 (r/8) + r%8: every condition is a range lo <= kr <=
      // hi, one or two compares against a constant per element.
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
        const int base = n0 + 32 * kb + 8 * h;
        int hi = p.Nkv - 1 - base;
        int lo = 0;
        if constexpr (MASK == MASK_CAUSAL || MASK == MASK_CSW) hi = min(hi, qrow - base);
        if constexpr (MASK == MASK_SW) hi = min(hi, qrow + p.window - 1 - base);
        if constexpr (MASK == MASK_SW || MASK == MASK_CSW) lo = qrow - p.window + 1 - base;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 16 * (r >> 3) + (r & 7);
          bool ok = kr <= hi;
          if constexpr (MASK == MASK_SW || MASK == MASK_CSW) ok = ok && kr >= lo;
          s[kb][r] = ok ? s[kb][r] : -INFINITY;
        }
      }
    }
    if constexpr (MASK == MASK_BSE) {
      // element mask of a partial block-sparse tile (rare; a uniform
      // branch): the bits of this lane's query row over the tile's 64 keys,
      // key block kb in half kb
      if (bst.partial(t)) {
        const int e = bst.entry(t);
        const int64_t word = (((int64_t)mb * p.bs_part_rs + (e - bs_nfull)) * p.bs_block_m + (qrow - m0)) *
                                 (p.bs_block_n / 64) + bst.sub_of(t);
        const uint32_t* bits = reinterpret_cast<const uint32_t*>(p.bs_row_bits + word);
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) {
          // shifted by this lane's 8 h once, so that every element tests a
          // constant bit (per-element lane shifts would be hoisted out of the
          // loop and held in registers)
          const uint32_t half = (qrow < p.Nq ? bits[kb] : 0u) >> (8 * h);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            s[kb][r] = (half & (1u << (16 * (r >> 3) + (r & 7)))) ? s[kb][r] : -INFINITY;
        }
      }
    }
    return lg;
  };

  // Running max of the biased, masked scores s of one tile (softmax only):
  // moves m_run when some row grew past the slack, with the O / l rescale,
  // and returns lg with the running max subtracted.
  auto rebase = [&](const f32x16* s, Logit lg) -> Logit {
    if constexpr (NORM == NORM_SOFTMAX) {
      float mz = -INFINITY;
      if constexpr (kAlibiOneSided) {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) {
          float mk = -INFINITY;
#pragma unroll
          for (int r = 0; r < 16; ++r) mk = fmaxf(mk, s[kb][r]);
          mz = fmaxf(mz, __builtin_fmaf(mk, lg.zc, lg.off[kb]));
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mz = fmaxf(mz, s[kb][r]);
        mz = __builtin_fmaf(mz, lg.zc, lg.off[0]);
      }
      const float mx = max_xor32(mz);
      // The rescale runs only when some row of the wave grew past the
      // slack.  It multiplies the accumulators in place (tied asm
      // operands): written as plain C++ inside the branch, the register
      // allocator gives the two paths different registers and copies every
      // accumulator on every iteration.  The s_nops give the MFMA->VALU
      // and VALU->MFMA dependencies on the accumulators their wait states,
      // which the hazard recognizer cannot see through the asm; alpha is an
      // operand of the nops so its v_exp is issued before them.
      const bool grow = mx > m_run + kTau;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float m_new = grow ? mx : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : : "v"(alpha));
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x = o[db][r];
            asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x) : "v"(alpha));
            o[db][r] = x;
          }
        lsum[0] *= alpha;
        lsum[1] *= alpha;
        asm volatile("s_nop 7");
        m_run = m_new;
      }
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) lg.off[kb] -= m_run;
    }
    return lg;
  };

  // P = 2^(logit) (or relu) of one tile in place and its rounded 16-bit P^T
  // as the B operands of the P V MFMA (one per 16 keys).
  auto softmax_tile = [&](f32x16* s, const Logit& lg, u32x4* pf) {
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = __builtin_fmaf(s[kb][r], lg.zc, lg.off[kb]);
        s[kb][r] = (NORM == NORM_SOFTMAX) ? __builtin_amdgcn_exp2f(x) : fmaxf(x, 0.f);
      }
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk) {
      const int kb = kk >> 1, j = kk & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[kk][i] = E::pack(s[kb][8 * j + 2 * i], s[kb][8 * j + 2 * i + 1]);
    }
  };
  // fp32 sums of the rounded P over this lane's 32 keys (the partner lane
  // l ^ 32 holds the other 32), one v_dot2 per packed pair: added into the
  // two running chains ...
  auto add_rowsum = [&](const u32x4* pf) {
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) E::dot_pair(pf[kk][i], lsum[i & 1]);
  };
  // ... or summed alone, over four chains, for the test of a lazy step
  auto tile_rowsum = [&](const u32x4* pf) -> float {
    float ts[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) E::dot_first(pf[0][i], ts[i]);
#pragma unroll
    for (int kk = 1; kk < BN / 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) E::dot_pair(pf[kk][i], ts[i]);
    E::sums_ready(ts[0], ts[1], ts[2], ts[3]);
    return (ts[0] + ts[1]) + (ts[2] + ts[3]);
  };

  // O += P V(t), V^T read transposed from its LDS slot.
  auto pv = [&](int par, const u32x4* pf) {
    const uint16_t* Vs = lds + (kSlots + par) * TILE;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int kk = 0; kk < BN / 16; ++kk) {
        const uint16_t* vt = Vs + 16 * kk * D;
        const u32x2 lo = lds_read_tr16(vt + voff[db][0]);
        const u32x2 hi = lds_read_tr16(vt + voff[db][1]);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
        o[db] = E::mfma32(va, pf[kk], o[db]);
      }
    }
  };
  // Pipelined form: the V^T operands are read kVAhead MFMAs ahead of the
  // MFMA that consumes them (read one by one, each MFMA waited out the LDS
  // round trip of its own transposing reads).  The scheduling barriers keep
  // the compiler from sinking each read back next to its MFMA.
  constexpr int kVOps = DB * (BN / 16);
#ifndef AF_FWD_V_AHEAD
#define AF_FWD_V_AHEAD(D) ((D) <= 64 ? 4 : 2)
#endif
  constexpr int kVAhead = kVOps < AF_FWD_V_AHEAD(D) ? kVOps : AF_FWD_V_AHEAD(D);
  auto read_vop = [&](int par, int i) -> u32x4 {
    const int kk = i / DB, db = i % DB;
    const uint16_t* vt = lds + (kSlots + par) * TILE + 16 * kk * D;
    const u32x2 lo = lds_read_tr16(vt + voff[db][0]);
    const u32x2 hi = lds_read_tr16(vt + voff[db][1]);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  auto pv_pipe = [&](int par, const u32x4* pf) {
    u32x4 vop[kVOps];
#pragma unroll
    for (int i = 0; i < kVAhead; ++i) vop[i] = read_vop(par, i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kVOps; ++i) {
      const int kk = i / DB, db = i % DB;
      o[db] = E::mfma32(vop[i], pf[kk], o[db]);
      if (i + kVAhead < kVOps) vop[i + kVAhead] = read_vop(par, i + kVAhead);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One step with the running max computed first (every step for relu and
  // ALiBi; the first step otherwise): bias, mask and max of tile t, then the score
  // MFMAs of tile t+1 in the same basic block as P of tile t, and P V(t).
  auto step_exact = [&](int t, int par, f32x16* s, f32x16* nxt) {
    u32x4 kop[KS];
    if constexpr (kBatchK) {
      read_k(par ^ 1, kop);
      __builtin_amdgcn_sched_barrier(0);
    }
    const Logit lg = rebase(s, bias_mask(t, s, true));
    if constexpr (kBatchK) {
      scores_k(par ^ 1, kop, nxt);
    } else {
      scores(par ^ 1, nxt);
    }
    u32x4 pf[BN / 16];
    softmax_tile(s, lg, pf);
    add_rowsum(pf);
    if constexpr (kBatchV) {
      pv_pipe(par, pf);
    } else {
      pv(par, pf);
    }
  };

  // Later softmax steps skip the max: P is taken against the current
  // running max, and the sums of the rounded P then tell whether the max has
  // to move.  If every lane's sum is below 2^kRedo, every P of the tile is
  // below 2^kRedo -- finite in fp16 and bf16, like the P <= 2^kTau of the
  // exact step -- and the step stands.  Otherwise (a row grew by more than
  // kRedo, or meets its first visible keys: m_run = -1e30 makes every P
  // infinite) the scores of tile t are recomputed from global memory, its K
  // slot already holding tile t+2, and the step runs exactly.  This saves
  // the max (16 v_max3, a lane swap and the compare) on almost every tile.
  constexpr float kRedo = 8192.f;  // 2^13
  auto step_lazy = [&](int t, int par, f32x16* s, f32x16* nxt) {
    u32x4 kop[KS];
    if constexpr (kBatchK) {
      read_k(par ^ 1, kop);
      __builtin_amdgcn_sched_barrier(0);
    }
    const Logit lg0 = bias_mask(t, s, true);
    Logit lg = lg0;
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) lg.off[kb] -= m_run;
    if constexpr (kBatchK) {
      scores_k(par ^ 1, kop, nxt);
    } else {
      scores(par ^ 1, nxt);
    }
    u32x4 pf[BN / 16];
    softmax_tile(s, lg, pf);
    float tsum = tile_rowsum(pf);
    if (__builtin_amdgcn_ballot_w64(!(tsum < kRedo)) != 0) {
      scores_global(t, s);
      const Logit lg1 = rebase(s, bias_mask(t, s, false));
      softmax_tile(s, lg1, pf);
      tsum = tile_rowsum(pf);
    }
    lsum[0] += tsum;
    if constexpr (kBatchV) {
      pv_pipe(par, pf);
    } else {
      pv(par, pf);
    }
  };

  // ---- deferred P V: one interleaved instruction stream per step ------------
  // Step t of the deferred pipeline runs the score MFMAs of tile t+1 and the
  // P V MFMAs of tile t-1 (P(t-1) kept packed from the previous step) while
  // the VALU computes P of tile t.  All three are independent, so the step
  // is one basic block in which every MFMA is followed by its share of the
  // softmax: a fused multiply-add, an exponential, a convert and a row-sum
  // dot of one packed pair, each pair's three stages one chunk apart, and
  // the LDS operand reads kOpAhead MFMAs ahead.  The scheduling barriers fix
  // that order.  Without them the lazy test (below) splits each step into
  // a VALU-only run before it and an MFMA-only run of P V after it.
  constexpr int kSM = 2 * KS;            // score MFMAs per tile
  constexpr int kPM = DB * (BN / 16);    // P V MFMAs per tile (== kSM)
  constexpr int kPairs = BN / 4;         // packed P pairs per lane and tile
  static_assert(kSM == kPM, "score and P V MFMAs alternate");
#ifndef AF_FWD_OP_AHEAD
#define AF_FWD_OP_AHEAD 4
#endif
  constexpr int kOpAhead = AF_FWD_OP_AHEAD;
  // operand of score MFMA j: key block j % 2, k-step j / 2
  auto read_sop = [&](int par, int j) -> u32x4 {
    return ld16(lds + par * TILE + 32 * (j & 1) * D + koff[j >> 1]);
  };
  // S(t+1) into nxt (key slot kpar), with PV: O += P(t-1) V(t-1) (value slot
  // vpar, P in pprev); P(t) of the scores s under lg into pf.  Returns the
  // fp32 sum of this lane's 32 rounded P of tile t.
  auto mix = [&](auto pv_on, int kpar, int vpar, f32x16* s, const Logit& lg, f32x16* nxt,
                 const u32x4* pprev, u32x4* pf) -> float {
    constexpr bool PV = decltype(pv_on)::value;
    constexpr int M = PV ? kSM + kPM : kSM;
    constexpr int A = M < kOpAhead ? M : kOpAhead;
    // pairs whose softmax starts in one chunk, and chunks between starts
    constexpr int PPC = kPairs >= M ? kPairs / M : 1;
    constexpr int CPP = M >= kPairs ? M / kPairs : 1;
    static_assert(PPC * M == kPairs * CPP, "pairs spread evenly over the chunks");
    // MFMA i: with PV even i is score MFMA i/2 and odd i P V MFMA i/2
    auto read_op = [&](int i) -> u32x4 {
      if (PV && (i & 1)) return read_vop(vpar, i >> 1);
      return read_sop(kpar, PV ? i >> 1 : i);
    };
    u32x4 op[M];
    float ts[4];
#pragma unroll
    for (int i = 0; i < A; ++i) op[i] = read_op(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < M + 2; ++c) {
      if (c < M) {
        if (PV && (c & 1)) {
          const int j = c >> 1;
          o[j % DB] = E::mfma32(op[c], pprev[j / DB], o[j % DB]);
        } else {
          const int j = PV ? c >> 1 : c;
          const int kb = j & 1, ks = j >> 1;
          nxt[kb] = E::mfma32(op[c], qf[ks], ks == 0 ? sinit : nxt[kb]);
        }
      }
      if (c + A < M) op[c + A] = read_op(c + A);
      // stage st of pair p runs in chunk p * M / kPairs + st: PPC pairs
      // start in every CPP-th chunk
#pragma unroll
      for (int st = 0; st < 3; ++st) {
        const int cs = c - st;
        if (cs < 0 || cs % CPP != 0 || cs / CPP * PPC >= kPairs) continue;
#pragma unroll
        for (int jp = 0; jp < PPC; ++jp) {
          const int p = cs / CPP * PPC + jp;
          const int kb = p >> 3, r = 2 * (p & 7);
          if (st == 0) {
            s[kb][r] = __builtin_fmaf(s[kb][r], lg.zc, lg.off[kb]);
            s[kb][r + 1] = __builtin_fmaf(s[kb][r + 1], lg.zc, lg.off[kb]);
          } else if (st == 1) {
            s[kb][r] = __builtin_amdgcn_exp2f(s[kb][r]);
            s[kb][r + 1] = __builtin_amdgcn_exp2f(s[kb][r + 1]);
          } else {
            const uint32_t w2 = E::pack(s[kb][r], s[kb][r + 1]);
            pf[2 * kb + (r >> 3)][(r & 7) >> 1] = w2;
            if (p < 4) E::dot_first(w2, ts[p & 3]);
            else E::dot_pair(w2, ts[p & 3]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    E::sums_ready(ts[0], ts[1], ts[2], ts[3]);
    return (ts[0] + ts[1]) + (ts[2] + ts[3]);
  };

  // ---- software pipeline ---------------------------------------------------
  // Iteration t issues the loads of K(t+2) and V(t+1), masks tile t (and for
  // an exact step updates the running max), then runs the score MFMAs of
  // tile t+1 (on the matrix pipe while this wave computes P of tile t on the
  // VALU) and P V(t).  In the last iteration the score MFMAs read a stale K
  // slot and their result is dropped.  Slot reuse: K(t+2) overwrites K(t),
  // last read by the score MFMAs of iteration t-1; V(t+1) overwrites V(t-1),
  // last read in iteration t-1; the barrier closing each iteration separates
  // the two.
  // The deferred pipeline (below) loads V(t) in step t instead, and the
  // unpipelined step loads K(t+1) and V(t+1).
  constexpr bool kUnpiped = fwd_unpipelined<D, MASK, BIAS, NORM>();
  if (ntiles > 0) {
    load_k(0, 0);
    if constexpr (!kDefer) load_v(0, 0);
  }
  if (!kUnpiped && ntiles > 1) load_k(1, 1);
  wait_lds_dma();
  __syncthreads();
  f32x16 sa[BN / 32], sb[BN / 32];
  if (!kUnpiped && ntiles > 0) scores(0, sa);
  // Step 0 loads K(2) into slot 0, which every wave has just read for
  // scores(0): no wave may issue that load before all of them have their
  // K(0) operands (each wave's reads complete before it reaches the
  // barrier).  In later steps the barrier closing step t-1 orders the reads
  // of slot par (scores(t), issued in step t-1) before the load into it.
  __syncthreads();
  // loads of K(t+2) into K slot par and V(t+1) into V slot par ^ 1
  auto issue = [&](int t, int par) {
    if (t + 2 < ntiles) load_k(t + 2, par);
    if (t + 1 < ntiles) load_v(t + 1, par ^ 1);
  };
  // this wave's loads have landed; after the barrier every wave's have, and
  // no wave reads slot K(t) / V(t) any more
  auto close = [&]() {
    wait_lds_dma();
    __syncthreads();
  };
  // Walked towards the query, ALiBi raises a row's max on nearly every tile
  // (by slope * 64), which would make every lazy step recompute its tile.
  // Causal-type ALiBi walks away from the query (kDescend) and two-sided
  // ALiBi outwards from it (kOutward), so ALiBi steps are lazy like the rest.
  constexpr bool kLazy = NORM == NORM_SOFTMAX && (BIAS != BIAS_ALIBI || kDescend || kOutward);
  static_assert(!kDefer || kLazy, "the deferred pipeline takes lazy steps");
  if constexpr (kDefer) {
    // Step t loads K(t+2) into K slot t & 1 and V(t) into V slot t & 1, reads
    // K(t+1) and V(t-1) from the other slots, and the P V of the last tile
    // follows the loop.  Slot reuse: K slot t & 1 held K(t), last read by
    // the score MFMAs of step t-1; V slot t & 1 held V(t-2), last read by the
    // P V of step t-1; the barrier closing step t-1 separates them.
    auto issue_d = [&](int t, int par) {
      if (t + 2 < ntiles) load_k(t + 2, par);
      load_v(t, par);
    };
    using no_pv = std::integral_constant<bool, false>;
    using with_pv = std::integral_constant<bool, true>;
    u32x4 pa[BN / 16], pb[BN / 16];
    // step t >= 1 of parity par: P V(t-1) with pprev, P(t) into pf
    auto step_d = [&](int t, int par, f32x16* s, f32x16* nxt, const u32x4* pprev, u32x4* pf) {
      issue_d(t, par);
      const Logit lg0 = bias_mask(t, s, true);
      Logit lg = lg0;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) lg.off[kb] -= m_run;
      float tsum = mix(with_pv{}, par ^ 1, par ^ 1, s, lg, nxt, pprev, pf);
      if (__builtin_amdgcn_ballot_w64(!(tsum < kRedo)) != 0) {
        scores_global(t, s);
        const Logit lg1 = rebase(s, bias_mask(t, s, false));
        softmax_tile(s, lg1, pf);
        tsum = tile_rowsum(pf);
      }
      lsum[0] += tsum;
      close();
    };
    if (ntiles > 0) {
      issue_d(0, 0);
      const Logit lg = rebase(sa, bias_mask(0, sa, true));
      lsum[0] += mix(no_pv{}, 1, 1, sa, lg, sb, pb, pa);
      close();
    }
    for (int t = 1; t < ntiles; t += 2) {
      step_d(t, 1, sb, sa, pa, pb);
      if (t + 1 < ntiles) step_d(t + 1, 0, sa, sb, pb, pa);
    }
    if (ntiles > 0) {
      // P(ntiles-1) is in pa for an even tile index, pb for an odd one
      if ((ntiles - 1) & 1) pv_pipe(1, pb);
      else pv_pipe(0, pa);
    }
  } else if constexpr (kUnpiped) {
    // Step t computes the scores, P and P V of tile t from slots t & 1 and
    // loads K(t+1), V(t+1) into the other slots, which every wave left at
    // the barrier closing step t-1.  The loads are issued after the score
    // MFMAs (issued first they delayed them: 1-2 % slower).  A lazy step
    // that fails its test recomputes the scores from the K slot, which
    // still holds K(t).  One score tile live instead of two leaves room for
    // a fourth wave per SIMD (a third with ALiBi's initial accumulator), and
    // the interleaving of the waves covers what the pipelined step
    // overlapped inside one wave.
    auto step_unpiped = [&](int t, int par, bool exact) {
      u32x4 kop[KS];
      read_k(par, kop);
      __builtin_amdgcn_sched_barrier(0);
      scores_k(par, kop, sa);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < ntiles) {
        load_k(t + 1, par ^ 1);
        load_v(t + 1, par ^ 1);
      }
      u32x4 pf[BN / 16];
      if (exact) {
        const Logit lg = rebase(sa, bias_mask(t, sa, true));
        softmax_tile(sa, lg, pf);
        add_rowsum(pf);
      } else {
        Logit lg = bias_mask(t, sa, true);
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) lg.off[kb] -= m_run;
        softmax_tile(sa, lg, pf);
        float tsum = tile_rowsum(pf);
        if (__builtin_amdgcn_ballot_w64(!(tsum < kRedo)) != 0) {
          scores(par, sa);
          const Logit lg1 = rebase(sa, bias_mask(t, sa, false));
          softmax_tile(sa, lg1, pf);
          tsum = tile_rowsum(pf);
        }
        lsum[0] += tsum;
      }
      pv_pipe(par, pf);
      close();
    };
    if (ntiles > 0) step_unpiped(0, 0, true);
    for (int t = 1; t < ntiles; t += 2) {
      step_unpiped(t, 1, !kLazy);
      if (t + 1 < ntiles) step_unpiped(t + 1, 0, !kLazy);
    }
  } else if constexpr (kLazy) {
    if (ntiles > 0) {
      issue(0, 0);
      step_exact(0, 0, sa, sb);
      close();
    }
    for (int t = 1; t < ntiles; t += 2) {
      issue(t, 1);
      step_lazy(t, 1, sb, sa);
      close();
      if (t + 1 < ntiles) {
        issue(t + 1, 0);
        step_lazy(t + 1, 0, sa, sb);
        close();
      }
    }
  } else {
    for (int t = 0; t < ntiles; t += 2) {
      issue(t, 0);
      step_exact(t, 0, sa, sb);
      close();
      if (t + 1 < ntiles) {
        issue(t + 1, 1);
        step_exact(t + 1, 1, sb, sa);
        close();
      }
    }
  }
  // ---- epilogue -------------------------------------------------------------
  // this lane's 32 keys of every tile, plus the partner lane's 32
  float lt = lsum[0] + lsum[1];
  lt += xor32(lt);
  // The lane's row and half are taken from the lane id again: kept from
  // the prologue, the compiler spilled them (and a 64-bit copy of the row)
  // across the loop at three waves per SIMD.
  int le = __lane_id();
  asm volatile("" : "+v"(le));
  const int he = le >> 5, qre = q0w + (le & 31);
  if (kIsBs<MASK> && bs_slot >= 0) {
    // a piece of a split row: unnormalised O and (m, l) for the combine
    if (qre < p.Nq) {
      const int64_t prow = ((int64_t)bs_slot * BH + bh) * BM + (qre - m0);
      float* orow = p.part_o + prow * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(orow + 32 * db + 8 * g + 4 * he) =
              f32x4{o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
      if (he == 0) *reinterpret_cast<f32x2*>(p.part_ml + 2 * prow) = f32x2{m_run, lt};
    }
    return;
  }
  const float inv = (lt == 0.f) ? 1.f : 1.f / lt;
  if (qre < p.Nq) {
    uint16_t* orow = p.o + b * p.os[0] + hq * p.os[1] + (int64_t)qre * p.os[2];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * he;
        u32x2 w2;
        w2[0] = E::pack(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
        w2[1] = E::pack(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d0) = w2;
      }
    if (p.lse != nullptr && he == 0) {
      float L = -INFINITY;
      if constexpr (NORM == NORM_SOFTMAX) {
        if (lt > 0.f) L = (m_run + __log2f(lt)) * kLn2;
      }
      p.lse[b * p.ls[0] + hq * p.ls[1] + (int64_t)qre * p.ls[2]] = L;
    }
  }
}

}  // namespace af
