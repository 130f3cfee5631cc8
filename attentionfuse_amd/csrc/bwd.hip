// Backward entry point: validation, grid shapes and the three launches
// (delta, dK/dV, dQ) on the caller's stream.
#include <string.h>

#include <algorithm>

#include "bs_split.hpp"
#include "bwd_launch.hpp"
#include "launch.hpp"
#include "validate.hpp"

namespace af {

// A caller's group_split must be a power of two dividing the group size.
bool group_split_valid(const af_bwd_args& a) {
  const int s = a.group_split;
  if (s == 0) return true;
  if (s < 0 || (s & (s - 1)) != 0 || a.heads_kv <= 0 || a.heads_q % a.heads_kv != 0) return false;
  return (a.heads_q / a.heads_kv) % s == 0;
}

int bwd_group_split(const af_bwd_args& a) {
  if (a.group_split > 0 && group_split_valid(a)) return a.group_split;
  if (a.batch <= 0 || a.heads_kv <= 0 || a.heads_q <= 0 || a.seqlen_kv <= 0 || a.heads_q % a.heads_kv != 0) return 1;
  const int G = a.heads_q / a.heads_kv;
  const int64_t base = (int64_t)((a.seqlen_kv + 127) / 128) * a.batch * a.heads_kv;
  int gs = 1;
  while (G % (2 * gs) == 0 && base * 2 * gs <= 512) gs *= 2;
  return gs;
}

// The block mask's K-major plan is used when its columns are split and the
// GQA query heads are not: the library then keeps the heads together (the
// column pieces already fill the grid) unless the caller asks for a split.
static bool kv_plan_wanted(const af_bwd_args& a, const af_blockmask* bm) {
  return bm != nullptr && a.key.mask == AF_MASK_BLOCK_SPARSE && a.key.dtype != AF_F32 && bm->kv_items != nullptr;
}

int bwd_group_split_for(const af_bwd_args& a, const af_blockmask* bm) {
  if (kv_plan_wanted(a, bm) && bm->n_kv_splits > 0 && a.group_split == 0) return 1;
  return bwd_group_split(a);
}

BwdWorkspace bwd_workspace_layout(const af_bwd_args& a, const af_blockmask* bm) {
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  BwdWorkspace w{0, 0, 0, 0, 0, 0, 0, 0, 0, 1, false, false};
  if (a.batch <= 0 || a.heads_q <= 0 || a.heads_kv <= 0 || a.seqlen_q < 0 || a.seqlen_kv < 0 || a.key.head_dim <= 0)
    return w;
  const size_t rows_q = (size_t)a.batch * a.heads_q * a.seqlen_q;
  const size_t rows_k = (size_t)a.batch * a.heads_kv * a.seqlen_kv;
  w.ld = 0;
  const size_t elem = a.key.dtype == AF_F32 ? 4 : 2;
  w.total = up(rows_q * 2 * sizeof(float));
  if (a.key.rope) {
    w.qr = w.total;
    w.total += up(rows_q * a.key.head_dim * elem);
    w.kr = w.total;
    w.total += up(rows_k * a.key.head_dim * elem);
  }
  w.g_split = bwd_group_split_for(a, bm);
  if (w.g_split > 1) {
    w.dkp = w.total;
    w.total += up((size_t)w.g_split * rows_k * a.key.head_dim * 4);
    w.dvp = w.total;
    w.total += up((size_t)w.g_split * rows_k * a.key.head_dim * 4);
  }
  // block-sparse work plans: partial rows of the split lists
  if (bm != nullptr && a.key.mask == AF_MASK_BLOCK_SPARSE && a.key.dtype != AF_F32) {
    w.q_plan = bm->q_items != nullptr;
    w.kv_plan = kv_plan_wanted(a, bm) && w.g_split == 1;
    if (w.q_plan && bm->n_q_slots > 0) {
      w.pdq = w.total;
      w.total += up((size_t)bm->n_q_slots * a.batch * a.heads_q * bm->block_m * a.key.head_dim * 4);
    }
    if (w.kv_plan && bm->n_kv_slots > 0) {
      const size_t part = up((size_t)bm->n_kv_slots * a.batch * a.heads_kv * bm->block_n * a.key.head_dim * 4);
      w.pdk = w.total;
      w.pdv = w.total + part;
      w.total += 2 * part;
    }
  }
  if (rows_q == 0 && rows_k == 0) w.total = 0;
  return w;
}

size_t bwd_workspace_bytes(const af_bwd_args& a, const af_blockmask* bm) { return bwd_workspace_layout(a, bm).total; }

static int bad(int code, const char* msg) {
  set_error("%s", msg);
  return code;
}

int run_bwd(const af_bwd_args* a, const af_blockmask* bm, void* workspace, size_t workspace_bytes,
            hipStream_t stream) {
  if (a == nullptr) return bad(AF_ERR_BAD_ARG, "args is NULL");
  const af_spec_key& k = a->key;
  const bool f32 = k.dtype == AF_F32;
  if (k.dtype != AF_F16 && k.dtype != AF_BF16 && !f32)
    return bad(AF_ERR_UNSUPPORTED, "backward takes fp16, bf16 or fp32");
  if (!head_dim_supported(k.head_dim)) return bad(AF_ERR_UNSUPPORTED, "backward head_dim must be 32, 64, 128 or 256");
  if (f32 && k.head_dim == 256) return bad(AF_ERR_UNSUPPORTED, "the fp32 backward takes head dims 32, 64 and 128");
  if (k.mask < 0 || k.mask > 4) return bad(AF_ERR_UNSUPPORTED, "unknown mask kind");
  if (k.bias != AF_BIAS_NONE && k.bias != AF_BIAS_ALIBI)
    return bad(AF_ERR_UNSUPPORTED, "backward supports no bias or ALiBi");
  if (k.norm != AF_NORM_SOFTMAX) return bad(AF_ERR_UNSUPPORTED, "backward supports softmax normalisation only");
  if (k.rope != 0 && k.rope != 1) return bad(AF_ERR_UNSUPPORTED, "unknown rope kind");
  int rc;
  const char* names[8] = {"q", "k", "v", "o", "dout", "dq", "dk", "dv"};
  const void* ptrs[8] = {a->q, a->k, a->v, a->o, a->dout, a->dq, a->dk, a->dv};
  const int64_t* strides[8] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride,
                               a->do_stride, a->dq_stride, a->dk_stride, a->dv_stride};
  // q, o, dout, dq have seqlen_q rows; k, v, dk, dv seqlen_kv
  const int64_t nrows[8] = {a->seqlen_q, a->seqlen_kv, a->seqlen_kv, a->seqlen_q,
                            a->seqlen_q,  a->seqlen_q,  a->seqlen_kv, a->seqlen_kv};
  for (int i = 0; i < 8; ++i)
    if ((rc = check_bhnd(names[i], ptrs[i], strides[i], nrows[i]))) return rc;
  if (a->lse == nullptr && a->seqlen_q > 0) return bad(AF_ERR_BAD_ARG, "lse is NULL");
  if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 ||
      a->heads_q % a->heads_kv != 0)
    return bad(AF_ERR_BAD_ARG, "bad sizes (or query heads not a multiple of key/value heads)");
  if ((k.mask == AF_MASK_CAUSAL || k.mask == AF_MASK_SLIDING_WINDOW || k.mask == AF_MASK_CAUSAL_SLIDING_WINDOW) &&
      a->seqlen_q != a->seqlen_kv)
    return bad(AF_ERR_BAD_ARG, "causal / sliding-window masks need seqlen_q == seqlen_kv");
  if ((k.mask == AF_MASK_SLIDING_WINDOW || k.mask == AF_MASK_CAUSAL_SLIDING_WINDOW) && a->window <= 0)
    return bad(AF_ERR_BAD_ARG, "sliding window size must be positive");
  if (k.rope) {
    if (a->cos == nullptr || a->sin == nullptr) return bad(AF_ERR_BAD_ARG, "rope needs cos and sin tables");
    if (a->rope_stride[1] != 1 || a->rope_stride[0] % 8 != 0 || !aligned16(a->cos) || !aligned16(a->sin))
      return bad(AF_ERR_BAD_ARG, "rope tables need unit d-stride, 16-byte aligned rows");
    if (a->rope_len < std::max(a->seqlen_q, a->seqlen_kv)) return bad(AF_ERR_BAD_ARG, "rope tables too short");
  }
  if (k.bias == AF_BIAS_ALIBI && a->alibi_slopes == nullptr) return bad(AF_ERR_BAD_ARG, "ALiBi needs slopes");
  if (!group_split_valid(*a))
    return bad(AF_ERR_BAD_ARG, "group_split must be 0 or a power of two dividing heads_q / heads_kv");
  // the kernels stage Q, dO, K, V and the RoPE tables through buffer
  // resources with a 32-bit byte range per (batch, head) slice
  auto fits = [&](int64_t rows, int64_t stride) {
    return rows <= 0 || ((rows - 1) * stride + k.head_dim) * 2 < (int64_t(1) << 32);
  };
  if (!f32 && (!fits(a->seqlen_q, a->q_stride[2]) || !fits(a->seqlen_q, a->do_stride[2]) ||
               !fits(a->seqlen_kv, a->k_stride[2]) || !fits(a->seqlen_kv, a->v_stride[2]) ||
               (k.rope && !fits(a->rope_len, a->rope_stride[0]))))
    return bad(AF_ERR_UNSUPPORTED, "a (batch, head) slice spans 4 GiB or more");
  // the block mask is validated before the workspace size is computed from it
  if (k.mask == AF_MASK_BLOCK_SPARSE) {
    if (bm == nullptr || bm->full_kv_num == nullptr || bm->full_kv_idx == nullptr || bm->kv_num_blocks == nullptr ||
        bm->kv_indices == nullptr || bm->q_num_blocks == nullptr || bm->q_indices == nullptr)
      return bad(AF_ERR_BAD_ARG, "block-sparse backward needs the Q-major and K-major block lists");
    if (bm->full_kv_stride < 1 || bm->kv_stride < 1 || bm->q_stride < 1)
      return bad(AF_ERR_BAD_ARG, "block mask row strides must be at least 1");
    if ((bm->block_m != 64 && bm->block_m != 128) || (bm->block_n != 64 && bm->block_n != 128))
      return bad(AF_ERR_UNSUPPORTED, "block-sparse backward supports 64 or 128 blocks");
    if (bm->n_q_blocks != (a->seqlen_q + bm->block_m - 1) / bm->block_m ||
        bm->n_kv_blocks != (a->seqlen_kv + bm->block_n - 1) / bm->block_n)
      return bad(AF_ERR_BAD_ARG, "block mask grid does not match the sequence lengths");
    if (bm->q_items != nullptr &&
        (rc = check_plan(bm->n_q_items, bm->q_splits, bm->n_q_splits, bm->n_q_slots, bm->n_q_blocks, "q")))
      return rc;
    if (bm->kv_items != nullptr &&
        (rc = check_plan(bm->n_kv_items, bm->kv_splits, bm->n_kv_splits, bm->n_kv_slots, bm->n_kv_blocks, "kv")))
      return rc;
  }
  const BwdWorkspace wl = bwd_workspace_layout(*a, k.mask == AF_MASK_BLOCK_SPARSE ? bm : nullptr);
  const size_t need = wl.total;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
    return bad(AF_ERR_WORKSPACE,
               k.mask == AF_MASK_BLOCK_SPARSE
                   ? "backward workspace too small (af_bwd_blocksparse_workspace_bytes)"
                   : "backward workspace too small (af_bwd_workspace_bytes)");

  BwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<const uint16_t*>(a->o);
  p.dout = static_cast<const uint16_t*>(a->dout);
  p.lse = a->lse;
  char* ws = static_cast<char*>(workspace);
  p.ld = reinterpret_cast<float*>(ws + wl.ld);
  if (k.rope) {
    p.qr = reinterpret_cast<uint16_t*>(ws + wl.qr);
    p.kr = reinterpret_cast<uint16_t*>(ws + wl.kr);
  }
  p.g_split = wl.g_split;
  if (wl.g_split > 1) {
    p.dkp = reinterpret_cast<float*>(ws + wl.dkp);
    p.dvp = reinterpret_cast<float*>(ws + wl.dvp);
  }
  p.dq = static_cast<uint16_t*>(a->dq);
  p.dk = static_cast<uint16_t*>(a->dk);
  p.dv = static_cast<uint16_t*>(a->dv);
  p.cos = static_cast<const uint16_t*>(a->cos);
  p.sin = static_cast<const uint16_t*>(a->sin);
  p.slopes = a->alibi_slopes;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = a->q_stride[i];
    p.ks[i] = a->k_stride[i];
    p.vs[i] = a->v_stride[i];
    p.os[i] = a->o_stride[i];
    p.dos[i] = a->do_stride[i];
    p.dqs[i] = a->dq_stride[i];
    p.dks[i] = a->dk_stride[i];
    p.dvs[i] = a->dv_stride[i];
  }
  for (int i = 0; i < 3; ++i) p.ls[i] = a->lse_stride[i];
  p.rs[0] = a->rope_stride[0];
  p.rs[1] = a->rope_stride[1];
  p.B = a->batch;
  p.Hq = a->heads_q;
  p.Hkv = a->heads_kv;
  p.Nq = a->seqlen_q;
  p.Nkv = a->seqlen_kv;
  p.G = a->heads_q / a->heads_kv;
  p.window = a->window;
  p.rope_len = a->rope_len;
  p.scale = a->scale;
  // the score kernels read q~ / k~ from the rotated workspace copies (RoPE)
  // or straight from the inputs
  const int64_t D = k.head_dim;
  if (k.rope) {
    p.qt = p.qr;
    p.kt = p.kr;
    const int64_t qts[4] = {(int64_t)a->heads_q * a->seqlen_q * D, (int64_t)a->seqlen_q * D, D, 1};
    const int64_t kts[4] = {(int64_t)a->heads_kv * a->seqlen_kv * D, (int64_t)a->seqlen_kv * D, D, 1};
    for (int i = 0; i < 4; ++i) {
      p.qts[i] = qts[i];
      p.kts[i] = kts[i];
    }
  } else {
    p.qt = p.q;
    p.kt = p.k;
    for (int i = 0; i < 4; ++i) {
      p.qts[i] = p.qs[i];
      p.kts[i] = p.ks[i];
    }
  }

  BwdGrids g;
  g.waves_kv = 4;
  g.waves_q = 4;
  if (k.mask == AF_MASK_BLOCK_SPARSE) {
    if (const int rc = check_elem_masks(bm, k.head_dim)) return rc;
    g.waves_kv = bm->block_n / 32;
    g.waves_q = bm->block_m / 32;
    p.bs_full_num = bm->full_kv_num;
    p.bs_full_idx = bm->full_kv_idx;
    p.bs_part_num = bm->kv_num_blocks;
    p.bs_part_idx = bm->kv_indices;
    p.bs_q_num = bm->q_num_blocks;
    p.bs_q_idx = bm->q_indices;
    p.bs_full_rs = bm->full_kv_stride;
    p.bs_part_rs = bm->kv_stride;
    p.bs_q_rs = bm->q_stride;
    p.bs_row_bits = bm->part_row_bits;
    p.bs_col_bits = bm->q_col_bits;
    p.bs_q_partial = bm->q_partial;
    p.bs_block_m = bm->block_m;
    p.bs_block_n = bm->block_n;
    if (wl.q_plan) {
      p.bs_q_items = bm->q_items;
      if (wl.pdq) p.part_dq = reinterpret_cast<float*>(ws + wl.pdq);
    }
    if (wl.kv_plan) {
      p.bs_kv_items = bm->kv_items;
      if (wl.pdk) {
        p.part_dk = reinterpret_cast<float*>(ws + wl.pdk);
        p.part_dv = reinterpret_cast<float*>(ws + wl.pdv);
      }
    }
  }
  if (a->seqlen_q == 0 && a->seqlen_kv == 0) return AF_OK;
  if (f32) {
    if (launch_bwd_f32(p, *a, stream) != 0) return bad(AF_ERR_UNSUPPORTED, "no fp32 backward for this head dim");
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("fp32 backward launch failed: %s", hipGetErrorString(e));
      return AF_ERR_LAUNCH;
    }
    return AF_OK;
  }
  const int BK = 32 * g.waves_kv, BMq = 32 * g.waves_q;
  p.n_kblocks = (a->seqlen_kv + BK - 1) / BK;
  p.n_qblocks = (a->seqlen_q + BMq - 1) / BMq;
  const int64_t rows = (int64_t)a->batch * a->heads_q * a->seqlen_q +
                       (k.rope ? (int64_t)a->batch * a->heads_kv * a->seqlen_kv : 0);
  const int rpb = 256 / (k.head_dim / 16);
  g.prep = (unsigned)std::max<int64_t>(1, (rows + rpb - 1) / rpb);
  // grid rows: key (query) blocks, or the block-sparse plans' items
  const int kv_rows = p.bs_kv_items != nullptr ? bm->n_kv_items : p.n_kblocks;
  const int q_rows = p.bs_q_items != nullptr ? bm->n_q_items : p.n_qblocks;
  // Under a causal mask key block kb sees N_q - kb BK queries, so the last
  // blocks are light: the last n_kblocks / (2 g_split) run all G heads in one
  // workgroup and store dK/dV directly (fewer partial rows to write and to
  // sum).  Measured at config 5 (g_split 2): combine 14.6 -> 11.6 us, dK/dV +
  // dQ 531 -> 527 us; leaving the last half unsplit (they then do no more
  // work than the first block's split workgroups) saved 5.7 us in the
  // combine but lengthened the tail by 11 us.
  p.n_split_kb = kv_rows;
  if (p.g_split > 1 && k.mask == AF_MASK_CAUSAL && p.bs_kv_items == nullptr)
    p.n_split_kb = p.n_kblocks - p.n_kblocks / (2 * p.g_split);
  p.split_keys = std::min(p.n_split_kb * BK, a->seqlen_kv);
  g.dkv = (unsigned)std::max(1, (p.n_split_kb * p.g_split + (kv_rows - p.n_split_kb)) * a->batch * a->heads_kv);
  g.dq = (unsigned)std::max(1, q_rows * a->batch * a->heads_q);
  if (k.mask == AF_MASK_BLOCK_SPARSE) {
    // the dQ walk re-reads k~ and V of its head, the dK/dV walk q~ and dO
    // of the G query heads of its key/value head
    const int64_t row_bytes = (int64_t)k.head_dim * 2;
    p.bs_q_rows = q_rows;
    p.bs_xcd_heads_q = bs_xcd_heads(a->batch * a->heads_q, 2 * a->seqlen_kv * row_bytes);
    p.bs_xcd_heads_kv = bs_xcd_heads(a->batch * a->heads_kv, 2 * (int64_t)p.G * a->seqlen_q * row_bytes);
  }
  g.combine = 0;
  if (p.g_split > 1) {
    const int64_t krows = (int64_t)a->batch * a->heads_kv * p.split_keys;
    g.combine = (unsigned)((krows + rpb - 1) / rpb);
  }

  const bool f16 = k.dtype == AF_F16;
  // block-sparse walks with element masks run their own instantiations
  const int mask = k.mask == AF_MASK_BLOCK_SPARSE && p.bs_row_bits != nullptr ? MASK_BSE : k.mask;
  int r = -1;
  switch (k.head_dim) {
    case 32:
      r = f16 ? launch_bwd_f16_d32(p, mask, k.bias, k.rope, g, stream)
              : launch_bwd_bf16_d32(p, mask, k.bias, k.rope, g, stream);
      break;
    case 64:
      r = f16 ? launch_bwd_f16_d64(p, mask, k.bias, k.rope, g, stream)
              : launch_bwd_bf16_d64(p, mask, k.bias, k.rope, g, stream);
      break;
    case 128:
      r = f16 ? launch_bwd_f16_d128(p, mask, k.bias, k.rope, g, stream)
              : launch_bwd_bf16_d128(p, mask, k.bias, k.rope, g, stream);
      break;
    case 256:
      r = f16 ? launch_bwd_f16_d256(p, mask, k.bias, k.rope, g, stream)
              : launch_bwd_bf16_d256(p, mask, k.bias, k.rope, g, stream);
      break;
  }
  if (r != 0) return bad(AF_ERR_UNSUPPORTED, "no backward instantiation for this key");
  // sums of the split lists' pieces: one launch for dQ, dV and dK
  BsGradCombineParams c;
  memset(&c, 0, sizeof(c));
  c.B = p.B;
  c.cos = p.cos;
  c.sin = p.sin;
  c.rs = p.rs[0];
  auto add = [&](const int32_t* splits, int n_splits, const float* part, uint16_t* out, const int64_t* os, int H,
                 int Nrows, int blk, float scale, bool rope) {
    BsGradTarget& t = c.t[c.n_targets++];
    t.splits = splits;
    t.n_splits = n_splits;
    t.part = part;
    t.out = out;
    for (int i = 0; i < 3; ++i) t.os[i] = os[i];
    t.H = H;
    t.N = Nrows;
    t.BLK = blk;
    t.scale = scale;
    t.rope = rope;
  };
  if (p.part_dq != nullptr && bm->n_q_splits > 0)
    add(bm->q_splits, bm->n_q_splits, p.part_dq, p.dq, p.dqs, p.Hq, p.Nq, bm->block_m, p.scale, k.rope != 0);
  if (p.part_dk != nullptr && bm->n_kv_splits > 0) {
    add(bm->kv_splits, bm->n_kv_splits, p.part_dv, p.dv, p.dvs, p.Hkv, p.Nkv, bm->block_n, 1.f, false);
    add(bm->kv_splits, bm->n_kv_splits, p.part_dk, p.dk, p.dks, p.Hkv, p.Nkv, bm->block_n, p.scale, k.rope != 0);
  }
  if (c.n_targets > 0) r = launch_bs_grad_combine(c, k.dtype, k.head_dim, stream);
  if (r != 0) return bad(AF_ERR_UNSUPPORTED, "no block-sparse combine for this key");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("backward launch failed: %s", hipGetErrorString(e));
    return AF_ERR_LAUNCH;
  }
  return AF_OK;
}

}  // namespace af
