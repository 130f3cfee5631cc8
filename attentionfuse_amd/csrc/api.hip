// C ABI of libattnfuse_hip.so: argument validation, specialisation-key ->
// instantiation selection and launch.  Declarations and the contract are in
// include/attnfuse_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "attnfuse_hip.h"
#include "bs_split.hpp"
#include "bwd_f32_kernel.hpp"
#include "bwd_launch.hpp"
#include "fwd_f32_kernel.hpp"
#include "launch.hpp"
#include "launch_decode.hpp"
#include "validate.hpp"

namespace af {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

namespace {

constexpr int kKeysPerStage = 64;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// allow_f32: the entry point has fp32 kernels (the forward, block-sparse
// included, and decode; af_bwd checks its own keys).
int check_key(const af_spec_key& k, bool allow_bs, bool allow_f32 = false) {
  if (k.dtype == AF_F32) {
    if (!allow_f32)
      return fail(AF_ERR_UNSUPPORTED, "dtype fp32: af_fwd and af_bwd take fp32 (dense / causal / windowed masks); "
                  "this entry point takes fp16 or bf16");

  } else if (k.dtype != AF_F16 && k.dtype != AF_BF16) {
    return fail(AF_ERR_UNSUPPORTED, "dtype %d: the gfx950 kernels take fp16, bf16 or (forward) fp32", k.dtype);
  }
  if (k.head_dim != 32 && k.head_dim != 64 && k.head_dim != 128 && k.head_dim != 256)
    return fail(AF_ERR_UNSUPPORTED, "head_dim %d: instantiated for 32, 64, 128 and 256", k.head_dim);
  if (k.head_dim == 256 && k.dtype == AF_F32)
    return fail(AF_ERR_UNSUPPORTED, "head_dim 256: the fp32 kernels take head dims 32, 64 and 128");
  if (k.mask < 0 || k.mask > 4 || (!allow_bs && k.mask == AF_MASK_BLOCK_SPARSE))
    return fail(AF_ERR_UNSUPPORTED, "mask kind %d not valid here", k.mask);
  if (k.bias < 0 || k.bias > 2) return fail(AF_ERR_UNSUPPORTED, "bias kind %d", k.bias);
  if (k.norm < 0 || k.norm > 1) return fail(AF_ERR_UNSUPPORTED, "norm kind %d", k.norm);
  if (k.rope != 0 && k.rope != 1) return fail(AF_ERR_UNSUPPORTED, "rope kind %d", k.rope);
  return AF_OK;
}

int check_fwd_common(const af_fwd_args* a) {
  if (a == nullptr) return fail(AF_ERR_BAD_ARG, "args is NULL");
  int rc;
  if ((rc = check_bhnd("q", a->q, a->q_stride, a->seqlen_q))) return rc;
  if ((rc = check_bhnd("k", a->k, a->k_stride, a->seqlen_kv))) return rc;
  if ((rc = check_bhnd("v", a->v, a->v_stride, a->seqlen_kv))) return rc;
  if ((rc = check_bhnd("o", a->o, a->o_stride, a->seqlen_q))) return rc;
  if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seqlen_q < 0 || a->seqlen_kv < 0)
    return fail(AF_ERR_BAD_ARG, "bad sizes B=%d Hq=%d Hkv=%d Nq=%d Nkv=%d", a->batch, a->heads_q,
                a->heads_kv, a->seqlen_q, a->seqlen_kv);
  if (a->heads_q % a->heads_kv != 0)
    return fail(AF_ERR_BAD_ARG, "query heads (%d) must be a multiple of key/value heads (%d)", a->heads_q,
                a->heads_kv);
  const af_spec_key& k = a->key;
  if ((k.mask == AF_MASK_CAUSAL || k.mask == AF_MASK_SLIDING_WINDOW ||
       k.mask == AF_MASK_CAUSAL_SLIDING_WINDOW) && a->seqlen_q != a->seqlen_kv)
    return fail(AF_ERR_BAD_ARG, "causal / sliding-window masks need seqlen_q == seqlen_kv (%d vs %d)",
                a->seqlen_q, a->seqlen_kv);
  if ((k.mask == AF_MASK_SLIDING_WINDOW || k.mask == AF_MASK_CAUSAL_SLIDING_WINDOW) && a->window <= 0)
    return fail(AF_ERR_BAD_ARG, "sliding window size must be positive");
  if (k.rope) {
    if (a->cos == nullptr || a->sin == nullptr) return fail(AF_ERR_BAD_ARG, "rope needs cos and sin tables");
    if (a->rope_stride[1] != 1 || a->rope_stride[0] % 8 != 0 || !aligned16(a->cos) || !aligned16(a->sin))
      return fail(AF_ERR_BAD_ARG, "rope tables need unit d-stride, 16-byte aligned rows");
    if (a->rope_len < std::max(a->seqlen_q, a->seqlen_kv))
      return fail(AF_ERR_BAD_ARG, "rope tables have %d rows, need %d", a->rope_len,
                  std::max(a->seqlen_q, a->seqlen_kv));
  }
  if (k.bias == AF_BIAS_ALIBI && a->alibi_slopes == nullptr) return fail(AF_ERR_BAD_ARG, "ALiBi needs slopes");
  if (k.bias == AF_BIAS_ADDITIVE) {
    if (a->bias == nullptr) return fail(AF_ERR_BAD_ARG, "additive bias pointer is NULL");
    if (a->bias_stride[3] != 1 || !aligned16(a->bias) || a->bias_stride[0] % 8 || a->bias_stride[1] % 8 ||
        a->bias_stride[2] % 8)
      return fail(AF_ERR_BAD_ARG, "additive bias needs unit key stride and 16-byte aligned rows");
  }
  return AF_OK;
}

FwdParams make_fwd_params(const af_fwd_args* a, int bm) {
  FwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->o);
  p.lse = a->lse;
  p.cos = static_cast<const uint16_t*>(a->cos);
  p.sin = static_cast<const uint16_t*>(a->sin);
  p.slopes = a->alibi_slopes;
  p.bias = static_cast<const uint16_t*>(a->bias);
  p.coverage = a->coverage;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = a->q_stride[i];
    p.ks[i] = a->k_stride[i];
    p.vs[i] = a->v_stride[i];
    p.os[i] = a->o_stride[i];
    p.bs[i] = a->bias_stride[i];
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
  p.n_mblocks = (a->seqlen_q + bm - 1) / bm;
  p.cov_nq = (a->seqlen_q + 31) / 32;
  p.cov_nk = (a->seqlen_kv + kKeysPerStage - 1) / kKeysPerStage;
  p.rope_len = a->rope_len;
  p.scale = a->scale;
  p.window = a->window;
  return p;
}

// The kernels address each (batch, head) slice of K, V and the RoPE tables
// through a raw buffer resource with a 32-bit byte range.
bool slice_fits_u32(int64_t rows, int64_t row_stride, int d) {
  return rows <= 0 || ((rows - 1) * row_stride + d) * 2 < (int64_t(1) << 32);
}

size_t fwd_workspace_bytes(const af_fwd_args& a) {
  if (!a.key.rope || a.batch <= 0 || a.heads_kv <= 0 || a.seqlen_kv <= 0 || a.key.head_dim <= 0) return 0;
  const size_t elem = a.key.dtype == AF_F32 ? 4 : 2;
  const size_t bytes = (size_t)a.batch * a.heads_kv * a.seqlen_kv * a.key.head_dim * elem;
  return (bytes + 255) & ~size_t(255);
}

// Workspace of a block-sparse forward: the rotated keys (RoPE), then with a
// Q-major work plan the fp32 partials of split rows, (slots, B*Hq, BLOCK_M)
// rows of D (unnormalised O) and of 2 (running max, row sum).  The fp32
// kernel walks whole rows and takes no partials.
struct BsFwdWorkspace {
  size_t part_o, part_ml, total;
};
BsFwdWorkspace bs_fwd_workspace(const af_fwd_args& a, const af_blockmask* bm) {
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  BsFwdWorkspace w{0, 0, fwd_workspace_bytes(a)};
  if (bm == nullptr || bm->q_items == nullptr || bm->n_q_slots <= 0 || a.key.dtype == AF_F32 || a.batch <= 0 ||
      a.heads_q <= 0 || a.key.head_dim <= 0 || bm->block_m <= 0)
    return w;
  const size_t rows = (size_t)bm->n_q_slots * a.batch * a.heads_q * bm->block_m;
  w.part_o = w.total;
  w.total += up(rows * a.key.head_dim * sizeof(float));
  w.part_ml = w.total;
  w.total += up(rows * 2 * sizeof(float));
  return w;
}

// With RoPE, rotate K once into the workspace and point the forward at k~.
int rotate_keys(FwdParams& p, const af_fwd_args& a, void* workspace, size_t workspace_bytes, hipStream_t s) {
  const size_t need = fwd_workspace_bytes(a);
  if (need == 0) return AF_OK;
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(AF_ERR_WORKSPACE, "forward with RoPE needs a %zu-byte workspace (16-byte aligned), got %zu", need,
                workspace_bytes);
  const int D = a.key.head_dim;
  RopeRowsParams r;
  r.x = static_cast<const uint16_t*>(a.k);
  r.out = static_cast<uint16_t*>(workspace);
  r.cos = static_cast<const uint16_t*>(a.cos);
  r.sin = static_cast<const uint16_t*>(a.sin);
  for (int i = 0; i < 3; ++i) r.xs[i] = a.k_stride[i];
  r.rs = a.rope_stride[0];
  r.rows = (int64_t)a.batch * a.heads_kv * a.seqlen_kv;
  r.H = a.heads_kv;
  r.N = a.seqlen_kv;
  const bool f16 = a.key.dtype == AF_F16;
  switch (D) {
    case 32: f16 ? launch_rope_f16_d32(r, s) : launch_rope_bf16_d32(r, s); break;
    case 64: f16 ? launch_rope_f16_d64(r, s) : launch_rope_bf16_d64(r, s); break;
    case 128: f16 ? launch_rope_f16_d128(r, s) : launch_rope_bf16_d128(r, s); break;
    case 256: f16 ? launch_rope_f16_d256(r, s) : launch_rope_bf16_d256(r, s); break;
  }
  p.k = r.out;
  p.ks[3] = 1;
  p.ks[2] = D;
  p.ks[1] = (int64_t)a.seqlen_kv * D;
  p.ks[0] = (int64_t)a.heads_kv * a.seqlen_kv * D;
  return AF_OK;
}

// Waves (32 query rows each) per forward workgroup for dense / causal /
// windowed masks.  Measured on MI355X at D = 64: 8-wave workgroups (one per
// CU) lose to two 4-wave workgroups per CU, whose barriers do not line up.
int fwd_waves(const af_spec_key&) { return 4; }

int dispatch_fwd(FwdParams p, const af_fwd_args& a, int waves, void* workspace, size_t workspace_bytes,
                 hipStream_t s) {
  const af_spec_key& k = a.key;
  if (!slice_fits_u32(p.Nkv, p.ks[2], k.head_dim) || !slice_fits_u32(p.Nkv, p.vs[2], k.head_dim))
    return fail(AF_ERR_UNSUPPORTED, "a (batch, head) slice of K or V spans 4 GiB or more");
  if (!(p.scale > 0.f) || p.scale == INFINITY)
    return fail(AF_ERR_BAD_ARG, "scale must be positive and finite (got %g)", (double)p.scale);
  int rc = rotate_keys(p, a, workspace, workspace_bytes, s);
  if (rc) return rc;
  const dim3 grid((unsigned)p.n_mblocks * (unsigned)(p.B * p.Hq));
  rc = -1;
  const bool f16 = k.dtype == AF_F16;
  // block-sparse walks with element masks run their own instantiations
  const int mask = k.mask == AF_MASK_BLOCK_SPARSE && p.bs_row_bits != nullptr ? MASK_BSE : k.mask;
  switch (k.head_dim) {
    case 32:
      rc = f16 ? launch_fwd_f16_d32(p, mask, k.bias, k.norm, k.rope, waves, grid, s)
               : launch_fwd_bf16_d32(p, mask, k.bias, k.norm, k.rope, waves, grid, s);
      break;
    case 64:
      rc = f16 ? launch_fwd_f16_d64(p, mask, k.bias, k.norm, k.rope, waves, grid, s)
               : launch_fwd_bf16_d64(p, mask, k.bias, k.norm, k.rope, waves, grid, s);
      break;
    case 128:
      rc = f16 ? launch_fwd_f16_d128(p, mask, k.bias, k.norm, k.rope, waves, grid, s)
               : launch_fwd_bf16_d128(p, mask, k.bias, k.norm, k.rope, waves, grid, s);
      break;
    case 256:
      rc = f16 ? launch_fwd_f16_d256(p, mask, k.bias, k.norm, k.rope, waves, grid, s)
               : launch_fwd_bf16_d256(p, mask, k.bias, k.norm, k.rope, waves, grid, s);
      break;
  }
  if (rc != 0) return fail(AF_ERR_UNSUPPORTED, "no forward instantiation for this key");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AF_ERR_LAUNCH, "forward launch failed: %s", hipGetErrorString(e));
  return AF_OK;
}

// fp32 forward: keys rotated once into the workspace with RoPE, then
// fwd_f32_kernel over 128-row query blocks.
int dispatch_fwd_f32(const af_fwd_args& a, void* workspace, size_t workspace_bytes, hipStream_t s,
                     const af_blockmask* bm = nullptr) {
  if (a.coverage != nullptr)
    return fail(AF_ERR_UNSUPPORTED, "tile-visit counters are kept by the fp16/bf16 kernels only");
  FwdF32Params fp;
  fp.f = make_fwd_params(&a, kF32BlockM);
  if (bm != nullptr) {
    FwdParams& q = fp.f;
    q.bs_block_m = bm->block_m;
    q.bs_block_n = bm->block_n;
    q.bs_full_num = bm->full_kv_num;
    q.bs_full_idx = bm->full_kv_idx;
    q.bs_part_num = bm->kv_num_blocks;
    q.bs_part_idx = bm->kv_indices;
    q.bs_full_rs = bm->full_kv_stride;
    q.bs_part_rs = bm->kv_stride;
    q.bs_row_bits = bm->part_row_bits;
  }
  fp.mask = a.key.mask;
  fp.bias = a.key.bias;
  fp.norm = a.key.norm;
  fp.rope = a.key.rope;
  FwdParams& p = fp.f;
  if (!(p.scale > 0.f) || p.scale == INFINITY)
    return fail(AF_ERR_BAD_ARG, "scale must be positive and finite (got %g)", (double)p.scale);
  const int D = a.key.head_dim;
  if (a.key.rope && a.seqlen_kv > 0) {
    const size_t need = fwd_workspace_bytes(a);
    if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
      return fail(AF_ERR_WORKSPACE, "forward with RoPE needs a %zu-byte workspace (16-byte aligned), got %zu", need,
                  workspace_bytes);
    const int64_t rows = (int64_t)a.batch * a.heads_kv * a.seqlen_kv;
    launch_rope_f32(static_cast<const float*>(a.k), static_cast<float*>(workspace), static_cast<const float*>(a.cos),
                    static_cast<const float*>(a.sin), a.k_stride, a.rope_stride[0], a.heads_kv, a.seqlen_kv, rows, D,
                    s);
    p.k = static_cast<const uint16_t*>(workspace);
    p.ks[2] = D;
    p.ks[1] = (int64_t)a.seqlen_kv * D;
    p.ks[0] = (int64_t)a.heads_kv * a.seqlen_kv * D;
  }
  const dim3 grid((unsigned)p.n_mblocks * (unsigned)(p.B * p.Hq));
  if (launch_fwd_f32(fp, D, grid, s) != 0) return fail(AF_ERR_UNSUPPORTED, "no fp32 forward for head_dim %d", D);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AF_ERR_LAUNCH, "fp32 forward launch failed: %s", hipGetErrorString(e));
  return AF_OK;
}

}  // namespace

// Validation and launch geometry of a decode call (af_decode and
// af_decode_noalloc): fills every field of *p except the workspace
// pointers and sets *need to the workspace bytes of the split count used.
// max_ws > 0 bounds the workspace: a library-chosen split count is lowered
// until the partials fit, and an explicit one that does not fit is refused.
int plan_decode(const af_decode_args* a, size_t max_ws, DecodeParams* out, size_t* need) {
  if (a == nullptr) return fail(AF_ERR_BAD_ARG, "args is NULL");
  int rc;
  if ((rc = check_bhnd("q", a->q, a->q_stride, 1))) return rc;
  if ((rc = check_bhnd("k", a->k, a->k_stride, a->seqlen_kv))) return rc;
  if ((rc = check_bhnd("v", a->v, a->v_stride, a->seqlen_kv))) return rc;
  if (a->o == nullptr) return fail(AF_ERR_BAD_ARG, "o is NULL");
  if (a->o_stride[3] != 1) return fail(AF_ERR_BAD_ARG, "o: head-dim stride must be 1");
  if ((rc = check_key(a->key, false, true))) return rc;
  if (a->key.mask != AF_MASK_FULL || a->key.rope != 0 || a->key.norm != AF_NORM_SOFTMAX ||
      (a->key.bias != AF_BIAS_NONE && a->key.bias != AF_BIAS_ALIBI))
    return fail(AF_ERR_UNSUPPORTED, "decode takes dense softmax with no bias or ALiBi, no RoPE");
  if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seqlen_kv <= 0 ||
      a->heads_q % a->heads_kv != 0)
    return fail(AF_ERR_BAD_ARG, "bad decode sizes B=%d Hq=%d Hkv=%d Nkv=%d", a->batch, a->heads_q, a->heads_kv,
                a->seqlen_kv);
  if (a->key.bias == AF_BIAS_ALIBI && a->alibi_slopes == nullptr) return fail(AF_ERR_BAD_ARG, "ALiBi needs slopes");
  const int D = a->key.head_dim;
  int S = a->num_splits > 0 ? a->num_splits
                            : af_decode_num_splits(a->batch, a->heads_q, a->heads_kv, a->seqlen_kv, D);
  // split length rounded up to 32 keys; empty trailing splits are dropped
  int split_len = 0;
  auto trim = [&]() {
    split_len = (a->seqlen_kv + S - 1) / S;
    split_len = (split_len + 31) & ~31;
    S = (a->seqlen_kv + split_len - 1) / split_len;
  };
  trim();
  // the limit applies to the splits that are launched, after the trim
  if (max_ws > 0) {
    const size_t per_split = af_decode_workspace_bytes(a->batch, a->heads_q, D, 1);
    const size_t fit = max_ws / per_split;
    if (fit == 0)
      return fail(AF_ERR_WORKSPACE, "decode partials of one split need %zu bytes, above the %zu-byte limit",
                  per_split, max_ws);
    if ((size_t)S > fit) {
      if (a->num_splits > 0)
        return fail(AF_ERR_WORKSPACE,
                    "%d splits (%d non-empty) need %zu bytes of partials, above the %zu-byte limit (at most %zu)",
                    a->num_splits, S, per_split * S, max_ws, fit);
      S = (int)fit;
      trim();                                       // only lowers S
    }
  }
  *need = af_decode_workspace_bytes(a->batch, a->heads_q, D, S);
  DecodeParams& p = *out;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->o);
  p.slopes = a->alibi_slopes;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = a->q_stride[i];
    p.ks[i] = a->k_stride[i];
    p.vs[i] = a->v_stride[i];
    p.os[i] = a->o_stride[i];
  }
  p.B = a->batch;
  p.Hq = a->heads_q;
  p.Hkv = a->heads_kv;
  p.Nkv = a->seqlen_kv;
  p.G = a->heads_q / a->heads_kv;
  // query heads sharing one workgroup's K/V reads: 16 (16-bit MFMA kernel)
  // or f32_decode_heads(D) (fp32 VALU kernel)
  const int gq = a->key.dtype == AF_F32 ? f32_decode_heads(D) : 16;
  p.nqc = (p.G + gq - 1) / gq;
  p.nsplit = S;
  p.split_len = split_len;
  p.scale = a->scale;
  return AF_OK;
}

// Split + combine of a planned decode call, with its partials at `workspace`.
int enqueue_decode(DecodeParams& p, const af_decode_args* a, void* workspace, hipStream_t s) {
  const size_t rows = (size_t)p.nsplit * p.B * p.Hq;
  p.ws_ml = static_cast<float*>(workspace);
  p.ws_acc = p.ws_ml + 2 * rows;
  const dim3 gs((unsigned)p.nsplit, (unsigned)(p.B * p.Hkv * p.nqc));
  const dim3 gc((unsigned)(p.B * p.Hq));
  if (launch_decode(p, a->key.dtype, a->key.head_dim, a->key.bias, gs, gc, s) != 0)
    return fail(AF_ERR_UNSUPPORTED, "no decode instantiation for this key");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AF_ERR_LAUNCH, "decode launch failed: %s", hipGetErrorString(e));
  return AF_OK;
}

}  // namespace af

using namespace af;

extern "C" {

const char* af_last_error(void) { return g_err; }

int af_abi_version(void) { return AF_ABI_VERSION; }

int af_query(const af_spec_key* key) {
  if (key == nullptr) return 0;
  return check_key(*key, true, true) == AF_OK ? 1 : 0;
}

int af_fwd_tile(const af_spec_key* key, int32_t* block_m, int32_t* block_n) {
  if (key == nullptr) return fail(AF_ERR_BAD_ARG, "key is NULL");
  int rc = check_key(*key, true, true);
  if (rc) return rc;
  if (key->dtype == AF_F32) {
    if (block_m) *block_m = kF32BlockM;
    if (block_n) *block_n = 32;
    return AF_OK;
  }
  if (block_m) *block_m = 32 * fwd_waves(*key);
  if (block_n) *block_n = kKeysPerStage;
  return AF_OK;
}

size_t af_fwd_workspace_bytes(const af_fwd_args* args) {
  return args == nullptr ? 0 : fwd_workspace_bytes(*args);
}

int af_fwd(const af_fwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_fwd_common(a);
  if (rc) return rc;
  if ((rc = check_key(a->key, false, true))) return rc;
  if (a->seqlen_q == 0) return AF_OK;
  if (a->key.dtype == AF_F32) return dispatch_fwd_f32(*a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  const int waves = fwd_waves(a->key);
  const FwdParams p = make_fwd_params(a, 32 * waves);
  return dispatch_fwd(p, *a, waves, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int af_fwd_blocksparse(const af_fwd_args* a, const af_blockmask* bm, void* workspace, size_t workspace_bytes,
                       void* stream) {
  int rc = check_fwd_common(a);
  if (rc) return rc;
  if ((rc = check_key(a->key, true, true))) return rc;
  if (a->key.mask != AF_MASK_BLOCK_SPARSE)
    return fail(AF_ERR_BAD_ARG, "af_fwd_blocksparse needs key.mask == AF_MASK_BLOCK_SPARSE");
  const bool f32 = a->key.dtype == AF_F32;
  if (bm == nullptr || bm->full_kv_num == nullptr || bm->full_kv_idx == nullptr ||
      bm->kv_num_blocks == nullptr || bm->kv_indices == nullptr)
    return fail(AF_ERR_BAD_ARG, "block mask lists are NULL");
  if (bm->full_kv_stride < 1 || bm->kv_stride < 1)
    return fail(AF_ERR_BAD_ARG, "block mask row strides must be at least 1");
  if (bm->block_m != 32 && bm->block_m != 64 && bm->block_m != 128)
    return fail(AF_ERR_UNSUPPORTED, "block-sparse BLOCK_M=%d: supported 32, 64, 128", bm->block_m);
  // key blocks are walked in 64-key stages (fp32: 32-key tiles)
  const int stage = f32 ? 32 : kKeysPerStage;
  if (bm->block_n <= 0 || bm->block_n % stage != 0)
    return fail(AF_ERR_UNSUPPORTED, "block-sparse BLOCK_N=%d: must be a multiple of %d", bm->block_n, stage);
  if (bm->n_q_blocks != (a->seqlen_q + bm->block_m - 1) / bm->block_m ||
      bm->n_kv_blocks != (a->seqlen_kv + bm->block_n - 1) / bm->block_n)
    return fail(AF_ERR_BAD_ARG, "block mask grid %dx%d does not match sequence lengths %d/%d", bm->n_q_blocks,
                bm->n_kv_blocks, a->seqlen_q, a->seqlen_kv);
  if ((rc = check_elem_masks(bm, a->key.head_dim))) return rc;
  if (a->seqlen_q == 0) return AF_OK;
  if (f32) {
    if (a->coverage != nullptr)
      return fail(AF_ERR_UNSUPPORTED, "tile-visit counters are kept by the fp16/bf16 kernels only");
    return dispatch_fwd_f32(*a, workspace, workspace_bytes, static_cast<hipStream_t>(stream), bm);
  }
  FwdParams p = make_fwd_params(a, bm->block_m);
  p.bs_block_m = bm->block_m;
  p.bs_full_num = bm->full_kv_num;
  p.bs_full_idx = bm->full_kv_idx;
  p.bs_part_num = bm->kv_num_blocks;
  p.bs_part_idx = bm->kv_indices;
  p.bs_full_rs = bm->full_kv_stride;
  p.bs_part_rs = bm->kv_stride;
  p.bs_block_n = bm->block_n;
  p.bs_row_bits = bm->part_row_bits;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const BsFwdWorkspace wl = bs_fwd_workspace(*a, bm);
  const bool split = bm->q_items != nullptr && bm->n_q_splits > 0;
  if (bm->q_items != nullptr) {
    if ((rc = check_plan(bm->n_q_items, bm->q_splits, bm->n_q_splits, bm->n_q_slots, bm->n_q_blocks, "q")))
      return rc;
    if (split && (workspace == nullptr || workspace_bytes < wl.total || !aligned16(workspace)))
      return fail(AF_ERR_WORKSPACE,
                  "block-sparse forward with split rows needs a %zu-byte workspace (16-byte aligned; "
                  "af_fwd_blocksparse_workspace_bytes), got %zu",
                  wl.total, workspace_bytes);
    p.bs_items = bm->q_items;
    p.n_mblocks = bm->n_q_items;  // grid rows: one per plan item
    if (split) {
      p.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.part_o);
      p.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.part_ml);
    }
  }
  // each listed key tile is re-read by every row that lists it: K and V of
  // a head
  p.bs_xcd_heads = bs_xcd_heads(a->batch * a->heads_q, 2 * (int64_t)a->seqlen_kv * a->key.head_dim * 2);
  if ((rc = dispatch_fwd(p, *a, bm->block_m / 32, workspace, workspace_bytes, s))) return rc;
  if (!split) return AF_OK;
  BsFwdCombineParams c;
  memset(&c, 0, sizeof(c));
  c.splits = bm->q_splits;
  c.part_o = p.part_o;
  c.part_ml = p.part_ml;
  c.o = static_cast<uint16_t*>(a->o);
  c.lse = a->lse;
  for (int i = 0; i < 4; ++i) c.os[i] = a->o_stride[i];
  for (int i = 0; i < 3; ++i) c.ls[i] = a->lse_stride[i];
  c.B = a->batch;
  c.H = a->heads_q;
  c.Nq = a->seqlen_q;
  c.BM = bm->block_m;
  c.softmax = a->key.norm == AF_NORM_SOFTMAX;
  if (launch_bs_fwd_combine(c, bm->n_q_splits, a->key.dtype, a->key.head_dim, s) != 0)
    return fail(AF_ERR_UNSUPPORTED, "no block-sparse combine for this key");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AF_ERR_LAUNCH, "block-sparse combine launch failed: %s", hipGetErrorString(e));
  return AF_OK;
}

size_t af_fwd_blocksparse_workspace_bytes(const af_fwd_args* a, const af_blockmask* bm) {
  return a == nullptr ? 0 : bs_fwd_workspace(*a, bm).total;
}

int32_t af_decode_num_splits(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seqlen_kv,
                             int32_t head_dim) {
  (void)head_dim;
  if (batch <= 0 || heads_q <= 0 || heads_kv <= 0 || seqlen_kv <= 0) return 1;
  const int g = heads_q / heads_kv;
  const int64_t groups = (int64_t)batch * heads_kv * ((g + 15) / 16);
  // ~512 workgroups: the split kernel keeps two steps of K/V per wave in
  // flight in 254 VGPRs, so two 4-wave workgroups fit a CU (256 CUs); at
  // least 256 keys per split.  Measured at config 3: 8 splits (512
  // workgroups) 180.6 us, 16 splits 186.0 us, 12 splits 183.0 us.
  int64_t s = (512 + groups - 1) / groups;
  s = std::min<int64_t>(s, std::max<int64_t>(1, seqlen_kv / 256));
  s = std::max<int64_t>(1, std::min<int64_t>(s, 256));
  return (int32_t)s;
}

size_t af_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t head_dim, int32_t num_splits) {
  if (batch <= 0 || heads_q <= 0 || head_dim <= 0 || num_splits <= 0) return 0;
  return (size_t)num_splits * batch * heads_q * (2 + head_dim) * sizeof(float);
}

int af_decode(const af_decode_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  DecodeParams p;
  size_t need = 0;
  int rc = plan_decode(a, 0, &p, &need);
  if (rc) return rc;
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(AF_ERR_WORKSPACE, "decode workspace needs %zu bytes (16-byte aligned), got %zu", need,
                workspace_bytes);
  return enqueue_decode(p, a, workspace, static_cast<hipStream_t>(stream));
}

size_t af_bwd_workspace_bytes(const af_bwd_args* args) {
  // a block-sparse launch sizes its workspace with its mask
  if (args == nullptr || args->key.mask == AF_MASK_BLOCK_SPARSE) return 0;
  return bwd_workspace_bytes(*args);
}

size_t af_bwd_blocksparse_workspace_bytes(const af_bwd_args* args, const af_blockmask* bm) {
  if (args == nullptr) return 0;
  return bwd_workspace_bytes(*args, args->key.mask == AF_MASK_BLOCK_SPARSE ? bm : nullptr);
}

int af_bwd(const af_bwd_args* a, const af_blockmask* bm, void* workspace, size_t workspace_bytes,
           void* stream) {
  return run_bwd(a, bm, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int af_bwd_tile(const af_bwd_args* a, const af_blockmask* bm, int32_t* block_m, int32_t* block_n,
                int32_t* group_split) {
  if (a == nullptr) return fail(AF_ERR_BAD_ARG, "args is NULL");
  if (!group_split_valid(*a))
    return fail(AF_ERR_BAD_ARG, "group_split must be 0 or a power of two dividing heads_q / heads_kv");
  // dQ: 4 waves x 32 query rows; dK/dV: 4 waves x 32 keys (the fp32
  // kernels: kBwdF32Block of each); block-sparse launches follow the mask's
  // blocks
  int bm_rows = 128, bn_keys = 128;
  if (a->key.dtype == AF_F32) bm_rows = bn_keys = kBwdF32Block;
  if (a->key.mask == AF_MASK_BLOCK_SPARSE && bm != nullptr) {
    bm_rows = bm->block_m;
    bn_keys = bm->block_n;
  }
  if (block_m) *block_m = bm_rows;
  if (block_n) *block_n = bn_keys;
  if (group_split)
    *group_split = bwd_group_split_for(*a, a->key.mask == AF_MASK_BLOCK_SPARSE ? bm : nullptr);
  return AF_OK;
}

}  // extern "C"
