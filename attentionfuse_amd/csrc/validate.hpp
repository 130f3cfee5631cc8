// Argument checks shared by the forward, decode and backward entry points.
#pragma once

#include <stdint.h>

#include "attnfuse_hip.h"

namespace af {

void set_error(const char* fmt, ...);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A block-mask work plan as af_blockmask_plan writes it: at least one item
// per list, and every split (two or more slots) listed.
inline int check_plan(int n_items, const int32_t* splits, int n_splits, int n_slots, int n_lists,
                      const char* which) {
  if (n_items < n_lists || n_splits < 0 || n_slots < 2 * n_splits || (n_splits > 0 && splits == nullptr)) {
    set_error("block mask %s work plan is inconsistent (%d items for %d lists, %d splits, %d slots)", which,
              n_items, n_lists, n_splits, n_slots);
    return AF_ERR_BAD_ARG;
  }
  return AF_OK;
}

// (B, H, N, D) tensor with unit D-stride and 16-byte aligned rows.  A
// tensor with no rows (N == 0) is never read or written and may be NULL.
inline int check_bhnd(const char* name, const void* ptr, const int64_t* st, int64_t rows) {
  if (rows == 0) return AF_OK;
  if (ptr == nullptr) {
    set_error("%s is NULL", name);
    return AF_ERR_BAD_ARG;
  }
  if (st[3] != 1) {
    set_error("%s: head-dim stride must be 1 (got %lld)", name, (long long)st[3]);
    return AF_ERR_BAD_ARG;
  }
  if (!aligned16(ptr)) {
    set_error("%s: base pointer must be 16-byte aligned", name);
    return AF_ERR_BAD_ARG;
  }
  for (int i = 0; i < 3; ++i)
    if (st[i] % 8 != 0) {
      set_error("%s: stride[%d]=%lld is not a multiple of 8 elements", name, i, (long long)st[i]);
      return AF_ERR_BAD_ARG;
    }
  return AF_OK;
}

// Element masks of a block mask: all three arrays or none, over key blocks of
// whole 64-bit words, head dims up to 128.
inline int check_elem_masks(const af_blockmask* bm, int head_dim) {
  const int n = (bm->part_row_bits != nullptr) + (bm->q_col_bits != nullptr) + (bm->q_partial != nullptr);
  if (n != 0 && n != 3) {
    set_error("block mask element masks: part_row_bits, q_col_bits and q_partial must be all NULL or all set");
    return AF_ERR_BAD_ARG;
  }
  if (n == 3 && head_dim > 128) {
    set_error("block mask element masks: head dims up to 128 (got %d)", head_dim);
    return AF_ERR_UNSUPPORTED;
  }
  if (n == 3 && bm->block_n % 64 != 0) {
    set_error("block mask element masks need BLOCK_N a multiple of 64 (got %d)", bm->block_n);
    return AF_ERR_UNSUPPORTED;
  }
  return AF_OK;
}

inline bool head_dim_supported(int d) { return d == 32 || d == 64 || d == 128 || d == 256; }

}  // namespace af
