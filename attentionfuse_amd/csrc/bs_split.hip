// Block-sparse work plans (af_blockmask_plan) and the combine launches for
// split rows / columns.
#include <algorithm>
#include <vector>

#include "attnfuse_hip.h"
#include "bs_split.hpp"
#include "validate.hpp"

namespace af {

namespace {

template <class E, int D>
void fwd_combine(const BsFwdCombineParams& p, int n_splits, hipStream_t s) {
  constexpr int RPB = 256 / (D / 8);
  const unsigned per = (unsigned)((p.BM + RPB - 1) / RPB);
  const dim3 grid((unsigned)n_splits * (unsigned)(p.B * p.H) * per);
  hipLaunchKernelGGL((bs_fwd_combine_kernel<E, D>), grid, dim3(256), 0, s, p);
}

template <class E, int D>
void grad_combine(BsGradCombineParams& p, hipStream_t s) {
  constexpr int RPB = 256 / (D / 16);
  unsigned wgs = 0;
  for (int i = 0; i < p.n_targets; ++i) {
    BsGradTarget& t = p.t[i];
    t.wg0 = (int32_t)wgs;
    wgs += (unsigned)t.n_splits * (unsigned)(p.B * t.H) * (unsigned)((t.BLK + RPB - 1) / RPB);
  }
  if (wgs > 0) hipLaunchKernelGGL((bs_grad_combine_kernel<E, D>), dim3(wgs), dim3(256), 0, s, p);
}

template <class E>
int fwd_combine_d(const BsFwdCombineParams& p, int n_splits, int d, hipStream_t s) {
  switch (d) {
    case 32: fwd_combine<E, 32>(p, n_splits, s); return 0;
    case 64: fwd_combine<E, 64>(p, n_splits, s); return 0;
    case 128: fwd_combine<E, 128>(p, n_splits, s); return 0;
    case 256: fwd_combine<E, 256>(p, n_splits, s); return 0;
  }
  return -1;
}

template <class E>
int grad_combine_d(BsGradCombineParams& p, int d, hipStream_t s) {
  switch (d) {
    case 32: grad_combine<E, 32>(p, s); return 0;
    case 64: grad_combine<E, 64>(p, s); return 0;
    case 128: grad_combine<E, 128>(p, s); return 0;
    case 256: grad_combine<E, 256>(p, s); return 0;
  }
  return -1;
}

}  // namespace

int launch_bs_fwd_combine(const BsFwdCombineParams& p, int n_splits, int dtype, int head_dim, hipStream_t s) {
  if (n_splits <= 0) return 0;
  if (dtype == 0) return fwd_combine_d<F16>(p, n_splits, head_dim, s);
  if (dtype == 1) return fwd_combine_d<BF16>(p, n_splits, head_dim, s);
  return -1;
}

int launch_bs_grad_combine(BsGradCombineParams& p, int dtype, int head_dim, hipStream_t s) {
  if (p.n_targets <= 0) return 0;
  if (dtype == 0) return grad_combine_d<F16>(p, head_dim, s);
  if (dtype == 1) return grad_combine_d<BF16>(p, head_dim, s);
  return -1;
}

}  // namespace af

using namespace af;

extern "C" int af_blockmask_plan(const int32_t* counts, int32_t n, int32_t chunk, int32_t* items, int32_t* splits,
                                 int32_t* sizes) {
  if (sizes == nullptr) {
    set_error("sizes is NULL");
    return AF_ERR_BAD_ARG;
  }
  if (n < 0 || (n > 0 && counts == nullptr)) {
    set_error("bad list count %d or NULL counts", n);
    return AF_ERR_BAD_ARG;
  }
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    if (counts[i] < 0) {
      set_error("list %d has a negative count (%d)", i, counts[i]);
      return AF_ERR_BAD_ARG;
    }
    total += counts[i];
  }
  // default piece length: twice the mean list length, at least 8 entries.
  // Measured at config 4 (BigBird, mean 7.7 entries) fwd / bwd: pieces of 8
  // 69 / 165 us, 16 59 / 149 us, 24 60 / 150 us, unsplit 93 / 255 us; each
  // piece pays its Q (or K/V) rows, its first tiles' latency and partial
  // traffic, so pieces near the mean cost more than the tail they remove.
  if (chunk <= 0) chunk = (int32_t)std::max<int64_t>(8, n > 0 ? 2 * ((total + n - 1) / n) : 8);
  struct Item {
    int32_t list, e0, ne, slot;
  };
  std::vector<Item> it;
  std::vector<int32_t> sp;
  it.reserve(n);
  int32_t slots = 0;
  for (int i = 0; i < n; ++i) {
    const int c = counts[i];
    const int pieces = c <= chunk ? 1 : (c + chunk - 1) / chunk;
    if (pieces == 1) {
      // every list keeps a workgroup, empty ones too: it writes O = 0 (or
      // zero gradients) for its rows
      it.push_back({i, 0, c, -1});
      continue;
    }
    sp.insert(sp.end(), {i, slots, pieces});
    for (int k = 0; k < pieces; ++k) {
      const int e0 = (int)((int64_t)k * c / pieces), e1 = (int)((int64_t)(k + 1) * c / pieces);
      it.push_back({i, e0, e1 - e0, slots + k});
    }
    slots += pieces;
  }
  // longest pieces first: they start while the short ones fill the tail
  std::stable_sort(it.begin(), it.end(), [](const Item& a, const Item& b) { return a.ne > b.ne; });
  sizes[0] = (int32_t)it.size();
  sizes[1] = (int32_t)(sp.size() / 3);
  sizes[2] = slots;
  if (items != nullptr)
    for (size_t k = 0; k < it.size(); ++k) {
      items[4 * k] = it[k].list;
      items[4 * k + 1] = it[k].e0;
      items[4 * k + 2] = it[k].ne;
      items[4 * k + 3] = it[k].slot;
    }
  if (splits != nullptr) std::copy(sp.begin(), sp.end(), splits);
  return AF_OK;
}
