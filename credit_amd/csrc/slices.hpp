// Row slices shared by the single-tensor-staged split kernels (softmax,
// rowwise quantisation): which rows and which slice of them a workgroup
// covers, the STAGED / SPLIT / READ plan for a row width, and the launch of
// a slice kernel as one plain grid (members == 1) or one co-resident wave of
// ticketed groups looping over their rows.
#pragma once

#include <initializer_list>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace slices {

struct Slice {
  int row, step, member, v0, vlen;
};

// Rows and slice of this workgroup.  members == 1: the grid has one
// workgroup per row (row = blockIdx.x, one pass).  members > 1: a
// co-resident grid of G groups; the ticketed member covers the same slice of
// rows group, group + G, group + 2G, ... (padding groups have group >= rows
// and do no pass).
__device__ __forceinline__ Slice slice_of(SplitGroup* g, int members, int k_values, int chunk,
                                          int nvec, const SplitArgs& sa) {
  Slice s{static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), 0, 0, 0};
  if (members > 1) {
    *g = split_join(sa, members, k_values);
    s.row = g->group;
    s.step = static_cast<int>(sa.grid) / members;
    s.member = g->member;
  }
  s.v0 = s.member * chunk;
  s.vlen = nvec - s.v0 < chunk ? nvec - s.v0 : chunk;
  return s;
}

// Buffer resource over this member's slice of a row of f32x4 vectors:
// loads beyond it return zeros and stores beyond it are dropped, so slice
// kernels need no per-lane bounds branch around their row traffic.
__device__ __forceinline__ buffer_rsrc_t slice_rsrc(const float* row, const Slice& s) {
  return make_rsrc(row + 4 * static_cast<size_t>(s.v0), static_cast<uint32_t>(s.vlen) * 16u);
}
__device__ __forceinline__ f32x4 slice_load(buffer_rsrc_t r, uint32_t offset) {
  return __builtin_bit_cast(f32x4, buffer_load_nt(r, offset));
}
__device__ __forceinline__ void slice_store(buffer_rsrc_t r, uint32_t offset, f32x4 v) {
  buffer_store_nt(r, offset, __builtin_bit_cast(u32x4, v));
}

template <class Fn>
struct Pick {
  Fn fn;
  int threads;
  int capacity;  // f32x4 per workgroup
};

template <class P, int N>
const P* pick_for(const P (&table)[N], int64_t chunk) {
  for (const P& p : table)
    if (chunk <= p.capacity) return &p;
  return nullptr;
}

inline bool vec_ok(int64_t cols, std::initializer_list<const void*> ptrs) {
  if (cols % 4 != 0) return false;
  for (const void* q : ptrs)
    if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return false;
  return true;
}

struct Plan {
  int variant;
  int members;
  int64_t chunk;
};

// Variant resolution shared by the slice operations; `capacity` is the
// widest slice (f32x4) one workgroup holds.  AUTO on a row wider than that
// splits it into slices of at most `auto_capacity` (default: capacity):
// smaller slices run on smaller workgroups, two of which share a CU.
inline int resolve(const credit_cfg* cfg, int64_t cols, bool vec, int64_t capacity, const char* op,
                   Plan* plan, int64_t auto_capacity = 0) {
  const int variant = cfg_variant(cfg);
  const int64_t nvec = cols / 4;
  if (variant == CREDIT_VARIANT_READ || (!vec && variant == CREDIT_VARIANT_AUTO)) {
    *plan = Plan{CREDIT_VARIANT_READ, 1, nvec};
    return CREDIT_OK;
  }
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "%s staged/split variants need cols %% 4 == 0 and 16-byte aligned buffers",
                     op);
  const int need = static_cast<int>((nvec + capacity - 1) / capacity);
  int p;
  if (variant == CREDIT_VARIANT_STAGED) {
    if (need > 1)
      return set_error(CREDIT_ERR_UNSUPPORTED, "%s staged variant holds at most %lld columns",
                       op, static_cast<long long>(capacity * 4));
    p = 1;
  } else if (variant == CREDIT_VARIANT_AUTO) {
    const int64_t cap = auto_capacity > 0 && need > 1 ? auto_capacity : capacity;
    p = static_cast<int>((nvec + cap - 1) / cap);
  } else {
    p = cfg_split(cfg);
    if (p == 0) p = need < 2 ? 2 : need;
    if (p < need)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "%s split %d leaves more than %lld columns per member", op, p,
                       static_cast<long long>(capacity * 4));
  }
  if (p > nvec) p = static_cast<int>(nvec);
  int64_t chunk = (nvec + p - 1) / p;
  int members = static_cast<int>((nvec + chunk - 1) / chunk);
  *plan = Plan{members > 1 ? CREDIT_VARIANT_SPLIT : CREDIT_VARIANT_STAGED, members, chunk};
  return CREDIT_OK;
}

// Launch a slice kernel over all rows: a plain grid of one workgroup per
// row (members == 1), or one co-resident wave of ticketed groups, each
// looping over its rows (`stages` exchanges per row).
template <class Fn, class Launch>
int launch_slices(const credit_cfg* cfg, int64_t rows, const Plan& plan, const Pick<Fn>* pk,
                  int k_values, int stages, const char* name, Launch&& launch) {
  if (plan.members == 1) {
    launch(static_cast<unsigned>(rows), SplitArgs{});
    return check_launch(name);
  }
  int64_t groups = 0;
  int dispensers = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(pk->fn), pk->threads, 0,
                               plan.members, &groups, &dispensers));
  if (groups == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED, "%s: %d groups of %d members do not fit the device",
                     name, kDispensers, plan.members);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  const int64_t per_group = (rows + groups - 1) / groups;
  if (per_group * stages > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_SHAPE, "%s: %lld rows per group exceed the exchange tags of "
                     "one launch", name, static_cast<long long>(per_group));
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, k_values, kSplitRing, 0, &ws));
  const uint32_t total = static_cast<uint32_t>(groups * plan.members);
  launch(total, make_split_args(ws, total, static_cast<uint32_t>(per_group * stages), kSplitRing,
                                dispensers));
  return check_launch(name);
}

inline size_t slice_workspace(int64_t rows, const Plan& p, int k_values, int cu_count) {
  if (p.members <= 1) return 0;
  int64_t groups = coresident_groups_bound(p.members, cu_count);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  return split_workspace_bytes(groups, p.members, k_values, kSplitRing, 0);
}

}  // namespace slices
}  // namespace credit
