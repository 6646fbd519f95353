// LayerNorm backward: the reference's own wide-row workload
// (dsmem_eval/workloads.py:53-61; kernels src/workloads/layernorm_backward.cu:
// 274-438), in fp32 and bf16.
//
//   mean = sum(x)/N,  var = sum((x - mean)^2)/N,  rstd = 1/sqrt(var + eps)
//   xhat = (x - mean) * rstd,  g = dy * gamma
//   dx   = (g - mean(g) - xhat * mean(g * xhat)) * rstd
//
// The statistics follow the two-pass definition of workloads.py:54-56 (the
// CUDA file's one-pass E[x^2] - mean^2, layernorm_backward.cu:293-294, is not
// inherited): they are accumulated as sum(x - x0) and sum((x - x0)^2) about
// the row's first element x0, in fp64 across lanes, waves and members, which
// has the cancellation behaviour of a two-pass variance in one pass.
// Two reduction stages per row, as the reference's cluster kernel (:376-438):
// stage 1 (sum(x - x0), sum((x - x0)^2)), stage 2 (sum g, sum g*xhat).
// Variants: STAGED / SPLIT hold x and dy in VGPRs (one HBM read of each),
// READ streams the row three times (stats; the two sums; the output), the
// counterpart of block_bwd_read_kernel (:274-321).
#include <initializer_list>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

// 16-byte vectors of fp32 (4 lanes) or bf16 (8 lanes).
template <class T>
struct Vec;
template <>
struct Vec<float> {
  using raw = f32x4;
  static constexpr int kN = 4;
  __device__ static float get(const raw& v, int i) { return v[i]; }
  __device__ static raw pack(const float (&a)[4]) { return raw{a[0], a[1], a[2], a[3]}; }
  __device__ static float scalar(const float* p) { return *p; }
  __device__ static void store_scalar(float* p, float v) { *p = v; }
};
template <>
struct Vec<uint16_t> {
  using raw = u32x4;
  static constexpr int kN = 8;
  __device__ static float get(const raw& v, int i) {
    return (i & 1) ? bf16_hi(v[i >> 1]) : bf16_lo(v[i >> 1]);
  }
  __device__ static raw pack(const float (&a)[8]) {
    return raw{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]),
               pack_bf16x2(a[6], a[7])};
  }
  __device__ static float scalar(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ static void store_scalar(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

// An empty asm that "redefines" each vector: values computed from the
// vectors before it cannot be reused after it.
template <int N, class R>
__device__ __forceinline__ void opaque_regs(R (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) __asm__ volatile("" : "+v"(v[k]));
}

struct RowStats {
  float mean, rstd;
};

__device__ __forceinline__ RowStats stats_from(double s1, double s2, float x0, int cols,
                                               float eps) {
  const double d = s1 / cols;
  const double var = s2 / cols - d * d;
  RowStats r;
  r.mean = static_cast<float>(static_cast<double>(x0) + d);
  r.rstd = static_cast<float>(1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps));
  return r;
}

template <class T, int THREADS, int VPT>
__device__ __forceinline__ void layernorm_bwd_slice_kernel_body(
    const T* __restrict__ x, const T* __restrict__ dy, const T* __restrict__ gamma,
    T* __restrict__ dx, int cols, int chunk, int members, int rows, float eps, SplitArgs sa) {
  using V = Vec<T>;
  using raw = typename V::raw;
  constexpr int NW = THREADS / kWave;
  constexpr int E = V::kN;
  // One slot array per stage: no workgroup reuses a stage's slots before
  // the barrier of the other stage (or of the exchanges) has passed.
  __shared__ double red1[2][NW];
  __shared__ double red2[2][NW];
  SplitGroup g;
  // members == 1: one workgroup per row.  members > 1: a co-resident grid
  // of G groups; the member covers its slice of rows group, group + G, ...
  int row0 = blockIdx.x, step = gridDim.x, member = 0;
  if (members > 1) {
    g = split_join(sa, members, 2);
    row0 = g.group;
    step = static_cast<int>(sa.grid) / members;
    member = g.member;
  }
  const int nvec = cols / E;
  const int v0 = member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  // Row traffic through buffer resources over the member's slice: lanes
  // beyond it read zeros and drop their stores, with no branch around a
  // load or store.
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  const buffer_rsrc_t grs = make_rsrc(gamma + static_cast<size_t>(E) * v0, slice_bytes);
  for (int row = row0; row < rows; row += step) {
    const size_t off = static_cast<size_t>(row) * cols + static_cast<size_t>(E) * v0;
    const buffer_rsrc_t xrs = make_rsrc(x + off, slice_bytes);
    const buffer_rsrc_t drs = make_rsrc(dy + off, slice_bytes);
    raw xv[VPT], dv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = __builtin_bit_cast(raw, buffer_load_nt(xrs, lane_off + k * kStride));
      dv[k] = __builtin_bit_cast(raw, buffer_load_nt(drs, lane_off + k * kStride));
    }
    const float x0 = V::scalar(x + static_cast<size_t>(row) * cols);
    float a1 = 0.0f, a2 = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      // Beyond the slice x reads 0: its shifted value -x0 must add nothing.
      float p1 = 0.0f, p2 = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float d = V::get(xv[k], e) - x0;
        p1 += d;
        p2 += d * d;
      }
      const bool in = lane_off + k * kStride < slice_bytes;
      a1 += in ? p1 : 0.0f;
      a2 += in ? p2 : 0.0f;
    }
    double s[2] = {a1, a2};
    block_reduce_sum_f64_multi<NW, 2>(s, red1);
    if (members > 1) {
      if (threadIdx.x == 0) {
        split_publish(g, 0, s[0]);
        split_publish(g, 1, s[1]);
      }
      split_exchange(g);
      s[0] = split_sum(g, 0);
      s[1] = split_sum(g, 1);
    }
    const RowStats st = stats_from(s[0], s[1], x0, cols, eps);
    // The loaded vectors stay packed in registers between the passes: each
    // pass unpacks them again (cheap) rather than keeping unpacked copies
    // alive (twice the registers for bf16).
    opaque_regs<VPT>(xv);
    opaque_regs<VPT>(dv);
    // Beyond the slice dy reads 0, so g = dy * gamma adds nothing.
    float b1 = 0.0f, b2 = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const raw gv = __builtin_bit_cast(raw, buffer_load(grs, lane_off + k * kStride));
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float gg = V::get(dv[k], e) * V::get(gv, e);
        b1 += gg;
        b2 += gg * ((V::get(xv[k], e) - st.mean) * st.rstd);
      }
    }
    double t[2] = {b1, b2};
    block_reduce_sum_f64_multi<NW, 2>(t, red2);
    if (members > 1) {
      if (threadIdx.x == 0) {
        split_publish(g, 0, t[0]);
        split_publish(g, 1, t[1]);
      }
      split_exchange(g);
      t[0] = split_sum(g, 0);
      t[1] = split_sum(g, 1);
    }
    const float mg = static_cast<float>(t[0] / cols);
    const float mgx = static_cast<float>(t[1] / cols);
    opaque_regs<VPT>(xv);
    opaque_regs<VPT>(dv);
    const buffer_rsrc_t ors = make_rsrc(dx + off, slice_bytes);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const raw gv = __builtin_bit_cast(raw, buffer_load(grs, lane_off + k * kStride));
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float xh = (V::get(xv[k], e) - st.mean) * st.rstd;
        o[e] = (V::get(dv[k], e) * V::get(gv, e) - mg - xh * mgx) * st.rstd;
      }
      buffer_store_nt(ors, lane_off + k * kStride, __builtin_bit_cast(u32x4, V::pack(o)));
    }
  }
}

template <class T, int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void layernorm_bwd_slice_kernel(
    const T* __restrict__ x, const T* __restrict__ dy, const T* __restrict__ gamma,
    T* __restrict__ dx, int cols, int chunk, int members, int rows, float eps, SplitArgs sa) {
  layernorm_bwd_slice_kernel_body<T, THREADS, VPT>(x, dy, gamma, dx, cols, chunk, members, rows, eps, sa);
  split_leave(sa);
}

// Three streaming passes over the row (any width and alignment).
template <class T, int THREADS>
__global__ __launch_bounds__(THREADS) void layernorm_bwd_read_kernel(
    const T* __restrict__ x, const T* __restrict__ dy, const T* __restrict__ gamma,
    T* __restrict__ dx, int cols, float eps) {
  using V = Vec<T>;
  constexpr int NW = THREADS / kWave;
  __shared__ double red[4][NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  const T* xr = x + off;
  const T* dr = dy + off;
  const float x0 = V::scalar(xr);
  double a1 = 0.0, a2 = 0.0;
  for (int c = tid; c < cols; c += THREADS) {
    const double d = static_cast<double>(V::scalar(xr + c) - x0);
    a1 += d;
    a2 += d * d;
  }
  const double s1 = block_reduce_sum_f64<NW>(a1, red[0]);
  const double s2 = block_reduce_sum_f64<NW>(a2, red[1]);
  const RowStats st = stats_from(s1, s2, x0, cols, eps);
  double b1 = 0.0, b2 = 0.0;
  for (int c = tid; c < cols; c += THREADS) {
    const float gg = V::scalar(dr + c) * V::scalar(gamma + c);
    b1 += gg;
    b2 += gg * ((V::scalar(xr + c) - st.mean) * st.rstd);
  }
  const float mg = static_cast<float>(block_reduce_sum_f64<NW>(b1, red[2]) / cols);
  const float mgx = static_cast<float>(block_reduce_sum_f64<NW>(b2, red[3]) / cols);
  for (int c = tid; c < cols; c += THREADS) {
    const float xh = (V::scalar(xr + c) - st.mean) * st.rstd;
    V::store_scalar(dx + off + c,
                    (V::scalar(dr + c) * V::scalar(gamma + c) - mg - xh * mgx) * st.rstd);
  }
}

template <class T>
using SliceFn = void (*)(const T*, const T*, const T*, T*, int, int, int, int, float,
                         SplitArgs);

template <class T>
struct Pick {
  SliceFn<T> fn;
  int threads;
  int capacity;  // vectors per workgroup
};

// x and dy staged: up to 8 vectors of each per lane.  bf16 unpacks to twice
// the floats per vector, so its 1024-lane slice stops at 4 per lane (8
// would spill).
template <class T>
struct Slices;
template <>
struct Slices<float> {
  static constexpr Pick<float> table[] = {
      {layernorm_bwd_slice_kernel<float, 64, 4>, 64, 256},
      {layernorm_bwd_slice_kernel<float, 128, 4>, 128, 512},
      {layernorm_bwd_slice_kernel<float, 256, 4>, 256, 1024},
      {layernorm_bwd_slice_kernel<float, 256, 8>, 256, 2048},
      {layernorm_bwd_slice_kernel<float, 512, 8>, 512, 4096},
      {layernorm_bwd_slice_kernel<float, 1024, 8>, 1024, 8192},
  };
  static constexpr int64_t capacity = 8192;
};
template <>
struct Slices<uint16_t> {
  static constexpr Pick<uint16_t> table[] = {
      {layernorm_bwd_slice_kernel<uint16_t, 64, 4>, 64, 256},
      {layernorm_bwd_slice_kernel<uint16_t, 128, 4>, 128, 512},
      {layernorm_bwd_slice_kernel<uint16_t, 256, 4>, 256, 1024},
      {layernorm_bwd_slice_kernel<uint16_t, 256, 8>, 256, 2048},
      {layernorm_bwd_slice_kernel<uint16_t, 512, 8>, 512, 4096},
      {layernorm_bwd_slice_kernel<uint16_t, 1024, 4>, 1024, 4096},
  };
  static constexpr int64_t capacity = 4096;
};

template <class T>
const Pick<T>* pick_for(int64_t chunk) {
  for (const Pick<T>& p : Slices<T>::table)
    if (chunk <= p.capacity) return &p;
  return nullptr;
}

struct Plan {
  int variant;
  int members;
  int64_t chunk;
};

int resolve(const credit_cfg* cfg, int64_t nvec, bool vec, int64_t kCapacity, Plan* plan) {
  const int variant = cfg_variant(cfg);
  if (variant == CREDIT_VARIANT_READ || (!vec && variant == CREDIT_VARIANT_AUTO)) {
    *plan = Plan{CREDIT_VARIANT_READ, 1, nvec};
    return CREDIT_OK;
  }
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_bwd staged/split variants need 16-byte rows and buffers");
  const int need = static_cast<int>((nvec + kCapacity - 1) / kCapacity);
  int p;
  if (variant == CREDIT_VARIANT_STAGED) {
    if (need > 1)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "layernorm_bwd staged variant holds at most %lld vectors per row",
                       static_cast<long long>(kCapacity));
    p = 1;
  } else if (variant == CREDIT_VARIANT_AUTO) {
    p = need;
  } else {
    p = cfg_split(cfg);
    if (p == 0) p = need < 2 ? 2 : need;
    if (p < need)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "layernorm_bwd split %d leaves more than %lld vectors per member", p,
                       static_cast<long long>(kCapacity));
  }
  if (p > nvec) p = static_cast<int>(nvec);
  const int64_t chunk = (nvec + p - 1) / p;
  const int members = static_cast<int>((nvec + chunk - 1) / chunk);
  *plan = Plan{members > 1 ? CREDIT_VARIANT_SPLIT : CREDIT_VARIANT_STAGED, members, chunk};
  return CREDIT_OK;
}

template <class T>
int layernorm_bwd(const T* x, const T* dy, const T* gamma, T* dx, int64_t rows, int64_t cols,
                  float eps, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_ptr(gamma, "gamma"));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, sizeof(T), "x"));
  CREDIT_TRY(check_aligned(dy, sizeof(T), "dy"));
  CREDIT_TRY(check_aligned(gamma, sizeof(T), "gamma"));
  CREDIT_TRY(check_aligned(dx, sizeof(T), "dx"));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (rows == 0) return CREDIT_OK;
  constexpr int E = Vec<T>::kN;
  bool vec = cols % E == 0;
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(dy),
                        static_cast<const void*>(gamma), static_cast<const void*>(dx)})
    vec = vec && reinterpret_cast<uintptr_t>(p) % 16 == 0;
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols / E, vec, Slices<T>::capacity, &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  if (plan.variant == CREDIT_VARIANT_READ) {
    layernorm_bwd_read_kernel<T, 256>
        <<<dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream>>>(x, dy, gamma, dx, c, eps);
    return check_launch("layernorm_bwd_read_kernel");
  }
  const Pick<T>* pk = pick_for<T>(plan.chunk);
  if (plan.members == 1) {
    hipLaunchKernelGGL(pk->fn, dim3(static_cast<unsigned>(rows)), dim3(pk->threads), 0, stream,
                       x, dy, gamma, dx, c, static_cast<int>(plan.chunk), 1,
                       static_cast<int>(rows), eps, SplitArgs{});
    return check_launch("layernorm_bwd_slice_kernel");
  }
  int64_t groups = 0;
  int dispensers = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(pk->fn), pk->threads, 0,
                               plan.members, &groups, &dispensers));
  if (groups == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_bwd: %d groups of %d members do not fit the device", kDispensers,
                     plan.members);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  const int64_t per_group = (rows + groups - 1) / groups;
  if (2 * per_group > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_SHAPE, "layernorm_bwd: %lld rows per group",
                     static_cast<long long>(per_group));
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, 2, kSplitRing, 0, &ws));
  const uint32_t total = static_cast<uint32_t>(groups * plan.members);
  hipLaunchKernelGGL(pk->fn, dim3(total), dim3(pk->threads), 0, stream, x, dy, gamma, dx, c,
                     static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows), eps,
                     make_split_args(ws, total, static_cast<uint32_t>(per_group * 2), kSplitRing,
                                     dispensers));
  return check_launch("layernorm_bwd_slice_kernel(split)");
}

}  // namespace

size_t layernorm_bwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int elem_bytes, int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  const int64_t e = 16 / elem_bytes;
  const int64_t cap = elem_bytes == 4 ? Slices<float>::capacity : Slices<uint16_t>::capacity;
  if (resolve(&c, cols / e, cols % e == 0, cap, &p) != CREDIT_OK || p.members <= 1) return 0;
  int64_t groups = coresident_groups_bound(p.members, cu_count);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  return split_workspace_bytes(groups, p.members, 2, kSplitRing, 0);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_layernorm_bwd_f32(const float* x, const float* dy, const float* gamma,
                                        float* dx, int64_t rows, int64_t cols, float eps,
                                        const credit_cfg* cfg) {
  return layernorm_bwd<float>(x, dy, gamma, dx, rows, cols, eps, cfg);
}

extern "C" int credit_layernorm_bwd_bf16(const uint16_t* x, const uint16_t* dy,
                                         const uint16_t* gamma, uint16_t* dx, int64_t rows,
                                         int64_t cols, float eps, const credit_cfg* cfg) {
  return layernorm_bwd<uint16_t>(x, dy, gamma, dx, rows, cols, eps, cfg);
}
