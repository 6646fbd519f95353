// Weighted-variance normalisation backward, fp32: the reference workload
// weighted_var_backward (dsmem_eval/workloads.py:72-85; kernels
// src/workloads/weighted_var_backward.cu:303-506).
//
//   inv_sum_w = 1 / (sum w + eps),  mean = sum(w x) * inv_sum_w,  d = x - mean
//   var       = sum(w d^2) * inv_sum_w,  inv_std = 1 / sqrt(var + eps)
//   dx        = inv_std (dy - w inv_sum_w sum(dy) - w d inv_std^2 inv_sum_w sum(dy d))
//
// with eps = 1e-5 for both, as the torch function (the CUDA file uses
// 1e-6, weighted_var_backward.cu:34).  The five row sums are accumulated
// about the row's first element x0 in one pass:
//   Sw = sum w, A = sum w (x - x0), B = sum w (x - x0)^2,
//   D = sum dy, E = sum dy (x - x0),
// from which, with c = mean - x0,  sum(w d^2) = B - 2 c A + c^2 Sw and
// sum(dy d) = E - c D: the cancellation of a two-pass computation about a
// point near the mean, in one reduction stage (the reference needs three:
// (sum w, sum w x), then sum w d^2, then (sum dy, sum dy d), :427-506).
// Per-lane partials are fp32, combined in fp64 across waves and members.
// Variants (rows of f32x4 vectors):
//  - STAGED: one workgroup per row, x, w and dy held in VGPRs (up to 4
//            f32x4 of each per lane): one HBM read of each, one write of dx.
//  - SPLIT : P members (P <= 12: five partials each per exchange) hold 1/P
//            of the row; a co-resident wave of ticketed groups looping rows.
//  - READ  : one workgroup per row streaming the row twice (sums, output),
//            for any width and alignment.
// Algorithmic traffic per element: 12 bytes read + 4 written.
#include "api_internal.hpp"
#include "common.hpp"
#include "slices.hpp"

namespace credit {
namespace {

using namespace slices;

constexpr int kWvarValues = 5;

struct Sums {
  float sw, a, b, d, e;
};

__device__ __forceinline__ void accumulate(Sums& s, float x, float w, float dy, float x0) {
  const float t = x - x0;
  const float wt = w * t;
  s.sw += w;
  s.a += wt;
  s.b += wt * t;
  s.d += dy;
  s.e += dy * t;
}
__device__ __forceinline__ void accumulate4(Sums& s, f32x4 x, f32x4 w, f32x4 dy, float x0) {
  accumulate(s, x.x, w.x, dy.x, x0);
  accumulate(s, x.y, w.y, dy.y, x0);
  accumulate(s, x.z, w.z, dy.z, x0);
  accumulate(s, x.w, w.w, dy.w, x0);
}

// Per-row coefficients: dx = c0 dy - w (c1 + d c2), d = (x - x0) - c with
// c = mean - x0 rounded once: d keeps the accuracy of x - x0 (exact for x
// near x0) where x - mean would round twice at the scale of |x|.
struct Coef {
  float x0, c, c0, c1, c2;
};
__device__ __forceinline__ Coef coefficients(const double (&v)[kWvarValues], float x0, float eps) {
  const double sw = v[0], a = v[1], b = v[2], d = v[3], e = v[4];
  const double inv_sum_w = 1.0 / (sw + eps);
  const double mean = (a + static_cast<double>(x0) * sw) * inv_sum_w;
  const double c = mean - x0;
  const double wvar = b - 2.0 * c * a + c * c * sw;
  const double var = wvar * inv_sum_w;
  const double inv_std = 1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps);
  const double sum_dyc = e - c * d;
  Coef k;
  k.x0 = x0;
  k.c = static_cast<float>(c);
  k.c0 = static_cast<float>(inv_std);
  k.c1 = static_cast<float>(inv_std * inv_sum_w * d);
  k.c2 = static_cast<float>(inv_std * inv_std * inv_std * inv_sum_w * sum_dyc);
  return k;
}
__device__ __forceinline__ float dx1(float x, float w, float dy, const Coef& k) {
  return k.c0 * dy - w * (k.c1 + ((x - k.x0) - k.c) * k.c2);
}
__device__ __forceinline__ f32x4 dx4(f32x4 x, f32x4 w, f32x4 dy, const Coef& k) {
  return f32x4{dx1(x.x, w.x, dy.x, k), dx1(x.y, w.y, dy.y, k), dx1(x.z, w.z, dy.z, k),
               dx1(x.w, w.w, dy.w, k)};
}

template <int THREADS, int VPT>
__device__ __forceinline__ void wvar_bwd_slice_kernel_body(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ dy,
    float* __restrict__ dx, int cols, int chunk, int members, int rows, float eps,
    SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[kWvarValues][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, kWvarValues, chunk, cols >> 2, sa);
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  for (int row = sl.row; row < rows; row += sl.step) {
    const size_t off = static_cast<size_t>(row) * cols;
    const buffer_rsrc_t xr = slice_rsrc(x + off, sl);
    const buffer_rsrc_t wr = slice_rsrc(w + off, sl);
    const buffer_rsrc_t dr = slice_rsrc(dy + off, sl);
    f32x4 xv[VPT], wv[VPT], dv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = slice_load(xr, lane_off + k * kStride);
      wv[k] = slice_load(wr, lane_off + k * kStride);
      dv[k] = slice_load(dr, lane_off + k * kStride);
    }
    const float x0 = x[off];
    // Beyond the slice w = dy = 0, which adds nothing to any sum.
    Sums s{0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < VPT; ++k) accumulate4(s, xv[k], wv[k], dv[k], x0);
    double v[kWvarValues] = {s.sw, s.a, s.b, s.d, s.e};
    block_reduce_sum_f64_multi<NW, kWvarValues>(v, red);
    if (members > 1) {
      if (threadIdx.x == 0)
#pragma unroll
        for (int i = 0; i < kWvarValues; ++i) split_publish(g, i, v[i]);
      split_exchange(g);
#pragma unroll
      for (int i = 0; i < kWvarValues; ++i) v[i] = split_sum(g, i);
    }
    const Coef k = coefficients(v, x0, eps);
    const buffer_rsrc_t out = slice_rsrc(dx + off, sl);
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      slice_store(out, lane_off + q * kStride, dx4(xv[q], wv[q], dv[q], k));
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void wvar_bwd_slice_kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ dy,
    float* __restrict__ dx, int cols, int chunk, int members, int rows, float eps,
    SplitArgs sa) {
  wvar_bwd_slice_kernel_body<THREADS, VPT>(x, w, dy, dx, cols, chunk, members, rows, eps, sa);
  split_leave(sa);
}

// Two passes over the row; VEC: f32x4 accesses.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void wvar_bwd_read_kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ dy,
    float* __restrict__ dx, int cols, float eps) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[kWvarValues][NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  const float x0 = x[off];
  // fp32 sums of one vector's four elements, accumulated per lane in fp64.
  double acc[kWvarValues] = {0, 0, 0, 0, 0};
  auto add = [&](const Sums& t) {
    acc[0] += t.sw;
    acc[1] += t.a;
    acc[2] += t.b;
    acc[3] += t.d;
    acc[4] += t.e;
  };
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    const f32x4* wv = reinterpret_cast<const f32x4*>(w + off);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dy + off);
    for (int i = tid; i < nvec; i += THREADS) {
      Sums t{0, 0, 0, 0, 0};
      accumulate4(t, load_nt(xv + i), load_nt(wv + i), load_nt(dv + i), x0);
      add(t);
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      Sums t{0, 0, 0, 0, 0};
      accumulate(t, x[off + c], w[off + c], dy[off + c], x0);
      add(t);
    }
  }
  block_reduce_sum_f64_multi<NW, kWvarValues>(acc, red);
  const double (&v)[kWvarValues] = acc;
  const Coef k = coefficients(v, x0, eps);
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    const f32x4* wv = reinterpret_cast<const f32x4*>(w + off);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dy + off);
    f32x4* out = reinterpret_cast<f32x4*>(dx + off);
    for (int i = tid; i < nvec; i += THREADS)
      store_nt(out + i, dx4(load_nt(xv + i), load_nt(wv + i), load_nt(dv + i), k));
  } else {
    for (int c = tid; c < cols; c += THREADS) dx[off + c] = dx1(x[off + c], w[off + c], dy[off + c], k);
  }
}

using WvarFn = void (*)(const float*, const float*, const float*, float*, int, int, int, int,
                        float, SplitArgs);

// Three tensors held: up to 4 f32x4 of each per lane.
const Pick<WvarFn> kWvar[] = {
    {wvar_bwd_slice_kernel<64, 4>, 64, 256},
    {wvar_bwd_slice_kernel<128, 4>, 128, 512},
    {wvar_bwd_slice_kernel<256, 4>, 256, 1024},
    {wvar_bwd_slice_kernel<512, 4>, 512, 2048},
    {wvar_bwd_slice_kernel<1024, 4>, 1024, 4096},
    {wvar_bwd_slice_kernel<512, 16>, 512, 8192},
};
// AUTO and STAGED hold at most 4096 vectors per workgroup; an explicit SPLIT
// may take the 512-lane 16-vector shape (192 VGPRs of row data, one
// workgroup per CU), which brings 262144 columns within 12 members (five
// partials each fill at most 64 exchange slots per stage).
constexpr int64_t kWvarCapacity = 4096;
constexpr int64_t kWvarSplitCapacity = 8192;

int wvar_plan(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  const int64_t capacity =
      cfg_variant(cfg) == CREDIT_VARIANT_SPLIT ? kWvarSplitCapacity : kWvarCapacity;
  CREDIT_TRY(resolve(cfg, cols, vec, capacity, "weighted_var_backward", plan));
  if (plan->members * kWvarValues > kMaxExchangeValues) {
    if (cfg_variant(cfg) != CREDIT_VARIANT_AUTO)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "weighted_var_backward: split %d exceeds %d members", plan->members,
                       kMaxExchangeValues / kWvarValues);
    *plan = Plan{CREDIT_VARIANT_READ, 1, cols / 4};
  }
  return CREDIT_OK;
}

}  // namespace

size_t wvar_bwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (wvar_plan(&c, cols, cols % 4 == 0, &p) != CREDIT_OK) return 0;
  return slice_workspace(rows, p, kWvarValues, cu_count);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_weighted_var_bwd_f32(const float* x, const float* weight, const float* dy,
                                           float* dx, int64_t rows, int64_t cols, float eps,
                                           const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(weight, "weight", rows));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(weight),
                        static_cast<const void*>(dy), static_cast<const void*>(dx)})
    CREDIT_TRY(check_aligned(p, 4, "weighted_var_backward buffer"));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps > 0.0f))
    return set_error(CREDIT_ERR_BAD_CONFIG, "weighted_var_backward: eps must be > 0");
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {x, weight, dy, dx});
  Plan plan;
  CREDIT_TRY(wvar_plan(cfg, cols, vec, &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      wvar_bwd_read_kernel<256, true><<<r, 256, 0, stream>>>(x, weight, dy, dx, c, eps);
    else
      wvar_bwd_read_kernel<256, false><<<r, 256, 0, stream>>>(x, weight, dy, dx, c, eps);
    return check_launch("wvar_bwd_read_kernel");
  }
  const Pick<WvarFn>* pk = pick_for(kWvar, plan.chunk);
  return launch_slices<WvarFn>(
      cfg, rows, plan, pk, kWvarValues, 1, "wvar_bwd_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, x, weight, dy, dx, c,
                           static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows),
                           eps, sa);
      });
}
