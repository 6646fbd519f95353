// Pearson-correlation backward, fp32: the reference workload
// pearson_backward (dsmem_eval/workloads.py:96-112; kernels
// src/workloads/pearson_backward.cu:311-482).
//
//   xc = x - mean(x),  yc = y - mean(y)
//   vx = sum xc^2, vy = sum yc^2, cov = sum xc yc
//   ix = 1/sqrt(vx + eps), iy = 1/sqrt(vy + eps)
//   dx = grad (yc ix iy - xc cov ix^3 iy),  dy = grad (xc ix iy - yc cov ix iy^3)
//
// eps = 1e-6 as the torch function (the CUDA file uses 1e-5,
// pearson_backward.cu:34); grad is one value per row.  The five row sums are
// accumulated about the row's first elements (x0, y0) in one pass:
//   Sx = sum(x - x0), Sy = sum(y - y0), Sxx, Syy, Sxy (of the shifted values)
// so that vx = Sxx - Sx^2/N, vy = Syy - Sy^2/N, cov = Sxy - Sx Sy/N carry only
// the cancellation of a two-pass computation about a point near the mean:
// one reduction stage (the reference needs two, the means then the three
// centred sums, :418-482).  Per-lane partials are fp32, combined in fp64.
// Variants (rows of f32x4 vectors):
//  - STAGED: one workgroup per row, x and y held in VGPRs (up to 8 f32x4 of
//            each per lane): one HBM read of each, one write of dx and dy.
//  - SPLIT : P members (P <= 12) hold 1/P of the row; a co-resident wave of
//            ticketed groups looping rows.
//  - READ  : one workgroup per row streaming the row twice, for any width
//            and alignment.
// Algorithmic traffic per element: 8 bytes read + 8 written (+4 per row).
#include "api_internal.hpp"
#include "common.hpp"
#include "slices.hpp"

namespace credit {
namespace {

using namespace slices;

constexpr int kPearsonValues = 5;

struct Sums {
  float sx, sy, sxx, syy, sxy;
};

__device__ __forceinline__ void accumulate(Sums& s, float x, float y, float x0, float y0) {
  const float a = x - x0, b = y - y0;
  s.sx += a;
  s.sy += b;
  s.sxx += a * a;
  s.syy += b * b;
  s.sxy += a * b;
}
__device__ __forceinline__ void accumulate4(Sums& s, f32x4 x, f32x4 y, float x0, float y0) {
  accumulate(s, x.x, y.x, x0, y0);
  accumulate(s, x.y, y.y, x0, y0);
  accumulate(s, x.z, y.z, x0, y0);
  accumulate(s, x.w, y.w, x0, y0);
}

// dx = yc a - xc bx, dy = xc a - yc by, with xc = (x - x0) - cx and
// cx = mean(x) - x0 rounded once (likewise yc): the centred values keep the
// accuracy of x - x0 where x - mean would round at the scale of |x|.
struct Coef {
  float x0, y0, cx, cy, a, bx, by;
};
__device__ __forceinline__ Coef coefficients(const double (&v)[kPearsonValues], float x0, float y0,
                                             float grad, int cols, float eps) {
  const double n = cols;
  const double sx = v[0], sy = v[1];
  const double vx = v[2] - sx * sx / n;
  const double vy = v[3] - sy * sy / n;
  const double cov = v[4] - sx * sy / n;
  const double ix = 1.0 / __builtin_sqrt((vx > 0.0 ? vx : 0.0) + eps);
  const double iy = 1.0 / __builtin_sqrt((vy > 0.0 ? vy : 0.0) + eps);
  const double gr = grad;
  Coef k;
  k.x0 = x0;
  k.y0 = y0;
  k.cx = static_cast<float>(sx / n);
  k.cy = static_cast<float>(sy / n);
  k.a = static_cast<float>(gr * ix * iy);
  k.bx = static_cast<float>(gr * cov * ix * ix * ix * iy);
  k.by = static_cast<float>(gr * cov * ix * iy * iy * iy);
  return k;
}

struct Pair4 {
  f32x4 dx, dy;
};
__device__ __forceinline__ Pair4 grads4(f32x4 x, f32x4 y, const Coef& k) {
  const f32x4 xc = (x - k.x0) - k.cx, yc = (y - k.y0) - k.cy;
  return Pair4{yc * k.a - xc * k.bx, xc * k.a - yc * k.by};
}

template <int THREADS, int VPT>
__device__ __forceinline__ void pearson_bwd_slice_kernel_body(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ grad,
    float* __restrict__ dx, float* __restrict__ dy, int cols, int chunk, int members, int rows,
    float eps, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[kPearsonValues][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, kPearsonValues, chunk, cols >> 2, sa);
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  const uint32_t slice_bytes = static_cast<uint32_t>(sl.vlen) * 16u;
  for (int row = sl.row; row < rows; row += sl.step) {
    const size_t off = static_cast<size_t>(row) * cols;
    const buffer_rsrc_t xr = slice_rsrc(x + off, sl);
    const buffer_rsrc_t yr = slice_rsrc(y + off, sl);
    f32x4 xv[VPT], yv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = slice_load(xr, lane_off + k * kStride);
      yv[k] = slice_load(yr, lane_off + k * kStride);
    }
    const float x0 = x[off], y0 = y[off];
    Sums s{0, 0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      // Beyond the slice the shifted values would be -x0, -y0: add nothing.
      Sums t{0, 0, 0, 0, 0};
      accumulate4(t, xv[k], yv[k], x0, y0);
      const bool in = lane_off + k * kStride < slice_bytes;
      s.sx += in ? t.sx : 0.0f;
      s.sy += in ? t.sy : 0.0f;
      s.sxx += in ? t.sxx : 0.0f;
      s.syy += in ? t.syy : 0.0f;
      s.sxy += in ? t.sxy : 0.0f;
    }
    double v[kPearsonValues] = {s.sx, s.sy, s.sxx, s.syy, s.sxy};
    block_reduce_sum_f64_multi<NW, kPearsonValues>(v, red);
    if (members > 1) {
      if (threadIdx.x == 0)
#pragma unroll
        for (int i = 0; i < kPearsonValues; ++i) split_publish(g, i, v[i]);
      split_exchange(g);
#pragma unroll
      for (int i = 0; i < kPearsonValues; ++i) v[i] = split_sum(g, i);
    }
    const Coef k = coefficients(v, x0, y0, grad[row], cols, eps);
    const buffer_rsrc_t dxo = slice_rsrc(dx + off, sl);
    const buffer_rsrc_t dyo = slice_rsrc(dy + off, sl);
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      const Pair4 r = grads4(xv[q], yv[q], k);
      slice_store(dxo, lane_off + q * kStride, r.dx);
      slice_store(dyo, lane_off + q * kStride, r.dy);
    }
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void pearson_bwd_slice_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ grad,
    float* __restrict__ dx, float* __restrict__ dy, int cols, int chunk, int members, int rows,
    float eps, SplitArgs sa) {
  pearson_bwd_slice_kernel_body<THREADS, VPT>(x, y, grad, dx, dy, cols, chunk, members, rows, eps, sa);
  split_leave(sa);
}

// Two passes over the row; VEC: f32x4 accesses.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void pearson_bwd_read_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ grad,
    float* __restrict__ dx, float* __restrict__ dy, int cols, float eps) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[kPearsonValues][NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  const float x0 = x[off], y0 = y[off];
  // fp32 sums of one vector's four elements, accumulated per lane in fp64.
  double v[kPearsonValues] = {0, 0, 0, 0, 0};
  auto add = [&](const Sums& t) {
    v[0] += t.sx;
    v[1] += t.sy;
    v[2] += t.sxx;
    v[3] += t.syy;
    v[4] += t.sxy;
  };
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    const f32x4* yv = reinterpret_cast<const f32x4*>(y + off);
    for (int i = tid; i < nvec; i += THREADS) {
      Sums t{0, 0, 0, 0, 0};
      accumulate4(t, load_nt(xv + i), load_nt(yv + i), x0, y0);
      add(t);
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      Sums t{0, 0, 0, 0, 0};
      accumulate(t, x[off + c], y[off + c], x0, y0);
      add(t);
    }
  }
  block_reduce_sum_f64_multi<NW, kPearsonValues>(v, red);
  const Coef k = coefficients(v, x0, y0, grad[blockIdx.x], cols, eps);
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    const f32x4* yv = reinterpret_cast<const f32x4*>(y + off);
    f32x4* dxo = reinterpret_cast<f32x4*>(dx + off);
    f32x4* dyo = reinterpret_cast<f32x4*>(dy + off);
    for (int i = tid; i < nvec; i += THREADS) {
      const Pair4 r = grads4(load_nt(xv + i), load_nt(yv + i), k);
      store_nt(dxo + i, r.dx);
      store_nt(dyo + i, r.dy);
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float xc = (x[off + c] - k.x0) - k.cx, yc = (y[off + c] - k.y0) - k.cy;
      dx[off + c] = yc * k.a - xc * k.bx;
      dy[off + c] = xc * k.a - yc * k.by;
    }
  }
}

using PearsonFn = void (*)(const float*, const float*, const float*, float*, float*, int, int,
                           int, int, float, SplitArgs);

// Two tensors held (x, y): up to 8 f32x4 of each per lane.
const Pick<PearsonFn> kPearson[] = {
    {pearson_bwd_slice_kernel<64, 4>, 64, 256},
    {pearson_bwd_slice_kernel<128, 4>, 128, 512},
    {pearson_bwd_slice_kernel<256, 4>, 256, 1024},
    {pearson_bwd_slice_kernel<256, 8>, 256, 2048},
    {pearson_bwd_slice_kernel<512, 8>, 512, 4096},
    {pearson_bwd_slice_kernel<1024, 8>, 1024, 8192},
};
constexpr int64_t kPearsonCapacity = 8192;
// AUTO on wider rows: 512-lane slices (measured at 4096 x 65536: 4 members
// of 4096 vectors beat 2 of 8192 by 4-13%, two workgroups per CU).
constexpr int64_t kAutoSlice = 4096;

int pearson_plan(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  CREDIT_TRY(resolve(cfg, cols, vec, kPearsonCapacity, "pearson_backward", plan, kAutoSlice));
  if (plan->members * kPearsonValues > kMaxExchangeValues && cfg_variant(cfg) == CREDIT_VARIANT_AUTO)
    CREDIT_TRY(resolve(cfg, cols, vec, kPearsonCapacity, "pearson_backward", plan));  // fewer, wider slices
  if (plan->members * kPearsonValues > kMaxExchangeValues) {
    if (cfg_variant(cfg) != CREDIT_VARIANT_AUTO)
      return set_error(CREDIT_ERR_UNSUPPORTED, "pearson_backward: split %d exceeds %d members",
                       plan->members, kMaxExchangeValues / kPearsonValues);
    *plan = Plan{CREDIT_VARIANT_READ, 1, cols / 4};
  }
  return CREDIT_OK;
}

}  // namespace

size_t pearson_bwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (pearson_plan(&c, cols, cols % 4 == 0, &p) != CREDIT_OK) return 0;
  return slice_workspace(rows, p, kPearsonValues, cu_count);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_pearson_bwd_f32(const float* x, const float* y, const float* grad,
                                      float* dx, float* dy, int64_t rows, int64_t cols,
                                      float eps, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(y, "y", rows));
  CREDIT_TRY(check_row_ptr(grad, "grad", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(y),
                        static_cast<const void*>(grad), static_cast<const void*>(dx),
                        static_cast<const void*>(dy)})
    CREDIT_TRY(check_aligned(p, 4, "pearson_backward buffer"));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps > 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "pearson_backward: eps must be > 0");
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {x, y, dx, dy});
  Plan plan;
  CREDIT_TRY(pearson_plan(cfg, cols, vec, &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      pearson_bwd_read_kernel<256, true><<<r, 256, 0, stream>>>(x, y, grad, dx, dy, c, eps);
    else
      pearson_bwd_read_kernel<256, false><<<r, 256, 0, stream>>>(x, y, grad, dx, dy, c, eps);
    return check_launch("pearson_bwd_read_kernel");
  }
  const Pick<PearsonFn>* pk = pick_for(kPearson, plan.chunk);
  return launch_slices<PearsonFn>(
      cfg, rows, plan, pk, kPearsonValues, 1, "pearson_bwd_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, x, y, grad, dx, dy,
                           c, static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows),
                           eps, sa);
      });
}
