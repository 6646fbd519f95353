// LARS momentum step, fp32: the reference workload lars_momentum
// (dsmem_eval/workloads.py:136-143; kernels
// src/workloads/lars_momentum.cu:283-416).
//
//   u      = 0.9 m + g + 0.01 w          (fp32, torch's operation order)
//   trust  = 0.02 ||w|| / (||u|| + 1e-6) (row norms accumulated in fp64)
//   w'     = w - (1e-3 trust) u
//
// Outputs w' and u.  One reduction stage per row carrying two partials
// (sum w^2, sum u^2), as the reference's cluster kernel (:365-416).
// Variants (rows of f32x4 vectors):
//  - STAGED: one workgroup per row; w and u held in VGPRs (up to 8 f32x4 of
//            each per lane): one HBM read of w, g, m, one write of w', u.
//  - SPLIT : P members hold 1/P of the row each and exchange their two
//            partials; a co-resident wave of ticketed groups looping rows.
//  - READ  : one workgroup per row streaming w, g, m twice (norms, then the
//            outputs), for any width and alignment (the counterpart of
//            block_lars_read_kernel, :283-319).
// Algorithmic traffic per element: 12 bytes read + 8 written.
#include "api_internal.hpp"
#include "common.hpp"
#include "slices.hpp"

namespace credit {
namespace {

using namespace slices;

// 0.9 m + g + 0.01 w with torch's fp32 roundings (each product and sum
// rounded; contraction to FMA off): the update output is bit-exact with the
// reference's torch function.
__device__ __forceinline__ float update1(float w, float g, float m) {
#pragma clang fp contract(off)
  const float a = 0.9f * m;
  const float b = a + g;
  const float c = 0.01f * w;
  return b + c;
}
__device__ __forceinline__ f32x4 update4(f32x4 w, f32x4 g, f32x4 m) {
  return f32x4{update1(w.x, g.x, m.x), update1(w.y, g.y, m.y), update1(w.z, g.z, m.z),
               update1(w.w, g.w, m.w)};
}
__device__ __forceinline__ float sq4(f32x4 v) {
  return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
}

// The step 1e-3 * trust, from the two row sums of squares.
__device__ __forceinline__ float lars_step(double ww, double uu) {
  const double trust = 0.02 * __builtin_sqrt(ww) / (__builtin_sqrt(uu) + 1.0e-6);
  return static_cast<float>(1.0e-3 * trust);
}

template <int THREADS, int VPT>
__device__ __forceinline__ void lars_slice_kernel_body(
    const float* __restrict__ w, const float* __restrict__ grad, const float* __restrict__ mom,
    float* __restrict__ w_out, float* __restrict__ u_out, int cols, int chunk, int members,
    int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[2][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 2, chunk, cols >> 2, sa);
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  for (int row = sl.row; row < rows; row += sl.step) {
    const size_t off = static_cast<size_t>(row) * cols;
    const buffer_rsrc_t wr = slice_rsrc(w + off, sl);
    const buffer_rsrc_t gr = slice_rsrc(grad + off, sl);
    const buffer_rsrc_t mr = slice_rsrc(mom + off, sl);
    // Beyond the slice w = g = m = 0, so u = 0: nothing added to the sums.
    f32x4 wv[VPT], uv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      wv[k] = slice_load(wr, lane_off + k * kStride);
      uv[k] = update4(wv[k], slice_load(gr, lane_off + k * kStride),
                      slice_load(mr, lane_off + k * kStride));
    }
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      a += sq4(wv[k]);
      b += sq4(uv[k]);
    }
    double v[2] = {a, b};
    block_reduce_sum_f64_multi<NW, 2>(v, red);
    double ww = v[0], uu = v[1];
    if (members > 1) {
      if (threadIdx.x == 0) {
        split_publish(g, 0, ww);
        split_publish(g, 1, uu);
      }
      split_exchange(g);
      ww = split_sum(g, 0);
      uu = split_sum(g, 1);
    }
    const float step = lars_step(ww, uu);
    const buffer_rsrc_t wo = slice_rsrc(w_out + off, sl);
    const buffer_rsrc_t uo = slice_rsrc(u_out + off, sl);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      slice_store(wo, lane_off + k * kStride, wv[k] - step * uv[k]);
      slice_store(uo, lane_off + k * kStride, uv[k]);
    }
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void lars_slice_kernel(
    const float* __restrict__ w, const float* __restrict__ grad, const float* __restrict__ mom,
    float* __restrict__ w_out, float* __restrict__ u_out, int cols, int chunk, int members,
    int rows, SplitArgs sa) {
  lars_slice_kernel_body<THREADS, VPT>(w, grad, mom, w_out, u_out, cols, chunk, members, rows, sa);
  split_leave(sa);
}

// Two passes over the row; VEC: f32x4 accesses.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void lars_read_kernel(
    const float* __restrict__ w, const float* __restrict__ grad, const float* __restrict__ mom,
    float* __restrict__ w_out, float* __restrict__ u_out, int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[2][NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  double a = 0.0, b = 0.0;
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* wv = reinterpret_cast<const f32x4*>(w + off);
    const f32x4* gv = reinterpret_cast<const f32x4*>(grad + off);
    const f32x4* mv = reinterpret_cast<const f32x4*>(mom + off);
    for (int i = tid; i < nvec; i += THREADS) {
      const f32x4 x = load_nt(wv + i);
      a += static_cast<double>(sq4(x));
      b += static_cast<double>(sq4(update4(x, load_nt(gv + i), load_nt(mv + i))));
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float x = w[off + c];
      const float u = update1(x, grad[off + c], mom[off + c]);
      a += static_cast<double>(x * x);
      b += static_cast<double>(u * u);
    }
  }
  double v[2] = {a, b};
  block_reduce_sum_f64_multi<NW, 2>(v, red);
  const float step = lars_step(v[0], v[1]);
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* wv = reinterpret_cast<const f32x4*>(w + off);
    const f32x4* gv = reinterpret_cast<const f32x4*>(grad + off);
    const f32x4* mv = reinterpret_cast<const f32x4*>(mom + off);
    f32x4* wo = reinterpret_cast<f32x4*>(w_out + off);
    f32x4* uo = reinterpret_cast<f32x4*>(u_out + off);
    for (int i = tid; i < nvec; i += THREADS) {
      const f32x4 x = load_nt(wv + i);
      const f32x4 u = update4(x, load_nt(gv + i), load_nt(mv + i));
      store_nt(wo + i, x - step * u);
      store_nt(uo + i, u);
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float x = w[off + c];
      const float u = update1(x, grad[off + c], mom[off + c]);
      w_out[off + c] = x - step * u;
      u_out[off + c] = u;
    }
  }
}

using LarsFn = void (*)(const float*, const float*, const float*, float*, float*, int, int, int,
                        int, SplitArgs);

// Two tensors held (w, u): up to 8 f32x4 of each per lane.
const Pick<LarsFn> kLars[] = {
    {lars_slice_kernel<64, 4>, 64, 256},
    {lars_slice_kernel<128, 4>, 128, 512},
    {lars_slice_kernel<256, 4>, 256, 1024},
    {lars_slice_kernel<256, 8>, 256, 2048},
    {lars_slice_kernel<512, 8>, 512, 4096},
    {lars_slice_kernel<1024, 8>, 1024, 8192},
};
constexpr int64_t kLarsCapacity = 8192;
// AUTO on wider rows: 512-lane slices (measured at 4096 x 65536: 4 members
// of 4096 vectors beat 2 of 8192 by 4-13%, two workgroups per CU).
constexpr int64_t kAutoSlice = 4096;
constexpr int kLarsValues = 2;

// Variant plan; AUTO falls back to READ where a split would exceed the
// exchange's partials per stage.
int lars_plan(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  CREDIT_TRY(resolve(cfg, cols, vec, kLarsCapacity, "lars_momentum", plan, kAutoSlice));
  if (plan->members * kLarsValues > kMaxExchangeValues && cfg_variant(cfg) == CREDIT_VARIANT_AUTO)
    CREDIT_TRY(resolve(cfg, cols, vec, kLarsCapacity, "lars_momentum", plan));  // fewer, wider slices
  if (plan->members * kLarsValues > kMaxExchangeValues) {
    if (cfg_variant(cfg) != CREDIT_VARIANT_AUTO)
      return set_error(CREDIT_ERR_UNSUPPORTED, "lars_momentum: split %d exceeds %d members",
                       plan->members, kMaxExchangeValues / kLarsValues);
    *plan = Plan{CREDIT_VARIANT_READ, 1, cols / 4};
  }
  return CREDIT_OK;
}

}  // namespace

size_t lars_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (lars_plan(&c, cols, cols % 4 == 0, &p) != CREDIT_OK) return 0;
  return slice_workspace(rows, p, kLarsValues, cu_count);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_lars_momentum_f32(const float* weight, const float* grad,
                                        const float* momentum, float* weight_out,
                                        float* update_out, int64_t rows, int64_t cols,
                                        const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(weight, "weight", rows));
  CREDIT_TRY(check_row_ptr(grad, "grad", rows));
  CREDIT_TRY(check_row_ptr(momentum, "momentum", rows));
  CREDIT_TRY(check_row_ptr(weight_out, "weight_out", rows));
  CREDIT_TRY(check_row_ptr(update_out, "update_out", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  for (const void* p : {static_cast<const void*>(weight), static_cast<const void*>(grad),
                        static_cast<const void*>(momentum), static_cast<const void*>(weight_out),
                        static_cast<const void*>(update_out)})
    CREDIT_TRY(check_aligned(p, 4, "lars_momentum buffer"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {weight, grad, momentum, weight_out, update_out});
  Plan plan;
  CREDIT_TRY(lars_plan(cfg, cols, vec, &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      lars_read_kernel<256, true><<<r, 256, 0, stream>>>(weight, grad, momentum, weight_out,
                                                          update_out, c);
    else
      lars_read_kernel<256, false><<<r, 256, 0, stream>>>(weight, grad, momentum, weight_out,
                                                           update_out, c);
    return check_launch("lars_read_kernel");
  }
  const Pick<LarsFn>* pk = pick_for(kLars, plan.chunk);
  return launch_slices<LarsFn>(
      cfg, rows, plan, pk, kLarsValues, 1, "lars_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, weight, grad,
                           momentum, weight_out, update_out, c, static_cast<int>(plan.chunk),
                           plan.members, static_cast<int>(rows), sa);
      });
}
