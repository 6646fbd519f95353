// C4: online softmax forward and backward over fp32 rows, and the
// reference's fused softmax-logits backward.
//
//   forward : m = max_j x,  s = sum_j e^(x - m),  P = e^(x - m) / s,
//             rowmax = m,  lse = m + ln s
//   backward: dx = P * (dy - sum_j P*dy)
//   logits backward (dsmem_eval/workloads.py:122-125,
//   src/workloads/softmax_logits_backward.cu:314-476):
//             p = softmax(logits),  dx = p * (dy - sum_j p*dy)
//
// Variants (the reference's block_read / block_smem / cluster_smem):
//  - STAGED: one workgroup holds the whole row (its slices) in VGPRs.
//  - SPLIT : P workgroups per row (ticketed groups, common.hpp).  Each
//            member reduces its slice to (max, sum of e^(x - max)); the
//            group exchanges the pairs once and every member merges them
//            in member order: m = max m_i, s = sum s_i e^(m_i - m).  The
//            forward then writes P from registers: one read, one write.
//  - READ  : one workgroup streams the row: an online (max, sum) pass,
//            then an output pass (forward: 2 reads + 1 write per element).
// e^x is exp_accurate (common.hpp): the hardware exp2 with the product
// x*log2(e) carried to double-float precision.
#include <initializer_list>

#include "api_internal.hpp"
#include "common.hpp"
#include "slices.hpp"

namespace credit {
namespace {

using namespace slices;

constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float max4(f32x4 v) {
  return fmax_nan(fmax_nan(v.x, v.y), fmax_nan(v.z, v.w));
}

__device__ __forceinline__ float sumexp4(f32x4 v, float m) {
  return (exp_accurate(v.x - m) + exp_accurate(v.y - m)) +
         (exp_accurate(v.z - m) + exp_accurate(v.w - m));
}

__device__ __forceinline__ f32x4 prob4(f32x4 v, float m, float inv_s) {
  return f32x4{exp_accurate(v.x - m) * inv_s, exp_accurate(v.y - m) * inv_s,
               exp_accurate(v.z - m) * inv_s, exp_accurate(v.w - m) * inv_s};
}

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
}

__device__ __forceinline__ f32x4 grad4(f32x4 p, f32x4 dy, float dot) {
  return f32x4{p.x * (dy.x - dot), p.y * (dy.y - dot), p.z * (dy.z - dot),
               p.w * (dy.w - dot)};
}

// e^(a - b) in double, 0 when a is -inf (an empty or all -inf partial).
__device__ __forceinline__ double rescale(double a, double b) {
  return a == -__builtin_inf() ? 0.0 : ::exp(a - b);
}

// One step of the streaming (max, sum) recurrence for a batch whose
// NaN-propagating max is bm: a larger max rescales the running sum; a NaN
// poisons the sum (every output of the row is then NaN); a batch that is
// all -inf while the running max is still -inf adds nothing.
__device__ __forceinline__ void online_update(float bm, float& m, double& s) {
  if (bm != bm) {
    s = __builtin_nan("");
  } else if (bm > m) {
    s *= rescale(m, bm);
    m = bm;
  }
}

// Block-wide (max, sum relative to max).  Every lane brings its max m and
// its sum s relative to m; the result is wave-uniform.  The NaN-propagating
// max keeps rowmax bit-exact with torch.amax; a NaN anywhere also turns the
// sum into NaN.
template <int NW>
__device__ __forceinline__ void block_maxsum(float m, double s, float* mslots, double* sslots,
                                             float* out_m, double* out_s) {
  const float M = block_reduce<NW>(m, MaxOp{}, mslots);
  const double scaled = s == 0.0 ? 0.0 : s * rescale(m, M);
  *out_s = block_reduce_sum_f64<NW>(scaled, sslots);
  *out_m = M;
}

// Merge the group's (max, sum) partials in member order (stage values 0, 1).
__device__ __forceinline__ void split_merge_maxsum(const SplitGroup& g, float* m, double* s) {
  double M = -__builtin_inf();
  for (int i = 0; i < g.members; ++i) M = __builtin_elementwise_maximum(M, split_get(g, 0, i));
  double S = 0.0;
  for (int i = 0; i < g.members; ++i) {
    const double si = split_get(g, 1, i);
    if (si != 0.0) S += si * rescale(split_get(g, 0, i), M);
  }
  *m = static_cast<float>(M);
  *s = S;
}

// --------------------------------------------------------- forward (C4) --
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_fwd_slice_kernel(
    const float* __restrict__ x, float* __restrict__ p, float* __restrict__ rowmax,
    float* __restrict__ lse, int cols, int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  __shared__ double sred[NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 2, chunk, cols >> 2, sa);
  for (int row = sl.row; row < rows; row += sl.step) {
  const int tid = opaque_lane_index();
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + static_cast<size_t>(row) * cols) + sl.v0;
  f32x4 v[VPT];
  // (xr + k*THREADS)[tid]: a uniform base per k and one lane offset, so no
  // per-k lane address stays live across the row loop.
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    v[k] = tid < sl.vlen - k * THREADS ? load_nt(&(xr + k * THREADS)[tid])
                                       : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
  float lm = kNegInf;
#pragma unroll
  for (int k = 0; k < VPT; ++k) lm = fmax_nan(lm, max4(v[k]));
  const float wm = block_reduce<NW>(lm, MaxOp{}, mred);
  float ls = 0.0f;
  if (wm != kNegInf) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) ls += sumexp4(v[k], wm);
  }
  double ws = block_reduce_sum_f64<NW>(static_cast<double>(ls), sred);
  float m = wm;
  double s = ws;
  if (members > 1) {
    if (tid == 0) {
      split_publish(g, 0, static_cast<double>(wm));
      split_publish(g, 1, ws);
    }
    split_exchange(g);
    split_merge_maxsum(g, &m, &s);
  }
  const float inv_s = static_cast<float>(1.0 / s);
  f32x4* pr = reinterpret_cast<f32x4*>(p + static_cast<size_t>(row) * cols) + sl.v0;
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    if (tid < sl.vlen - k * THREADS) store_nt(&(pr + k * THREADS)[tid], prob4(v[k], m, inv_s));
  if (sl.member == 0 && tid == 0) {
    rowmax[row] = m;
    lse[row] = static_cast<float>(static_cast<double>(m) + ::log(s));
  }
  }
}

// Streaming forward: online (max, sum) pass, then the output pass.  VEC:
// f32x4 loads (cols % 4 == 0, 16-byte aligned rows); else element loads.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void softmax_fwd_read_kernel(
    const float* __restrict__ x, float* __restrict__ p, float* __restrict__ rowmax,
    float* __restrict__ lse, int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  __shared__ double sred[NW];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const float* xr = x + static_cast<size_t>(row) * cols;
  float* pr = p + static_cast<size_t>(row) * cols;
  float m = kNegInf;  // running max of the finite path
  double s = 0.0;     // sum of e^(x - m)
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(xr);
    int i = tid;
    for (; i + THREADS < nvec; i += 2 * THREADS) {
      const f32x4 a = load_nt(xv + i), b = load_nt(xv + i + THREADS);
      online_update(fmax_nan(max4(a), max4(b)), m, s);
      if (m != kNegInf) s += static_cast<double>(sumexp4(a, m) + sumexp4(b, m));
    }
    for (; i < nvec; i += THREADS) {
      const f32x4 a = load_nt(xv + i);
      online_update(max4(a), m, s);
      if (m != kNegInf) s += static_cast<double>(sumexp4(a, m));
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float v = xr[c];
      online_update(v, m, s);
      if (m != kNegInf) s += static_cast<double>(exp_accurate(v - m));
    }
  }
  float M;
  double S;
  block_maxsum<NW>(m, s, mred, sred, &M, &S);
  const float inv_s = static_cast<float>(1.0 / S);
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(xr);
    f32x4* pv = reinterpret_cast<f32x4*>(pr);
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS) {
      const f32x4 a = load_nt(xv + i), b = load_nt(xv + i + THREADS),
                  c = load_nt(xv + i + 2 * THREADS), d = load_nt(xv + i + 3 * THREADS);
      store_nt(pv + i, prob4(a, M, inv_s));
      store_nt(pv + i + THREADS, prob4(b, M, inv_s));
      store_nt(pv + i + 2 * THREADS, prob4(c, M, inv_s));
      store_nt(pv + i + 3 * THREADS, prob4(d, M, inv_s));
    }
    for (; i < nvec; i += THREADS) store_nt(pv + i, prob4(load_nt(xv + i), M, inv_s));
  } else {
    for (int c = tid; c < cols; c += THREADS) pr[c] = exp_accurate(xr[c] - M) * inv_s;
  }
  if (tid == 0) {
    // rowmax must carry NaN like torch.amax: S is NaN exactly when the row
    // holds a NaN.
    rowmax[row] = S != S ? __builtin_nanf("") : M;
    lse[row] = static_cast<float>(static_cast<double>(M) + ::log(S));
  }
}

// -------------------------------------------------------- backward (C4) --
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_bwd_slice_kernel(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int cols,
    int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double sred[NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 1, chunk, cols >> 2, sa);
  for (int row = sl.row; row < rows; row += sl.step) {
  const int tid = opaque_lane_index();
  const size_t off = static_cast<size_t>(row) * cols;
  const f32x4* pr = reinterpret_cast<const f32x4*>(p + off) + sl.v0;
  const f32x4* dr = reinterpret_cast<const f32x4*>(dy + off) + sl.v0;
  f32x4 pv[VPT], dv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const bool in = tid < sl.vlen - k * THREADS;
    pv[k] = in ? load_nt(&(pr + k * THREADS)[tid]) : f32x4{0, 0, 0, 0};
    dv[k] = in ? load_nt(&(dr + k * THREADS)[tid]) : f32x4{0, 0, 0, 0};
  }
  float ld = 0.0f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) ld += dot4(pv[k], dv[k]);
  double dot = block_reduce_sum_f64<NW>(static_cast<double>(ld), sred);
  if (members > 1) {
    if (tid == 0) split_publish(g, 0, dot);
    split_exchange(g);
    dot = split_sum(g, 0);
  }
  const float d = static_cast<float>(dot);
  f32x4* xr = reinterpret_cast<f32x4*>(dx + off) + sl.v0;
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    if (tid < sl.vlen - k * THREADS) store_nt(&(xr + k * THREADS)[tid], grad4(pv[k], dv[k], d));
  }
}

template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void softmax_bwd_read_kernel(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ double sred[NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  double acc = 0.0;
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* pv = reinterpret_cast<const f32x4*>(p + off);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dy + off);
    int i = tid;
    for (; i + THREADS < nvec; i += 2 * THREADS) {
      const f32x4 a = load_nt(pv + i), b = load_nt(pv + i + THREADS);
      const f32x4 da = load_nt(dv + i), db = load_nt(dv + i + THREADS);
      acc += static_cast<double>(dot4(a, da) + dot4(b, db));
    }
    for (; i < nvec; i += THREADS) acc += static_cast<double>(dot4(load_nt(pv + i), load_nt(dv + i)));
  } else {
    for (int c = tid; c < cols; c += THREADS) acc += static_cast<double>(p[off + c] * dy[off + c]);
  }
  const float d = static_cast<float>(block_reduce_sum_f64<NW>(acc, sred));
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* pv = reinterpret_cast<const f32x4*>(p + off);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dy + off);
    f32x4* xv = reinterpret_cast<f32x4*>(dx + off);
    int i = tid;
    for (; i + THREADS < nvec; i += 2 * THREADS) {
      const f32x4 a = load_nt(pv + i), b = load_nt(pv + i + THREADS);
      const f32x4 da = load_nt(dv + i), db = load_nt(dv + i + THREADS);
      store_nt(xv + i, grad4(a, da, d));
      store_nt(xv + i + THREADS, grad4(b, db, d));
    }
    for (; i < nvec; i += THREADS) store_nt(xv + i, grad4(load_nt(pv + i), load_nt(dv + i), d));
  } else {
    for (int c = tid; c < cols; c += THREADS) dx[off + c] = p[off + c] * (dy[off + c] - d);
  }
}

// ------------------------------------------- softmax-logits backward ----
// Two stages: (max, sum) of the logits, then sum p*dy with p formed in
// registers (src/workloads/softmax_logits_backward.cu:410-476 runs the same
// math as three cluster reductions).
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_logits_bwd_slice_kernel(
    const float* __restrict__ logits, const float* __restrict__ dy, float* __restrict__ dx,
    int cols, int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  __shared__ double sred[2][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 2, chunk, cols >> 2, sa);
  for (int row = sl.row; row < rows; row += sl.step) {
  const int tid = opaque_lane_index();
  const size_t off = static_cast<size_t>(row) * cols;
  const f32x4* lr = reinterpret_cast<const f32x4*>(logits + off) + sl.v0;
  const f32x4* dr = reinterpret_cast<const f32x4*>(dy + off) + sl.v0;
  f32x4 v[VPT], dv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const bool in = tid < sl.vlen - k * THREADS;
    v[k] = in ? load_nt(&(lr + k * THREADS)[tid]) : f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    dv[k] = in ? load_nt(&(dr + k * THREADS)[tid]) : f32x4{0, 0, 0, 0};
  }
  float lm = kNegInf;
#pragma unroll
  for (int k = 0; k < VPT; ++k) lm = fmax_nan(lm, max4(v[k]));
  const float wm = block_reduce<NW>(lm, MaxOp{}, mred);
  float ls = 0.0f;
  if (wm != kNegInf) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) ls += sumexp4(v[k], wm);
  }
  const double ws = block_reduce_sum_f64<NW>(static_cast<double>(ls), sred[0]);
  float m = wm;
  double s = ws;
  if (members > 1) {
    if (tid == 0) {
      split_publish(g, 0, static_cast<double>(wm));
      split_publish(g, 1, ws);
    }
    split_exchange(g);
    split_merge_maxsum(g, &m, &s);
  }
  const float inv_s = static_cast<float>(1.0 / s);
  float ld = 0.0f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    v[k] = prob4(v[k], m, inv_s);  // out-of-slice lanes: e^-inf = 0
    ld += dot4(v[k], dv[k]);
  }
  double dot = block_reduce_sum_f64<NW>(static_cast<double>(ld), sred[1]);
  if (members > 1) {
    if (tid == 0) split_publish(g, 0, dot);
    split_exchange(g, 1);  // stage 2 carries the dot only
    dot = split_sum(g, 0);
  }
  const float d = static_cast<float>(dot);
  f32x4* xr = reinterpret_cast<f32x4*>(dx + off) + sl.v0;
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    if (tid < sl.vlen - k * THREADS) store_nt(&(xr + k * THREADS)[tid], grad4(v[k], dv[k], d));
  }
}

// Streaming logits backward: online (max, sum) over the logits; sum p*dy
// (re-reading logits and dy); output pass (re-reading both again).
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void softmax_logits_bwd_read_kernel(
    const float* __restrict__ logits, const float* __restrict__ dy, float* __restrict__ dx,
    int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  __shared__ double sred[2][NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  const float* lr = logits + off;
  const float* dr = dy + off;
  float m = kNegInf;
  double s = 0.0;
  const int nvec = cols >> 2;
  if (VEC) {
    const f32x4* lv = reinterpret_cast<const f32x4*>(lr);
    for (int i = tid; i < nvec; i += THREADS) {
      const f32x4 a = load_nt(lv + i);
      online_update(max4(a), m, s);
      if (m != kNegInf) s += static_cast<double>(sumexp4(a, m));
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float v = lr[c];
      online_update(v, m, s);
      if (m != kNegInf) s += static_cast<double>(exp_accurate(v - m));
    }
  }
  float M;
  double S;
  block_maxsum<NW>(m, s, mred, sred[0], &M, &S);
  const float inv_s = static_cast<float>(1.0 / S);
  double acc = 0.0;
  if (VEC) {
    const f32x4* lv = reinterpret_cast<const f32x4*>(lr);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dr);
    for (int i = tid; i < nvec; i += THREADS)
      acc += static_cast<double>(dot4(prob4(load_nt(lv + i), M, inv_s), load_nt(dv + i)));
  } else {
    for (int c = tid; c < cols; c += THREADS)
      acc += static_cast<double>(exp_accurate(lr[c] - M) * inv_s * dr[c]);
  }
  const float d = static_cast<float>(block_reduce_sum_f64<NW>(acc, sred[1]));
  if (VEC) {
    const f32x4* lv = reinterpret_cast<const f32x4*>(lr);
    const f32x4* dv = reinterpret_cast<const f32x4*>(dr);
    f32x4* xv = reinterpret_cast<f32x4*>(dx + off);
    for (int i = tid; i < nvec; i += THREADS)
      store_nt(xv + i, grad4(prob4(load_nt(lv + i), M, inv_s), load_nt(dv + i), d));
  } else {
    for (int c = tid; c < cols; c += THREADS)
      dx[off + c] = exp_accurate(lr[c] - M) * inv_s * (dr[c] - d);
  }
}

// ------------------------------------------------------------ dispatch ---
using FwdFn = void (*)(const float*, float*, float*, float*, int, int, int, int, SplitArgs);
using BwdFn = void (*)(const float*, const float*, float*, int, int, int, int, SplitArgs);

// One tensor staged (forward): up to 16 f32x4 per lane.  Two tensors staged
// (backward, logits backward): up to 8 f32x4 of each per lane.
const Pick<FwdFn> kFwd[] = {
    {softmax_fwd_slice_kernel<64, 4>, 64, 256},
    {softmax_fwd_slice_kernel<128, 4>, 128, 512},
    {softmax_fwd_slice_kernel<256, 4>, 256, 1024},
    {softmax_fwd_slice_kernel<256, 8>, 256, 2048},
    {softmax_fwd_slice_kernel<512, 8>, 512, 4096},
    {softmax_fwd_slice_kernel<1024, 8>, 1024, 8192},
    {softmax_fwd_slice_kernel<1024, 16>, 1024, 16384},
};
const Pick<BwdFn> kBwd[] = {
    {softmax_bwd_slice_kernel<64, 4>, 64, 256},
    {softmax_bwd_slice_kernel<128, 4>, 128, 512},
    {softmax_bwd_slice_kernel<256, 4>, 256, 1024},
    {softmax_bwd_slice_kernel<256, 8>, 256, 2048},
    {softmax_bwd_slice_kernel<512, 8>, 512, 4096},
    {softmax_bwd_slice_kernel<1024, 8>, 1024, 8192},
};
const Pick<BwdFn> kLogits[] = {
    {softmax_logits_bwd_slice_kernel<64, 4>, 64, 256},
    {softmax_logits_bwd_slice_kernel<128, 4>, 128, 512},
    {softmax_logits_bwd_slice_kernel<256, 4>, 256, 1024},
    {softmax_logits_bwd_slice_kernel<256, 8>, 256, 2048},
    {softmax_logits_bwd_slice_kernel<512, 8>, 512, 4096},
    {softmax_logits_bwd_slice_kernel<1024, 8>, 1024, 8192},
};

constexpr int64_t kFwdCapacity = 16384;
constexpr int64_t kBwdCapacity = 8192;

}  // namespace

size_t softmax_workspace(int op, int64_t rows, int64_t cols, int variant, int split,
                         int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  const int64_t cap = op == CREDIT_OP_SOFTMAX_FWD ? kFwdCapacity : kBwdCapacity;
  if (resolve(&c, cols, cols % 4 == 0, cap, "softmax", &p) != CREDIT_OK) return 0;
  const int k = op == CREDIT_OP_SOFTMAX_BWD ? 1 : 2;
  return slice_workspace(rows, p, k, cu_count);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_softmax_fwd_f32(const float* x, float* p, float* rowmax, float* lse,
                                      int64_t rows, int64_t cols, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(p, "p", rows));
  CREDIT_TRY(check_row_ptr(rowmax, "rowmax", rows));
  CREDIT_TRY(check_row_ptr(lse, "lse", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, 4, "x"));
  CREDIT_TRY(check_aligned(p, 4, "p"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols, vec_ok(cols, {x, p}), kFwdCapacity, "softmax_fwd", &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec_ok(cols, {x, p}))
      softmax_fwd_read_kernel<256, true><<<r, 256, 0, stream>>>(x, p, rowmax, lse, c);
    else
      softmax_fwd_read_kernel<256, false><<<r, 256, 0, stream>>>(x, p, rowmax, lse, c);
    return check_launch("softmax_fwd_read_kernel");
  }
  const Pick<FwdFn>* pk = pick_for(kFwd, plan.chunk);
  return launch_slices<FwdFn>(
      cfg, rows, plan, pk, 2, 1, "softmax_fwd_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, x, p, rowmax, lse,
                           c, static_cast<int>(plan.chunk), plan.members,
                           static_cast<int>(rows), sa);
      });
}

extern "C" int credit_softmax_bwd_f32(const float* p, const float* dy, float* dx, int64_t rows,
                                      int64_t cols, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(p, "p", rows));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(p, 4, "p"));
  CREDIT_TRY(check_aligned(dy, 4, "dy"));
  CREDIT_TRY(check_aligned(dx, 4, "dx"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {p, dy, dx});
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols, vec, kBwdCapacity, "softmax_bwd", &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      softmax_bwd_read_kernel<256, true><<<r, 256, 0, stream>>>(p, dy, dx, c);
    else
      softmax_bwd_read_kernel<256, false><<<r, 256, 0, stream>>>(p, dy, dx, c);
    return check_launch("softmax_bwd_read_kernel");
  }
  const Pick<BwdFn>* pk = pick_for(kBwd, plan.chunk);
  return launch_slices<BwdFn>(
      cfg, rows, plan, pk, 1, 1, "softmax_bwd_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, p, dy, dx, c,
                           static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows),
                           sa);
      });
}

extern "C" int credit_softmax_logits_bwd_f32(const float* logits, const float* dy, float* dx,
                                             int64_t rows, int64_t cols,
                                             const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(logits, "logits", rows));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(logits, 4, "logits"));
  CREDIT_TRY(check_aligned(dy, 4, "dy"));
  CREDIT_TRY(check_aligned(dx, 4, "dx"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {logits, dy, dx});
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols, vec, kBwdCapacity, "softmax_logits_bwd", &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      softmax_logits_bwd_read_kernel<256, true><<<r, 256, 0, stream>>>(logits, dy, dx, c);
    else
      softmax_logits_bwd_read_kernel<256, false><<<r, 256, 0, stream>>>(logits, dy, dx, c);
    return check_launch("softmax_logits_bwd_read_kernel");
  }
  const Pick<BwdFn>* pk = pick_for(kLogits, plan.chunk);
  return launch_slices<BwdFn>(
      cfg, rows, plan, pk, 2, 2, "softmax_logits_bwd_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, logits, dy, dx,
                           c, static_cast<int>(plan.chunk), plan.members,
                           static_cast<int>(rows), sa);
      });
}
