// Row-wise int8 quantisation, fp32 in: the reference workload rowwise_quant
// (dsmem_eval/workloads.py:150-154; src/workloads/rowwise_quant.cu:260-363).
//
//   max_abs = max_j |x_j|
//   inv     = max_abs > 0 ? (1 / max_abs) * 127 : 0   (two fp32 roundings:
//             torch evaluates the reference's 127.0 / max_abs as
//             reciprocal * 127)
//   q_j     = int8(clamp(rint(x_j * inv), -127, 127))  (round half to even)
//   scale   = max_abs / 127                            (one fp32 division)
//
// Every step is an exact fp32 operation, so q and scale are bit-exact
// against the reference's PyTorch function for finite inputs.
//
// Variants (rows of f32x4 vectors, as the softmax kernels):
//  - STAGED: one workgroup per row, the row held in VGPRs (up to 16 f32x4
//            per lane): one HBM read of x, one write of q.
//  - SPLIT : P members hold 1/P of the row each and exchange their partial
//            maximum (one stage, exact: fp32 bits); a co-resident wave of
//            ticketed groups looping over the rows.
//  - READ  : one workgroup per row, max pass then quantise pass (x read
//            twice), for any width and alignment.
// Algorithmic traffic per row: 4*cols (x) + cols (q) + 4 (scale) bytes.
#include "api_internal.hpp"
#include "common.hpp"
#include "slices.hpp"

namespace credit {
namespace {

using namespace slices;

__device__ __forceinline__ float absmax4(f32x4 v) {
  return fmax_nan(fmax_nan(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                  fmax_nan(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
}

__device__ __forceinline__ uint32_t quant1(float x, float inv) {
  float q = __builtin_rintf(x * inv);
  q = __builtin_fminf(127.0f, __builtin_fmaxf(-127.0f, q));
  return static_cast<uint32_t>(static_cast<int32_t>(q)) & 0xFFu;
}

// Four int8 codes packed little-endian (element 0 in the low byte).
__device__ __forceinline__ uint32_t quant4(f32x4 v, float inv) {
  return quant1(v.x, inv) | (quant1(v.y, inv) << 8) | (quant1(v.z, inv) << 16) |
         (quant1(v.w, inv) << 24);
}

// inv as the reference's torch function computes it.
__device__ __forceinline__ float inv_scale(float max_abs) {
  return max_abs > 0.0f ? (1.0f / max_abs) * 127.0f : 0.0f;
}

template <int THREADS, int VPT>
__device__ __forceinline__ void rowwise_quant_slice_kernel_body(
    const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scale, int cols,
    int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 1, chunk, cols >> 2, sa);
  for (int row = sl.row; row < rows; row += sl.step) {
    const int tid = opaque_lane_index();
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + static_cast<size_t>(row) * cols) + sl.v0;
    f32x4 v[VPT];
    // (p + k*THREADS)[tid]: a uniform base per k and one lane offset, so no
    // per-k lane address stays live across the row loop.
#pragma unroll
    for (int k = 0; k < VPT; ++k)
      v[k] = tid < sl.vlen - k * THREADS ? load_nt(&(xr + k * THREADS)[tid]) : f32x4{0, 0, 0, 0};
    float lm = 0.0f;  // |x| >= 0: 0 is the identity
#pragma unroll
    for (int k = 0; k < VPT; ++k) lm = fmax_nan(lm, absmax4(v[k]));
    float m = block_reduce<NW>(lm, MaxOp{}, mred);
    if (members > 1) {
      if (threadIdx.x == 0) split_publish(g, 0, static_cast<double>(m));
      split_exchange(g);
      m = static_cast<float>(split_get(g, 0, 0));
      for (int i = 1; i < g.members; ++i) m = fmax_nan(m, static_cast<float>(split_get(g, 0, i)));
    }
    const float inv = inv_scale(m);
    uint32_t* qr = reinterpret_cast<uint32_t*>(q + static_cast<size_t>(row) * cols) + sl.v0;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
      if (tid < sl.vlen - k * THREADS)
        __builtin_nontemporal_store(quant4(v[k], inv), &(qr + k * THREADS)[tid]);
    if (sl.member == 0 && threadIdx.x == 0) scale[row] = m / 127.0f;
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void rowwise_quant_slice_kernel(
    const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scale, int cols,
    int chunk, int members, int rows, SplitArgs sa) {
  rowwise_quant_slice_kernel_body<THREADS, VPT>(x, q, scale, cols, chunk, members, rows, sa);
  split_leave(sa);
}

// Two passes over the row; VEC: f32x4 loads and 4-byte q stores.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void rowwise_quant_read_kernel(
    const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scale, int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ float mred[NW];
  const int tid = threadIdx.x;
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  float lm = 0.0f;
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    int i = tid;
    for (; i + THREADS < nvec; i += 2 * THREADS)
      lm = fmax_nan(lm, fmax_nan(absmax4(load_nt(xv + i)), absmax4(load_nt(xv + i + THREADS))));
    for (; i < nvec; i += THREADS) lm = fmax_nan(lm, absmax4(load_nt(xv + i)));
  } else {
    for (int c = tid; c < cols; c += THREADS) lm = fmax_nan(lm, __builtin_fabsf(x[off + c]));
  }
  const float m = block_reduce<NW>(lm, MaxOp{}, mred);
  const float inv = inv_scale(m);
  if (VEC) {
    const int nvec = cols >> 2;
    const f32x4* xv = reinterpret_cast<const f32x4*>(x + off);
    uint32_t* qv = reinterpret_cast<uint32_t*>(q + off);
    for (int i = tid; i < nvec; i += THREADS) __builtin_nontemporal_store(quant4(load_nt(xv + i), inv), qv + i);
  } else {
    for (int c = tid; c < cols; c += THREADS)
      q[off + c] = static_cast<int8_t>(static_cast<int32_t>(quant1(x[off + c], inv) << 24) >> 24);
  }
  if (tid == 0) scale[blockIdx.x] = m / 127.0f;
}

using QuantFn = void (*)(const float*, int8_t*, float*, int, int, int, int, SplitArgs);

// One tensor staged: up to 16 f32x4 per lane (as the softmax forward).
const Pick<QuantFn> kQuant[] = {
    {rowwise_quant_slice_kernel<64, 4>, 64, 256},
    {rowwise_quant_slice_kernel<128, 4>, 128, 512},
    {rowwise_quant_slice_kernel<256, 4>, 256, 1024},
    {rowwise_quant_slice_kernel<256, 8>, 256, 2048},
    {rowwise_quant_slice_kernel<512, 8>, 512, 4096},
    {rowwise_quant_slice_kernel<1024, 8>, 1024, 8192},
    {rowwise_quant_slice_kernel<1024, 16>, 1024, 16384},
};
constexpr int64_t kQuantCapacity = 16384;

bool quant_vec(int64_t cols, const float* x, const int8_t* q) {
  return vec_ok(cols, {x}) && reinterpret_cast<uintptr_t>(q) % 4 == 0;
}

}  // namespace

size_t rowwise_quant_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (resolve(&c, cols, cols % 4 == 0, kQuantCapacity, "rowwise_quant", &p) != CREDIT_OK) return 0;
  return slice_workspace(rows, p, 1, cu_count);
}

}  // namespace credit

using namespace credit;

extern "C" int credit_rowwise_quant_f32(const float* x, int8_t* q, float* scale, int64_t rows,
                                        int64_t cols, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(q, "q", rows));
  CREDIT_TRY(check_row_ptr(scale, "scale", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, 4, "x"));
  CREDIT_TRY(check_aligned(scale, 4, "scale"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  const bool vec = quant_vec(cols, x, q);
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols, vec, kQuantCapacity, "rowwise_quant", &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const unsigned r = static_cast<unsigned>(rows);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      rowwise_quant_read_kernel<256, true><<<r, 256, 0, stream>>>(x, q, scale, c);
    else
      rowwise_quant_read_kernel<256, false><<<r, 256, 0, stream>>>(x, q, scale, c);
    return check_launch("rowwise_quant_read_kernel");
  }
  const Pick<QuantFn>* pk = pick_for(kQuant, plan.chunk);
  return launch_slices<QuantFn>(
      cfg, rows, plan, pk, 1, 1, "rowwise_quant_slice_kernel",
      [&](unsigned grid, const SplitArgs& sa) {
        hipLaunchKernelGGL(pk->fn, dim3(grid), dim3(pk->threads), 0, stream, x, q, scale, c,
                           static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows),
                           sa);
      });
}
