// C2: LayerNorm forward, bf16 in/out with fp32 statistics.
//
// y = (x - mean) * rstd * gamma + beta,  mean = sum(x)/N,
// var = sum((x - mean)^2)/N (the statistics of dsmem_eval/workloads.py:54-56),
// rstd = 1/sqrt(var + eps).  The reference only has the backward kernel; its
// statistics pass is src/workloads/layernorm_backward.cu:286-295.
//
// Statistics of a row held in registers: one pass forms sum(x) and sum(x^2)
// with v_dot2_f32_bf16 (two bf16 elements per instruction: x.lo*1 + x.hi*1
// and x.lo^2 + x.hi^2, products exact in fp32), lane partials in fp32 over at
// most 64 elements, then fp64 across lanes and waves.  var = E[x^2] - mean^2
// then carries a relative error of about 64 ulp(fp32) * E[x^2] / var, so the
// one-pass value is kept only when mean^2 <= var / 4 (E[x^2] <= 1.25 var:
// rstd within ~2e-6); otherwise -- rows with a large offset, constant rows --
// a second pass over the same registers sums (x - mean)^2, the two-pass
// form.  The branch is workgroup-uniform.
//
// Variants:
//  - STAGED: one workgroup per row, the row held in VGPRs as packed bf16
//            (VPT dwordx4 per lane), statistics and output pass from
//            registers: one HBM read of x, one write of y.
//  - PIPE  : (AUTO on tall matrices with 2049..4096 vectors per row) one
//            persistent workgroup of 512 lanes per CU, gamma and beta staged
//            once in LDS, and a two-row register pipeline: the loads of row
//            r+G are in flight while row r is reduced and stored.  Measured
//            at 2048x32768, settled: 45.2 us against 47.5 us for the earlier
//            1024-lane three-row pipeline with two-pass statistics (47.6 us
//            for 512 lanes with two-pass statistics: at two waves per SIMD
//            the VALU work of the second pass shows).
//  - READ  : one workgroup per row streaming the row three times (sum, sum of
//            squared deviations, output), for shapes the staged layout does
//            not cover (cols not a multiple of 8, misaligned rows, very wide
//            rows).
// Algorithmic traffic per row: 2*cols (x) + 2*cols (y) + 8 (mean, rstd) bytes,
// plus 4*cols once for gamma and beta.
#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

__device__ __forceinline__ float sqdev8(u32x4 v, float mu) {
  float a = bf16_lo(v.x) - mu, b = bf16_hi(v.x) - mu;
  float c = bf16_lo(v.y) - mu, d = bf16_hi(v.y) - mu;
  float e = bf16_lo(v.z) - mu, f = bf16_hi(v.z) - mu;
  float g = bf16_lo(v.w) - mu, h = bf16_hi(v.w) - mu;
  return ((a * a + b * b) + (c * c + d * d)) + ((e * e + f * f) + (g * g + h * h));
}

__device__ __forceinline__ uint32_t norm2(uint32_t xv, uint32_t gv, uint32_t bv,
                                          float mu, float rs) {
  const float lo = (bf16_lo(xv) - mu) * rs * bf16_lo(gv) + bf16_lo(bv);
  const float hi = (bf16_hi(xv) - mu) * rs * bf16_hi(gv) + bf16_hi(bv);
  return pack_bf16x2(lo, hi);
}

__device__ __forceinline__ u32x4 norm8(u32x4 xv, u32x4 gv, u32x4 bv, float mu,
                                       float rs) {
  return u32x4{norm2(xv.x, gv.x, bv.x, mu, rs), norm2(xv.y, gv.y, bv.y, mu, rs),
               norm2(xv.z, gv.z, bv.z, mu, rs), norm2(xv.w, gv.w, bv.w, mu, rs)};
}

struct RowStats {
  double mean;
  float mu;  // mean rounded to fp32: the centre of the output pass
  float rs;
};

// Statistics of one row whose 8-element bf16 vectors sit in v (lanes past
// the row's end hold zeros).  slots is [3][NW] LDS, not reused by this
// workgroup before a later barrier.  Contains one barrier (two on the
// two-pass branch).
template <int THREADS, int VPT>
__device__ __forceinline__ RowStats row_stats(const u32x4 (&v)[VPT], int cols, float eps,
                                              double (*slots)[THREADS / kWave], int tid) {
  constexpr int NW = THREADS / kWave;
  constexpr uint32_t kOnes = 0x3f803f80u;  // bf16 (1.0, 1.0)
  float s0 = 0.0f, s1 = 0.0f, q0 = 0.0f, q1 = 0.0f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    s0 = dot2_bf16(v[k].x, kOnes, s0);
    q0 = dot2_bf16(v[k].x, v[k].x, q0);
    s1 = dot2_bf16(v[k].y, kOnes, s1);
    q1 = dot2_bf16(v[k].y, v[k].y, q1);
    s0 = dot2_bf16(v[k].z, kOnes, s0);
    q0 = dot2_bf16(v[k].z, v[k].z, q0);
    s1 = dot2_bf16(v[k].w, kOnes, s1);
    q1 = dot2_bf16(v[k].w, v[k].w, q1);
  }
  double sums[2] = {static_cast<double>(s0) + s1, static_cast<double>(q0) + q1};
  block_reduce_sum_f64_multi<NW, 2>(sums, slots);
  RowStats st;
  st.mean = sums[0] / cols;
  st.mu = static_cast<float>(st.mean);
  double var = sums[1] / cols - st.mean * st.mean;
  if (st.mean * st.mean > 0.25 * var) {
    const int nvec = cols >> 3;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const float d = sqdev8(v[k], st.mu);
      q += tid + k * THREADS < nvec ? d : 0.0f;
    }
    const double sq = block_reduce_sum_f64<NW>(static_cast<double>(q), slots[2]);
    // Deviations were taken from the fp32-rounded mean; the variance about
    // the exact mean differs by (mu - mean)^2, which the correction removes.
    const double dmu = static_cast<double>(st.mu) - st.mean;
    var = sq / cols - dmu * dmu;
  }
  st.rs = static_cast<float>(1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps));
  return st;
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void layernorm_fwd_staged_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int cols,
    float eps) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[3][NW];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + static_cast<size_t>(row) * cols);
  u32x4 v[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int idx = tid + k * THREADS;
    v[k] = idx < nvec ? load_nt(xr + idx) : u32x4{0, 0, 0, 0};
  }
  const RowStats st = row_stats<THREADS, VPT>(v, cols, eps, red, tid);
  const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
  const u32x4* br = reinterpret_cast<const u32x4*>(beta);
  u32x4* yr = reinterpret_cast<u32x4*>(y + static_cast<size_t>(row) * cols);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int idx = tid + k * THREADS;
    if (idx < nvec) store_nt(yr + idx, norm8(v[k], gr[idx], br[idx], st.mu, st.rs));
  }
  if (tid == 0) {
    mean_out[row] = static_cast<float>(st.mean);
    rstd_out[row] = st.rs;
  }
}

// ------------------------------------------------------------------ PIPE --
// Row loads and stores go through buffer resources: a row past the end has
// num_records 0 and reads zeros, a lane past the row's end reads zeros and
// its store is dropped, all without branches.  With no memory operation
// under a branch the waitcnt pass counts the operations in flight exactly and
// waits for the oldest row only (a load under a branch made it drain every
// load in flight, vmcnt(0)).
constexpr int kPipeThreads = 512;
constexpr int kPipeVpt = 8;
constexpr int kPipeVec = kPipeThreads * kPipeVpt;  // 16-byte vectors per row, at most
constexpr size_t kPipeLds = static_cast<size_t>(kPipeVec) * 2 * 16;  // gamma + beta, 128 KiB

template <int THREADS, int VPT>
__device__ __forceinline__ void pipe_load(u32x4 (&v)[VPT], const uint16_t* x, int row, int rows,
                                          int cols, int tid) {
  const buffer_rsrc_t r = make_rsrc(x + static_cast<size_t>(row < rows ? row : 0) * cols,
                                    row < rows ? static_cast<uint32_t>(cols) * 2u : 0u);
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    v[k] = buffer_load_nt(r, static_cast<uint32_t>(tid + k * THREADS) * 16u);
}

// Statistics and output of one row held in v.  red is this row's [3][NW]
// slot set; the pipeline alternates two sets, so a slot is rewritten only
// after the next row's barrier.  gb holds gamma vectors [THREADS * VPT],
// then beta vectors.
template <int THREADS, int VPT>
__device__ __forceinline__ void pipe_row(const u32x4 (&v)[VPT], const u32x4* gb, uint16_t* y,
                                         float* mean_out, float* rstd_out, int row, int cols,
                                         float eps, double (*red)[THREADS / kWave], int tid) {
  const RowStats st = row_stats<THREADS, VPT>(v, cols, eps, red, tid);
  const buffer_rsrc_t yr = make_rsrc(y + static_cast<size_t>(row) * cols,
                                     static_cast<uint32_t>(cols) * 2u);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int idx = tid + k * THREADS;
    buffer_store_nt(yr, static_cast<uint32_t>(idx) * 16u,
                    norm8(v[k], gb[idx], gb[THREADS * VPT + idx], st.mu, st.rs));
  }
  // Lane 0 writes the statistics (4-byte resources; other lanes' offsets
  // fall outside them).  The builtin takes the bits of the value.
  const uint32_t off = static_cast<uint32_t>(tid) * 4u;
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(static_cast<float>(st.mean)),
                                        make_rsrc(mean_out + row, 4u), off, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(st.rs), make_rsrc(rstd_out + row, 4u),
                                        off, 0, 0);
}

// Workgroup g of G handles rows g, g + G, g + 2G, ...; cols % 8 == 0,
// cols / 8 <= THREADS * VPT, 16-byte aligned rows, gamma and beta.
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void layernorm_fwd_pipe_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int rows, int cols,
    float eps) {
  constexpr int NW = THREADS / kWave;
  extern __shared__ u32x4 gb[];
  __shared__ double red[2][3][NW];
  const int tid = threadIdx.x;
  const int G = gridDim.x;
  int row = blockIdx.x;
  // gamma and beta first: the wait before they are written to LDS then
  // leaves the first row's loads in flight.
  const buffer_rsrc_t grs = make_rsrc(gamma, static_cast<uint32_t>(cols) * 2u);
  const buffer_rsrc_t brs = make_rsrc(beta, static_cast<uint32_t>(cols) * 2u);
  u32x4 gv[VPT], bv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    gv[k] = buffer_load(grs, static_cast<uint32_t>(tid + k * THREADS) * 16u);
    bv[k] = buffer_load(brs, static_cast<uint32_t>(tid + k * THREADS) * 16u);
  }
  u32x4 v0[VPT], v1[VPT];
  pipe_load<THREADS, VPT>(v0, x, row, rows, cols, tid);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    gb[tid + k * THREADS] = gv[k];
    gb[THREADS * VPT + tid + k * THREADS] = bv[k];
  }
  __syncthreads();
  // Unrolled by two so that the register buffers alternate without copies.
  for (; row < rows; row += 2 * G) {
    pipe_load<THREADS, VPT>(v1, x, row + G, rows, cols, tid);
    pipe_row<THREADS, VPT>(v0, gb, y, mean_out, rstd_out, row, cols, eps, red[0], tid);
    if (row + G >= rows) break;
    pipe_load<THREADS, VPT>(v0, x, row + 2 * G, rows, cols, tid);
    pipe_row<THREADS, VPT>(v1, gb, y, mean_out, rstd_out, row + G, cols, eps, red[1], tid);
  }
}

template <int THREADS>
__global__ __launch_bounds__(THREADS) void layernorm_fwd_read_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int cols,
    float eps) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red0[NW];
  __shared__ double red1[NW];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + static_cast<size_t>(row) * cols;
  double s = 0.0;
  for (int c = tid; c < cols; c += THREADS) s += bf16_to_f32(xr[c]);
  const double total = block_reduce_sum_f64<NW>(s, red0);
  const double mean = total / cols;
  double q = 0.0;
  for (int c = tid; c < cols; c += THREADS) {
    const double d = bf16_to_f32(xr[c]) - mean;
    q += d * d;
  }
  const double var = block_reduce_sum_f64<NW>(q, red1) / cols;
  const float rs = static_cast<float>(1.0 / __builtin_sqrt(var + eps));
  const float mu = static_cast<float>(mean);
  uint16_t* yr = y + static_cast<size_t>(row) * cols;
  for (int c = tid; c < cols; c += THREADS) {
    const float v = (bf16_to_f32(xr[c]) - mu) * rs * bf16_to_f32(gamma[c]) +
                    bf16_to_f32(beta[c]);
    yr[c] = f32_to_bf16(v);
  }
  if (tid == 0) {
    mean_out[row] = mu;
    rstd_out[row] = rs;
  }
}

using StagedFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*,
                          uint16_t*, float*, float*, int, float);

struct StagedPick {
  StagedFn fn;
  int threads;
  int max_vec;  // threads * VPT
};

// Row widths the register-staged kernel covers, smallest footprint first.
// VPT stays at 4-8 dwordx4 per lane; deeper register staging makes the
// compiler hoist the gamma/beta loads of the output loop and spill.
const StagedPick kStaged[] = {
    {layernorm_fwd_staged_kernel<64, 4>, 64, 256},
    {layernorm_fwd_staged_kernel<128, 4>, 128, 512},
    {layernorm_fwd_staged_kernel<256, 4>, 256, 1024},
    {layernorm_fwd_staged_kernel<256, 8>, 256, 2048},
    {layernorm_fwd_staged_kernel<512, 8>, 512, 4096},
    {layernorm_fwd_staged_kernel<1024, 8>, 1024, 8192},
};

}  // namespace
}  // namespace credit

using namespace credit;

extern "C" int credit_layernorm_fwd_bf16(const uint16_t* x, const uint16_t* gamma,
                                         const uint16_t* beta, uint16_t* y,
                                         float* mean, float* rstd, int64_t rows,
                                         int64_t cols, float eps,
                                         const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(gamma, "gamma"));
  CREDIT_TRY(check_ptr(beta, "beta"));
  CREDIT_TRY(check_row_ptr(y, "y", rows));
  CREDIT_TRY(check_row_ptr(mean, "mean", rows));
  CREDIT_TRY(check_row_ptr(rstd, "rstd", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, 2, "x"));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps >= 0.0f))
    return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (rows == 0) return CREDIT_OK;
  int variant = cfg_variant(cfg);
  if (variant == CREDIT_VARIANT_SPLIT)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_fwd: split-row variant not built");
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const bool vec_ok = (cols % 8 == 0) &&
                      reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(beta) % 16 == 0;
  const int64_t nvec = cols / 8;
  const StagedPick* pick = nullptr;
  if (vec_ok) {
    for (const StagedPick& p : kStaged) {
      if (nvec <= p.max_vec) {
        pick = &p;
        break;
      }
    }
  }
  if (variant == CREDIT_VARIANT_STAGED && pick == nullptr)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_fwd staged variant needs cols %% 8 == 0, "
                     "16-byte aligned buffers and cols <= 65536");
  if (variant == CREDIT_VARIANT_READ || pick == nullptr) {
    layernorm_fwd_read_kernel<256><<<dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                                     stream>>>(x, gamma, beta, y, mean, rstd, c, eps);
    return check_launch("layernorm_fwd_read_kernel");
  }
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  // AUTO: the pipeline once every CU has at least two rows to overlap.
  if (variant == CREDIT_VARIANT_AUTO && nvec > kPipeVec / 2 && nvec <= kPipeVec &&
      rows >= 2 * static_cast<int64_t>(props->cu_count) &&
      rows <= INT32_MAX - 2 * static_cast<int64_t>(props->cu_count)) {  // row + 2G fits an int
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(layernorm_fwd_pipe_kernel<kPipeThreads, kPipeVpt>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kPipeLds));
    if (attr != hipSuccess) return hip_failure(attr, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    hipLaunchKernelGGL((layernorm_fwd_pipe_kernel<kPipeThreads, kPipeVpt>),
                       dim3(static_cast<unsigned>(props->cu_count)), dim3(kPipeThreads), kPipeLds,
                       stream, x, gamma, beta, y, mean, rstd, static_cast<int>(rows), c, eps);
    return check_launch("layernorm_fwd_pipe_kernel");
  }
  hipLaunchKernelGGL(pick->fn, dim3(static_cast<unsigned>(rows)), dim3(pick->threads),
                     0, stream, x, gamma, beta, y, mean, rstd, c, eps);
  return check_launch("layernorm_fwd_staged_kernel");
}
