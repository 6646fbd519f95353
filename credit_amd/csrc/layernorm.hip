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
  // Each vector passes through an empty asm before it is normalised, so the
  // compiler cannot unpack every vector (and read its gamma and beta) ahead
  // of the first store: 235 -> 113 VGPRs, C2 -0.5 to -1.5 us (alternating
  // runs on two boxes).
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int idx = tid + k * THREADS;
    u32x4 xv = v[k];
    __asm__ volatile("" : "+v"(xv));
    buffer_store_nt(yr, static_cast<uint32_t>(idx) * 16u,
                    norm8(xv, gb[idx], gb[THREADS * VPT + idx], st.mu, st.rs));
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

// ----------------------------------------------------------------- SPLIT --
// P = members > 1 workgroups per row (one co-resident wave of ticketed
// groups, each looping over rows group, group + G, ...), every member
// holding a slice of VPT vectors per lane in registers.  Stage 1 exchanges
// the slice's (sum x, sum x^2); every member forms the same totals in member
// order, so every member takes the same branch: the one-pass variance when
// mean^2 <= var/4, else a second stage exchanging the slice's sum of squared
// deviations about the mean.  Partials travel as fp32 (the block sums before
// them are fp64).  One HBM read of x, one write of y.
template <int THREADS, int VPT>
__device__ __forceinline__ void layernorm_fwd_slice_kernel_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int cols, int chunk,
    int members, int rows, float eps, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  constexpr uint32_t kOnes = 0x3f803f80u;  // bf16 (1.0, 1.0)
  __shared__ double red[2][3][NW];
  SplitGroup g = split_join(sa, members, 2);
  const int step = static_cast<int>(sa.grid) / members;
  const int nvec = cols >> 3;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  const buffer_rsrc_t grs = make_rsrc(gamma + 8 * static_cast<size_t>(v0), slice_bytes);
  const buffer_rsrc_t brs = make_rsrc(beta + 8 * static_cast<size_t>(v0), slice_bytes);
  int parity = 0;
  for (int row = g.group; row < rows; row += step, parity ^= 1) {
    double (*slots)[NW] = red[parity];
    const size_t off = static_cast<size_t>(row) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t xrs = make_rsrc(x + off, slice_bytes);
    u32x4 v[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) v[k] = buffer_load_nt(xrs, lane_off + k * kStride);
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
    if (threadIdx.x == 0) {
      split_publish(g, 0, sums[0]);
      split_publish(g, 1, sums[1]);
    }
    split_exchange(g, 2);
    const double mean = split_sum(g, 0) / cols;
    const float mu = static_cast<float>(mean);
    double var = split_sum(g, 1) / cols - mean * mean;
    if (mean * mean > 0.25 * var) {
      float q = 0.0f;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const float d = sqdev8(v[k], mu);
        q += lane_off + k * kStride < slice_bytes ? d : 0.0f;
      }
      const double sq = block_reduce_sum_f64<NW>(static_cast<double>(q), slots[2]);
      if (threadIdx.x == 0) split_publish(g, 0, sq);
      split_exchange(g, 1);
      const double dmu = static_cast<double>(mu) - mean;
      var = split_sum(g, 0) / cols - dmu * dmu;
    }
    const float rs = static_cast<float>(1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps));
    const buffer_rsrc_t yrs = make_rsrc(y + off, slice_bytes);
    // Output in groups of four vectors: gamma and beta of one group in
    // flight at a time (the compiler otherwise hoists all of them, 8 VGPRs
    // per vector, above the first store).
#pragma unroll
    for (int k0 = 0; k0 < VPT; k0 += 4) {
      u32x4 gv[4], bv[4];
#pragma unroll
      for (int j = 0; j < 4 && k0 + j < VPT; ++j) {
        gv[j] = buffer_load(grs, lane_off + (k0 + j) * kStride);
        bv[j] = buffer_load(brs, lane_off + (k0 + j) * kStride);
      }
#pragma unroll
      for (int j = 0; j < 4 && k0 + j < VPT; ++j)
        buffer_store_nt(yrs, lane_off + (k0 + j) * kStride, norm8(v[k0 + j], gv[j], bv[j], mu, rs));
      __builtin_amdgcn_sched_barrier(0);
    }
    if (g.member == 0 && threadIdx.x == 0) {
      mean_out[row] = static_cast<float>(mean);
      rstd_out[row] = rs;
    }
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void layernorm_fwd_slice_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int cols, int chunk,
    int members, int rows, float eps, SplitArgs sa) {
  layernorm_fwd_slice_kernel_body<THREADS, VPT>(x, gamma, beta, y, mean_out, rstd_out, cols, chunk, members, rows, eps, sa);
  split_leave(sa);
}

// ------------------------------------------------------------------ READ --
// One workgroup per row streaming it three times (sum; squared deviations
// about the mean; output).  VEC: 16-byte vectors of 8 bf16, four in flight
// per lane (cols % 8 == 0, 16-byte aligned x, y, gamma, beta); else 2-byte
// element loads for any width and alignment.
template <int THREADS, bool VEC>
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
  uint16_t* yr = y + static_cast<size_t>(row) * cols;
  const int nvec = VEC ? cols >> 3 : 0;
  const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
  double s = 0.0;
  if (VEC) {
    constexpr uint32_t kOnes = 0x3f803f80u;
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS) {
      const u32x4 a = xv[i], b = xv[i + THREADS], c = xv[i + 2 * THREADS],
                  d = xv[i + 3 * THREADS];
      float t = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t = dot2_bf16(a[e], kOnes, t);
        t = dot2_bf16(b[e], kOnes, t);
        t = dot2_bf16(c[e], kOnes, t);
        t = dot2_bf16(d[e], kOnes, t);
      }
      s += t;
    }
    for (; i < nvec; i += THREADS) {
      const u32x4 a = xv[i];
      float t = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) t = dot2_bf16(a[e], kOnes, t);
      s += t;
    }
  } else {
    for (int c = tid; c < cols; c += THREADS) s += bf16_to_f32(xr[c]);
  }
  const double total = block_reduce_sum_f64<NW>(s, red0);
  const double mean = total / cols;
  const float mu = static_cast<float>(mean);
  double q = 0.0;
  if (VEC) {
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS)
      q += static_cast<double>((sqdev8(xv[i], mu) + sqdev8(xv[i + THREADS], mu)) +
                               (sqdev8(xv[i + 2 * THREADS], mu) + sqdev8(xv[i + 3 * THREADS], mu)));
    for (; i < nvec; i += THREADS) q += static_cast<double>(sqdev8(xv[i], mu));
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const double d = bf16_to_f32(xr[c]) - mean;
      q += d * d;
    }
  }
  // Deviations taken from the fp32 mean: remove (mu - mean)^2 (VEC), or
  // exact fp64 deviations (scalar path).
  const double dmu = VEC ? static_cast<double>(mu) - mean : 0.0;
  const double var = block_reduce_sum_f64<NW>(q, red1) / cols - dmu * dmu;
  const float rs = static_cast<float>(1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps));
  if (VEC) {
    const u32x4* gv = reinterpret_cast<const u32x4*>(gamma);
    const u32x4* bv = reinterpret_cast<const u32x4*>(beta);
    u32x4* yv = reinterpret_cast<u32x4*>(yr);
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS) {
      const u32x4 a = load_nt(xv + i), b = load_nt(xv + i + THREADS),
                  c = load_nt(xv + i + 2 * THREADS), d = load_nt(xv + i + 3 * THREADS);
      store_nt(yv + i, norm8(a, gv[i], bv[i], mu, rs));
      store_nt(yv + i + THREADS, norm8(b, gv[i + THREADS], bv[i + THREADS], mu, rs));
      store_nt(yv + i + 2 * THREADS,
               norm8(c, gv[i + 2 * THREADS], bv[i + 2 * THREADS], mu, rs));
      store_nt(yv + i + 3 * THREADS,
               norm8(d, gv[i + 3 * THREADS], bv[i + 3 * THREADS], mu, rs));
    }
    for (; i < nvec; i += THREADS) store_nt(yv + i, norm8(load_nt(xv + i), gv[i], bv[i], mu, rs));
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float v = (bf16_to_f32(xr[c]) - mu) * rs * bf16_to_f32(gamma[c]) +
                      bf16_to_f32(beta[c]);
      yr[c] = f32_to_bf16(v);
    }
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

using SliceFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*,
                        float*, int, int, int, int, float, SplitArgs);
struct SlicePick {
  SliceFn fn;
  int threads;
  int max_vec;
};
// Member slices of the SPLIT kernel, smallest footprint first.
const SlicePick kSlice[] = {
    {layernorm_fwd_slice_kernel<256, 4>, 256, 1024},
    {layernorm_fwd_slice_kernel<256, 8>, 256, 2048},
    {layernorm_fwd_slice_kernel<512, 8>, 512, 4096},
};
// No 1024-lane slice shape: at 128 VGPRs per lane its row, exchange and
// output state spill to scratch (the counters saw 2.4x the HBM bytes).
constexpr int64_t kSliceCapacity = 8192;       // vectors of the STAGED kernel
constexpr int64_t kSplitSliceCapacity = 4096;  // vectors per SPLIT member
constexpr int kMaxSliceMembers = kMaxExchangeValues / 2;  // (sum, sum of squares)

struct Plan {
  int variant;
  int members;
  int64_t chunk;
};

// READ: explicit, or shapes without the 16-byte vector layout.  STAGED /
// pipeline: rows of at most 65536 columns.  SPLIT: explicit, or AUTO on a
// wider row, with just enough members that every slice fits one workgroup.
int resolve(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  const int variant = cfg_variant(cfg);
  const int64_t nvec = cols / 8;
  if (variant == CREDIT_VARIANT_READ || (!vec && variant == CREDIT_VARIANT_AUTO)) {
    *plan = Plan{CREDIT_VARIANT_READ, 1, nvec};
    return CREDIT_OK;
  }
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_fwd staged/split variants need cols %% 8 == 0 and 16-byte "
                     "aligned buffers");
  if (variant == CREDIT_VARIANT_STAGED || (variant == CREDIT_VARIANT_AUTO && nvec <= kSliceCapacity)) {
    if (nvec > kSliceCapacity)
      return set_error(CREDIT_ERR_UNSUPPORTED, "layernorm_fwd staged variant holds at most %lld columns",
                       static_cast<long long>(kSliceCapacity * 8));
    *plan = Plan{CREDIT_VARIANT_STAGED, 1, nvec};
    return CREDIT_OK;
  }
  int p = variant == CREDIT_VARIANT_SPLIT ? cfg_split(cfg) : 0;
  if (p == 0) p = static_cast<int>((nvec + kSplitSliceCapacity - 1) / kSplitSliceCapacity);
  if (p < 2) p = 2;
  if (p > nvec) p = static_cast<int>(nvec);
  const int64_t chunk = (nvec + p - 1) / p;
  const int members = static_cast<int>((nvec + chunk - 1) / chunk);
  if (chunk > kSplitSliceCapacity)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_fwd split %d leaves %lld vectors per member (at most %lld)", p,
                     static_cast<long long>(chunk), static_cast<long long>(kSplitSliceCapacity));
  if (members > kMaxSliceMembers)
    return set_error(CREDIT_ERR_UNSUPPORTED, "layernorm_fwd split of %d members (at most %d)",
                     members, kMaxSliceMembers);
  *plan = members < 2 ? Plan{CREDIT_VARIANT_STAGED, 1, nvec} : Plan{CREDIT_VARIANT_SPLIT, members, chunk};
  return CREDIT_OK;
}

const SlicePick* slice_for(int64_t chunk) {
  for (const SlicePick& p : kSlice)
    if (chunk <= p.max_vec) return &p;
  return nullptr;
}

}  // namespace

size_t layernorm_fwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (resolve(&c, cols, cols % 8 == 0, &p) != CREDIT_OK || p.variant != CREDIT_VARIANT_SPLIT)
    return 0;
  int64_t groups = coresident_groups_bound(p.members, cu_count);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  return split_workspace_bytes(groups, p.members, 2, kSplitRing, 0);
}

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
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const bool vec_ok = (cols % 8 == 0) &&
                      reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(beta) % 16 == 0;
  const int64_t nvec = cols / 8;
  Plan plan;
  CREDIT_TRY(resolve(cfg, cols, vec_ok, &plan));
  const dim3 row_grid(static_cast<unsigned>(rows));
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec_ok)
      layernorm_fwd_read_kernel<256, true><<<row_grid, dim3(256), 0, stream>>>(
          x, gamma, beta, y, mean, rstd, c, eps);
    else
      layernorm_fwd_read_kernel<256, false><<<row_grid, dim3(256), 0, stream>>>(
          x, gamma, beta, y, mean, rstd, c, eps);
    return check_launch("layernorm_fwd_read_kernel");
  }
  if (plan.variant == CREDIT_VARIANT_SPLIT) {
    const SlicePick* sp = slice_for(plan.chunk);
    int64_t groups = 0;
    int dispensers = 0;
    CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(sp->fn), sp->threads, 0,
                                 plan.members, &groups, &dispensers));
    if (groups == 0)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "layernorm_fwd: %d groups of %d members do not fit the device",
                       kDispensers, plan.members);
    if (groups > padded_groups(rows)) groups = padded_groups(rows);
    const int64_t per_group = (rows + groups - 1) / groups;
    if (2 * per_group > int64_t{credit::plan::kMaxLaunchStages})
      return set_error(CREDIT_ERR_BAD_SHAPE, "layernorm_fwd: %lld rows per group",
                       static_cast<long long>(per_group));
    SplitWorkspace ws;
    CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, 2, kSplitRing, 0, &ws));
    const uint32_t total = static_cast<uint32_t>(groups * plan.members);
    // Two stages per row at most (the second only for offset rows).
    const SplitArgs sa = make_split_args(ws, total, static_cast<uint32_t>(2 * per_group),
                                         kSplitRing, dispensers);
    hipLaunchKernelGGL(sp->fn, dim3(total), dim3(sp->threads), 0, stream, x, gamma, beta, y,
                       mean, rstd, c, static_cast<int>(plan.chunk), plan.members,
                       static_cast<int>(rows), eps, sa);
    return check_launch("layernorm_fwd_slice_kernel");
  }
  const StagedPick* pick = nullptr;
  for (const StagedPick& p : kStaged) {
    if (nvec <= p.max_vec) {
      pick = &p;
      break;
    }
  }
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  // AUTO: the pipeline once every CU has at least two rows to overlap.
  if (cfg_variant(cfg) == CREDIT_VARIANT_AUTO && nvec > kPipeVec / 2 && nvec <= kPipeVec &&
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
  hipLaunchKernelGGL(pick->fn, row_grid, dim3(pick->threads), 0, stream, x, gamma, beta, y, mean,
                     rstd, c, eps);
  return check_launch("layernorm_fwd_staged_kernel");
}
