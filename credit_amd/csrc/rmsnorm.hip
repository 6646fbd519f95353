// C3: RMSNorm forward and backward, bf16 in/out with fp32 statistics.
//
//   forward : rstd = 1/sqrt(mean(x^2) + eps),  y = x * rstd * w
//   backward: g = dy * w,  xhat = x * rstd,  c = mean(g * xhat),
//             dx = rstd * (g - xhat * c),    dw = sum over rows of dy * xhat
//
// The reference has no RMSNorm; its nearest pattern is the row sum of
// squares of src/workloads/lars_momentum.cu:283-319 (block_read, block_smem
// and cluster_smem variants).  gfx950 variants:
//  - STAGED: one workgroup per row holds the row in VGPRs (a 1024-lane
//            workgroup holds 8192 dwordx4 = a 128 KiB bf16 row at 32 VGPRs
//            per lane): one HBM read of x, one write of y.
//  - SPLIT : P workgroups per row (ticketed groups, common.hpp) each hold a
//            1/P slice and exchange their partial sum of squares once.
//  - READ  : one workgroup per row streams the row twice (sum of squares,
//            then the output pass); any width, any alignment.
// Backward: a group of P members covers a block of R rows; member m owns
// column slice m for all R rows, so it accumulates dw for its slice across
// the block in fp64 registers (dy*x is exact in fp32 and the product with
// rstd is exact in fp64, so the column sums carry no per-term rounding) and
// writes one fp64 partial row per block.  A second kernel sums the blocks'
// partials in block order, which keeps dw deterministic with no float
// atomics.  The row reduction c comes from the per-row exchange (SPLIT, P>1),
// from the whole row held by one member (STAGED, P=1), or from a streaming
// pre-pass (READ: rmsnorm_bwd_rowdot_kernel, then the slice kernel reading c).
//
// Algorithmic traffic (bytes): forward 2MN (x) + 2N (w) + 2MN (y) + 4M
// (rstd); backward 4MN (x, dy) + 2N + 4M + 2MN (dx) + 4N (dw).
#include <initializer_list>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

// ------------------------------------------------------- bf16x8 helpers --
// Sum of squares of 8 packed bf16: four v_dot2_f32_bf16 (products exact in
// fp32).
__device__ __forceinline__ float sumsq8(u32x4 v) {
  return dot2_bf16(v.w, v.w, dot2_bf16(v.z, v.z, dot2_bf16(v.y, v.y, dot2_bf16(v.x, v.x, 0.0f))));
}

__device__ __forceinline__ uint32_t scale2(uint32_t xv, uint32_t wv, float rs) {
  return pack_bf16x2(bf16_lo(xv) * rs * bf16_lo(wv), bf16_hi(xv) * rs * bf16_hi(wv));
}

__device__ __forceinline__ u32x4 scale8(u32x4 x, u32x4 w, float rs) {
  return u32x4{scale2(x.x, w.x, rs), scale2(x.y, w.y, rs), scale2(x.z, w.z, rs),
               scale2(x.w, w.w, rs)};
}

// sum over the 8 lanes of a vector of (dy*w) * x   (the row dot without rstd)
__device__ __forceinline__ float gx8(u32x4 x, u32x4 dy, u32x4 w) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += bf16_lo(dy[i]) * bf16_lo(w[i]) * bf16_lo(x[i]);
    s += bf16_hi(dy[i]) * bf16_hi(w[i]) * bf16_hi(x[i]);
  }
  return s;
}

// dx for one vector: rs * (dy*w - x*rs*c)
__device__ __forceinline__ u32x4 dx8(u32x4 x, u32x4 dy, u32x4 w, float rs, float c) {
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = rs * (bf16_lo(dy[i]) * bf16_lo(w[i]) - bf16_lo(x[i]) * rs * c);
    const float hi = rs * (bf16_hi(dy[i]) * bf16_hi(w[i]) - bf16_hi(x[i]) * rs * c);
    out[i] = pack_bf16x2(lo, hi);
  }
  return out;
}

// ------------------------------------------------------------- forward ---
// One workgroup = one member of a row's group (members == 1: the whole row).
// The member's slice is vectors [v0, v0 + vlen) of the row, held in VPT
// dwordx4 registers per lane.
template <int THREADS, int VPT>
__device__ __forceinline__ void rmsnorm_fwd_slice_kernel_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, float* __restrict__ rstd_out, int cols, int chunk,
    int members, int rows, float eps, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[1][NW];
  SplitGroup g;
  // members == 1: one workgroup per row.  members > 1: a co-resident grid
  // of G groups; the member covers its slice of rows group, group + G, ...
  int row0 = blockIdx.x, step = gridDim.x, member = 0;
  if (members > 1) {
    g = split_join(sa, members, 1);
    row0 = g.group;
    step = static_cast<int>(sa.grid) / members;
    member = g.member;
  }
  const int nvec = cols >> 3;
  const int v0 = member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  // Row traffic through buffer resources over the member's slice: lanes
  // beyond it read zeros (adding nothing to the sum of squares) and drop
  // their stores, with no branch around a load or store.
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  const buffer_rsrc_t wrs = make_rsrc(w + 8 * static_cast<size_t>(v0), slice_bytes);
  for (int row = row0; row < rows; row += step) {
    const size_t off = static_cast<size_t>(row) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t xrs = make_rsrc(x + off, slice_bytes);
    u32x4 v[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) v[k] = buffer_load_nt(xrs, lane_off + k * kStride);
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) ss += sumsq8(v[k]);
    double total[1] = {ss};
    block_reduce_sum_f64_multi<NW, 1>(total, red);
    if (members > 1) {
      if (threadIdx.x == 0) split_publish(g, 0, total[0]);
      split_exchange(g);
      total[0] = split_sum(g, 0);
    }
    const float rs = static_cast<float>(1.0 / __builtin_sqrt(total[0] / cols + eps));
    const buffer_rsrc_t yrs = make_rsrc(y + off, slice_bytes);
#pragma unroll
    for (int k = 0; k < VPT; ++k)
      buffer_store_nt(yrs, lane_off + k * kStride,
                      scale8(v[k], buffer_load(wrs, lane_off + k * kStride), rs));
    if (member == 0 && threadIdx.x == 0) rstd_out[row] = rs;
  }
}

// The 1024-lane shape is held to 64 VGPRs (8 waves per SIMD), so two
// workgroups share a CU: one streams while the other waits on its row's
// exchange (C3 forward, 1024 x 131072 at P = 2: 97.3 -> 95.9 us).
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(THREADS == 1024 ? 8 : 1)))
void rmsnorm_fwd_slice_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, float* __restrict__ rstd_out, int cols, int chunk,
    int members, int rows, float eps, SplitArgs sa) {
  rmsnorm_fwd_slice_kernel_body<THREADS, VPT>(x, w, y, rstd_out, cols, chunk, members, rows, eps, sa);
  split_leave(sa);
}

// Streaming forward: pass 1 sum of squares, pass 2 output.  VEC: rows are
// 16-byte aligned and cols % 8 == 0, so both passes use dwordx4 with four
// loads in flight per lane; otherwise element loads.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void rmsnorm_fwd_read_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, float* __restrict__ rstd_out, int cols, float eps) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[NW];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + static_cast<size_t>(row) * cols;
  uint16_t* yr = y + static_cast<size_t>(row) * cols;
  double ss = 0.0;
  if (VEC) {
    const int nvec = cols >> 3;
    const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS) {
      const u32x4 a = xv[i], b = xv[i + THREADS], c = xv[i + 2 * THREADS],
                  d = xv[i + 3 * THREADS];
      ss += static_cast<double>((sumsq8(a) + sumsq8(b)) + (sumsq8(c) + sumsq8(d)));
    }
    for (; i < nvec; i += THREADS) ss += static_cast<double>(sumsq8(xv[i]));
  } else {
    for (int c = tid; c < cols; c += THREADS) {
      const float v = bf16_to_f32(xr[c]);
      ss += static_cast<double>(v * v);
    }
  }
  const double total = block_reduce_sum_f64<NW>(ss, red);
  const float rs = static_cast<float>(1.0 / __builtin_sqrt(total / cols + eps));
  if (VEC) {
    const int nvec = cols >> 3;
    const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
    const u32x4* wv = reinterpret_cast<const u32x4*>(w);
    u32x4* yv = reinterpret_cast<u32x4*>(yr);
    int i = tid;
    for (; i + 3 * THREADS < nvec; i += 4 * THREADS) {
      const u32x4 a = load_nt(xv + i), b = load_nt(xv + i + THREADS),
                  c = load_nt(xv + i + 2 * THREADS), d = load_nt(xv + i + 3 * THREADS);
      store_nt(yv + i, scale8(a, wv[i], rs));
      store_nt(yv + i + THREADS, scale8(b, wv[i + THREADS], rs));
      store_nt(yv + i + 2 * THREADS, scale8(c, wv[i + 2 * THREADS], rs));
      store_nt(yv + i + 3 * THREADS, scale8(d, wv[i + 3 * THREADS], rs));
    }
    for (; i < nvec; i += THREADS) store_nt(yv + i, scale8(load_nt(xv + i), wv[i], rs));
  } else {
    for (int c = tid; c < cols; c += THREADS)
      yr[c] = f32_to_bf16(bf16_to_f32(xr[c]) * rs * bf16_to_f32(w[c]));
  }
  if (tid == 0) rstd_out[row] = rs;
}

// ------------------------------------------------------------ backward ---
// mode of the backward slice kernel: where the row reduction c comes from.
constexpr int kBwdExchange = 0;  // ticketed group of `members`, one exchange per row
constexpr int kBwdWhole = 1;     // members == 1: the member holds the whole row
constexpr int kBwdGiven = 2;     // c precomputed in rowdot[] (READ variant)

// Member `member` of group `group` covers rows [group*R, group*R + R) and
// vectors [member*chunk, ...) of each.  Per lane: VPT dwordx4 of x and of dy
// for the current row plus the same for the next row, whose loads are
// issued before the current row's reduction and exchange wait, so HBM
// traffic continues through them.  The dw accumulators (8*VPT fp64 per
// lane) live in LDS, laid out [slot][lane] so each lane's read-add-write
// touches consecutive banks; that keeps VGPRs low enough for two
// workgroups per CU.
template <int THREADS, int VPT>
__device__ __forceinline__ void rmsnorm_bwd_slice_kernel_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ rstd,
    const float* __restrict__ rowdot, uint16_t* __restrict__ dx,
    double* __restrict__ dw_part, int rows, int cols, int chunk, int members,
    int rows_per_group, int mode, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  constexpr int kSlots = 8 * VPT;
  extern __shared__ double dw_lds[];  // [kSlots][THREADS]
  __shared__ double red[2][NW];
  const int tid = threadIdx.x;
  SplitGroup g;
  int group, member;
  if (mode == kBwdExchange) {
    g = split_join(sa, members, 1);
    group = g.group;
    member = g.member;
    if (group * rows_per_group >= rows) return;  // padding group
  } else {
    group = blockIdx.x / members;
    member = blockIdx.x - group * members;
  }
  const int nvec = cols >> 3;
  const int v0 = member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const int r0 = group * rows_per_group;
  const int r1 = r0 + rows_per_group < rows ? r0 + rows_per_group : rows;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w) + v0;
#pragma unroll
  for (int q = 0; q < kSlots; ++q) dw_lds[q * THREADS + tid] = 0.0;

  u32x4 xv[VPT], dv[VPT], xn[VPT], dn[VPT];
  auto load_row = [&](u32x4 (&xa)[VPT], u32x4 (&da)[VPT], int r) {
    const size_t off = static_cast<size_t>(r) * cols;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + off) + v0;
    const u32x4* dyr = reinterpret_cast<const u32x4*>(dy + off) + v0;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = tid + k * THREADS;
      const bool in = idx < vlen;
      xa[k] = in ? load_nt(xr + idx) : u32x4{0, 0, 0, 0};
      da[k] = in ? load_nt(dyr + idx) : u32x4{0, 0, 0, 0};
    }
  };
  load_row(xv, dv, r0);
  for (int r = r0; r < r1; ++r) {
    if (r + 1 < r1) load_row(xn, dn, r + 1);
    const float rs = rstd[r];
    double dot;
    if (mode == kBwdGiven) {
      dot = static_cast<double>(rowdot[r]);
    } else {
      float part = 0.0f;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int idx = tid + k * THREADS;
        if (idx < vlen) part += gx8(xv[k], dv[k], wr[idx]);
      }
      dot = block_reduce_sum_f64<NW>(static_cast<double>(part), red[r & 1]);
      if (mode == kBwdExchange) {
        if (tid == 0) split_publish(g, 0, dot);
        split_exchange(g);
        dot = split_sum(g, 0);
      }
    }
    // c = mean(g * xhat) = rs * sum(dy*w*x) / cols
    const float c = static_cast<float>(dot * rs / cols);
    const double rsd = static_cast<double>(rs);
    u32x4* dxr = reinterpret_cast<u32x4*>(dx + static_cast<size_t>(r) * cols) + v0;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int idx = tid + k * THREADS;
      if (idx < vlen) {
        store_nt(dxr + idx, dx8(xv[k], dv[k], wr[idx], rs, c));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // dy*x is exact in fp32 (bf16 x bf16); times rstd it is exact in fp64.
          double* a = dw_lds + (k * 8 + 2 * i) * THREADS + tid;
          a[0] += static_cast<double>(bf16_lo(dv[k][i]) * bf16_lo(xv[k][i])) * rsd;
          a[THREADS] += static_cast<double>(bf16_hi(dv[k][i]) * bf16_hi(xv[k][i])) * rsd;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = xn[k];
      dv[k] = dn[k];
    }
  }
  // One fp64 partial row per block: rounding the block sums to fp32 here
  // would add ~ulp(block sum) per block to dw.
  double* pr = dw_part + static_cast<size_t>(group) * cols + 8 * static_cast<size_t>(v0);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int idx = tid + k * THREADS;
    if (idx < vlen) {
      f64x2* q = reinterpret_cast<f64x2*>(pr + 8 * static_cast<size_t>(idx));
      const double* a = dw_lds + k * 8 * THREADS + tid;
      q[0] = f64x2{a[0], a[THREADS]};
      q[1] = f64x2{a[2 * THREADS], a[3 * THREADS]};
      q[2] = f64x2{a[4 * THREADS], a[5 * THREADS]};
      q[3] = f64x2{a[6 * THREADS], a[7 * THREADS]};
    }
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void rmsnorm_bwd_slice_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ rstd,
    const float* __restrict__ rowdot, uint16_t* __restrict__ dx,
    double* __restrict__ dw_part, int rows, int cols, int chunk, int members,
    int rows_per_group, int mode, SplitArgs sa) {
  rmsnorm_bwd_slice_kernel_body<THREADS, VPT>(x, w, dy, rstd, rowdot, dx, dw_part, rows, cols, chunk, members, rows_per_group, mode, sa);
  split_leave(sa);
}

// SPLIT variant.  The workgroup is THREADS data lanes (VPT dwordx4 of x
// and of dy per lane and row) plus one communication wave.  Member `member`
// of group `group` (of G) covers rows group, group + G, group + 2G, ... and
// vectors [member*chunk, member*chunk + THREADS*VPT) of each.
//
// No workgroup barrier in the row loop.  In the step of row i each data
// wave issues the loads of row i+DEPTH+AHEAD, reduces row i+DEPTH (loaded
// AHEAD steps earlier) to a wave partial in LDS and counts itself in with
// an LDS atomic; the wave that arrives last sums the partials in wave order
// and publishes the member's partial of row i+DEPTH.  The communication
// wave runs ahead on its own: it polls each row's exchange, writes the
// group total into an LDS ring of RING entries and advances an LDS ready
// count.  A data wave waits (LDS spin) for row i's total, writes dx of row
// i and folds row i into its dw accumulators.  Row i is published DEPTH
// steps before it is needed, so the exchange round trip (~2000 cycles idle,
// ~3 us under this kernel's own load) overlaps the data waves' work, and
// no wave waits for another wave's loads; AHEAD steps of loads stay in
// flight.  DEPTH + AHEAD + 1 row buffers rotate through registers.  At C3
// (16 members of 1024 vectors), against DEPTH 2 / AHEAD 1 on the same box:
// the backward at DEPTH 3 / AHEAD 2 160.3 -> 157.6 us on one box and
// unchanged (161.0) on another, the fused forward + backward at 2 / 2
// 227 -> 217 and 229.5 -> 221.3 us; later, the backward at DEPTH 4 / AHEAD 2
// (seven row buffers, 162 VGPRs) 148.7 -> 147.5 us against 3 / 2 (three
// alternating runs, one box; 3 / 3 and 2 / 3 no better, AHEAD 1 spills);
// DEPTH 1 is exchange-bound (225 us), and
// a build whose communication wave does not wait at all is slower (169.5
// us), so the exchange is not what bounds the kernel.  The LDS ring, partial and
// counter slots of row k are reused by row k+RING only (RING >= DEPTH + 2):
// a wave reaches the step that rewrites them after row k+RING-DEPTH-1's
// total is ready, which orders it after every access to them for row k.
// The device slot ring must exceed the 2 DEPTH + 1 stages between the
// fastest publisher and the slowest poller.  Every wait ends: the poll is
// bounded (watchdog), and the ready count then still advances.
//
// The data loop has no branches around its row traffic: every load and
// store goes through a buffer resource whose num_records covers the
// member's slice, or 0 for a row beyond the group, so lanes out of range
// read zeros and drop their stores; the waitcnt pass then waits for row
// i+DEPTH while the later rows' loads stay in flight (on gfx9 one vmcnt
// counts loads and stores in order; a load under a branch makes the count
// path-dependent and the wait after the join a full drain).  dw
// accumulators: fp64 in LDS, [8*VPT][THREADS], one owner lane each.
// The group pipeline of the backward and of the fused forward + backward.
// FUSED: the row's sum of squares travels in the same exchange as
// sum(dy*w*x) (two values per member), rstd comes from it instead of the
// forward, and y = x * rstd * w is written beside dx.
// Exchange stages in the device slot ring of the group kernels.
constexpr int kGroupSlotRing = 16;

template <int THREADS, int VPT, bool FUSED, int DEPTH, int AHEAD>
__device__ __forceinline__ void rmsnorm_group_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ rstd, float* __restrict__ rstd_out,
    uint16_t* __restrict__ y, uint16_t* __restrict__ dx, double* __restrict__ dw_part, int rows,
    int cols, int chunk, int members, int rows_per_group, float eps, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  constexpr int K = FUSED ? 2 : 1;  // values per member per row
  constexpr int kSlots = 8 * VPT;
  constexpr int NB = DEPTH + AHEAD + 1;       // row buffers per lane
  constexpr int RING = DEPTH + 2 <= 4 ? 4 : 8;  // LDS entries per row slot
  static_assert(DEPTH >= 1 && AHEAD >= 1 && DEPTH + 2 <= 8, "pipeline depth");
  static_assert(2 * DEPTH + 1 < kGroupSlotRing, "device slot ring too short for DEPTH");
  extern __shared__ double dw_lds[];  // [kSlots][THREADS]
  __shared__ double red[RING][K][NW];  // wave partials of row k at [(k - r0) % RING]
  __shared__ double ring[RING][K];     // group totals of row k at [(k - r0) % RING]
  __shared__ uint32_t arrivals[RING];
  __shared__ uint32_t ready;           // rows r0 .. r0 + ready - 1 have totals
  const int tid = threadIdx.x;
  if (tid < RING) arrivals[tid] = 0;
  if (tid == 0) ready = 0;
  const SplitGroup g = split_join(sa, members, K);  // its barrier covers the stores above
  // Rows are dealt to the G groups round-robin: group g's k-th row is
  // g + k G, so the rows in flight at any moment are adjacent in memory.
  // Contiguous blocks per group put the concurrent rows 16 MiB apart at C3
  // (a power-of-two stride): 160.3 -> 146.5 us for the backward, 221.5 ->
  // 206 us fused, bit-identical outputs.  Below, i counts the group's rows
  // (0 .. r1-1) and row_of(i) is the tensor row.
  // G: the groups that take rows (the launch pads the grid to a multiple
  // of the dispensers; padding groups, and their dweight partial rows where
  // there are any, stay out).  Each takes at most rows_per_group rows, the
  // host's bound on its exchange tags.
  const int G = (rows + rows_per_group - 1) / rows_per_group;
  if (g.group >= G) return;  // padding group
  const int r0 = 0;
  const int r1 = (rows - g.group + G - 1) / G;
  auto row_of = [&](int i) { return g.group + i * G; };
  const int nvec = cols >> 3;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;

  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS) {
    // ---- communication wave: poll every row's exchange in order ----
    // The backward's communication wave runs at raised issue priority: 146.5
    // -> 144.9 us at C3 (two sessions of three alternating runs).  The same
    // raise slowed the fused forward + backward by 7.5%, the forward group
    // pipeline by 5% and the softmax group kernels by 3-5%, which keep the
    // default priority.
    if constexpr (!FUSED) __builtin_amdgcn_s_setprio(3);
    for (int k = r0; k < r1; ++k) {
      const uint32_t bits = split_poll(g, k - r0, K);
      const double dot = split_wave_sum(bits, members, 0);
      const double ssq = FUSED ? split_wave_sum(bits, members, 1) : 0.0;
      if (tid == THREADS) {
        ring[(k - r0) % RING][0] = dot;
        if (FUSED) ring[(k - r0) % RING][K - 1] = ssq;
        __hip_atomic_store(&ready, static_cast<uint32_t>(k - r0 + 1), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    return;
  }

  // ---- data waves ----
  const int wid = tid / kWave;
  const bool lead = (tid & (kWave - 1)) == 0;
  const uint32_t lane_off = static_cast<uint32_t>(tid) * 16u;
  constexpr uint32_t kStride = THREADS * 16u;  // bytes between a lane's vectors
  struct Row {
    u32x4 x[VPT], d[VPT];
  };
  Row b[NB];
  // Row r's slice, or zeros (no traffic) when r is beyond the group.
  auto load_row = [&](Row& b, int r) {
    const bool live = r < r1;
    const size_t off =
        static_cast<size_t>(row_of(live ? r : r0)) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t xs = make_rsrc(x + off, live ? slice_bytes : 0u);
    const buffer_rsrc_t ds = make_rsrc(dy + off, live ? slice_bytes : 0u);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      b.x[k] = buffer_load_nt(xs, lane_off + k * kStride);
      b.d[k] = buffer_load_nt(ds, lane_off + k * kStride);
    }
  };
  // The member's weight slice stays in registers for the whole loop.
  const buffer_rsrc_t wrs = make_rsrc(w + 8 * static_cast<size_t>(v0), slice_bytes);
  u32x4 wk[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) wk[q] = buffer_load(wrs, lane_off + q * kStride);
  // Reduce row k to a wave partial; the last wave in publishes the member's.
  auto publish_row = [&](const Row& b, int k) {
    float part = 0.0f, ss = 0.0f;
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      part += gx8(b.x[q], b.d[q], wk[q]);
      if (FUSED) ss += sumsq8(b.x[q]);
    }
    const double v = wave_reduce_sum_f64(static_cast<double>(part));
    const double vs = FUSED ? wave_reduce_sum_f64(static_cast<double>(ss)) : 0.0;
    const int slot = (k - r0) % RING;
    if (lead) {
      red[slot][0][wid] = v;
      if (FUSED) red[slot][K - 1][wid] = vs;
      const uint32_t t = __hip_atomic_fetch_add(&arrivals[slot], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
      if (t == NW - 1) {
#pragma unroll
        for (int e = 0; e < K; ++e) {
          double s = red[slot][e][0];
#pragma unroll
          for (int q = 1; q < NW; ++q) s += red[slot][e][q];
          split_publish_at(g, k - r0, e, s);
        }
        arrivals[slot] = 0;
      }
    }
  };
  auto wait_total = [&](int i) {
    const uint32_t need = static_cast<uint32_t>(i - r0 + 1);
    while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < need)
      __builtin_amdgcn_s_sleep(1);
    return (i - r0) % RING;
  };
  const double inv_cols = 1.0 / cols;
  auto finish_row = [&](Row& b, int r, int slot) {
    if constexpr (AHEAD > 1) {
      // The row's unpacked products were formed at its publish, DEPTH steps
      // earlier; kept live across the steps they take ~50 VGPRs per dwordx4
      // and the deeper pipeline spills.  Recompute them from the packed row.
#pragma unroll
      for (int q = 0; q < VPT; ++q) {
        __asm__ volatile("" : "+v"(b.x[q]));
        __asm__ volatile("" : "+v"(b.d[q]));
      }
    }
    const double dot = ring[slot][0];
    float rs;
    if (FUSED) {
      const double ms = ring[slot][K - 1] / cols;
      rs = static_cast<float>(1.0 / __builtin_sqrt(ms + eps));
    } else {
      rs = rstd[row_of(r)];
    }
    // c = mean(g * xhat) = rs * sum(dy*w*x) / cols
    const float c = static_cast<float>(dot * (rs * inv_cols));
    const double rsd = static_cast<double>(rs);
    const size_t off = static_cast<size_t>(row_of(r)) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t out = make_rsrc(dx + off, slice_bytes);
    if (FUSED) {
      const buffer_rsrc_t yrs = make_rsrc(y + off, slice_bytes);
#pragma unroll
      for (int q = 0; q < VPT; ++q)
        buffer_store_nt(yrs, lane_off + q * kStride, scale8(b.x[q], wk[q], rs));
      if (g.member == 0 && tid == 0) rstd_out[row_of(r)] = rs;
    }
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      buffer_store_nt(out, lane_off + q * kStride, dx8(b.x[q], b.d[q], wk[q], rs, c));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // dy*x is exact in fp32 (bf16 x bf16); times rstd it is exact in
        // fp64.  Lanes beyond the slice hold zeros and add nothing.  Each
        // lane owns its accumulators, so the add is an uncontended LDS fp64
        // atomic (ds_add_f64): no read-back registers, half the LDS
        // traffic, and the same rounding and order as a read-add-write.
        double* a = dw_lds + (q * 8 + 2 * i) * THREADS + tid;
        lds_add(a, static_cast<double>(bf16_lo(b.d[q][i]) * bf16_lo(b.x[q][i])) * rsd);
        lds_add(a + THREADS, static_cast<double>(bf16_hi(b.d[q][i]) * bf16_hi(b.x[q][i])) * rsd);
      }
    }
  };
  // Step of row i (buffer S = i - r0 mod NB): cur = row i, row i+DEPTH
  // (loaded) is reduced and published, buffer (S + DEPTH + AHEAD) % NB
  // receives row i+DEPTH+AHEAD.
  auto step = [&]<int S>(std::integral_constant<int, S>, int i) {
    load_row(b[(S + DEPTH + AHEAD) % NB], i + DEPTH + AHEAD);
    __builtin_amdgcn_sched_barrier(0);
    if (i + DEPTH < r1) publish_row(b[(S + DEPTH) % NB], i + DEPTH);
    finish_row(b[S], i, wait_total(i));
  };

#pragma unroll
  for (int q = 0; q < kSlots; ++q) dw_lds[q * THREADS + tid] = 0.0;
  [&]<int... J>(std::integer_sequence<int, J...>) {
    (load_row(b[J], r0 + J), ...);
  }(std::make_integer_sequence<int, DEPTH + AHEAD>{});
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ((r0 + J < r1 ? publish_row(b[J], r0 + J) : void()), ...);
  }(std::make_integer_sequence<int, DEPTH>{});
  // Rotate the NB buffers through statically indexed registers.
  int i = r0;
  for (; i + NB - 1 < r1; i += NB)
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (step(std::integral_constant<int, S>{}, i + S), ...);
    }(std::make_integer_sequence<int, NB>{});
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((i + S < r1 ? step(std::integral_constant<int, S>{}, i + S) : void()), ...);
  }(std::make_integer_sequence<int, NB - 1>{});
  // One fp64 partial row per group member slice (own lanes' accumulators).
  const buffer_rsrc_t prs =
      make_rsrc(dw_part + static_cast<size_t>(g.group) * cols + 8 * static_cast<size_t>(v0),
                slice_bytes * 4u);
#pragma unroll
  for (int v = 0; v < VPT; ++v)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      buffer_store(prs, (lane_off + v * kStride) * 4u + 16u * q,
                   __builtin_bit_cast(u32x4, f64x2{dw_lds[(v * 8 + 2 * q) * THREADS + tid],
                                                   dw_lds[(v * 8 + 2 * q + 1) * THREADS + tid]}));
}

// Forward group pipeline (SPLIT of at most 32 members of 1025-2048 vectors, and AUTO on
// rows of 8193-16384 vectors: C3's 131072 columns run as 8 members): the
// backward's pipeline on x alone -- VPT dwordx4 of x per lane and row in
// DEPTH + AHEAD + 1 rotating buffers, the weight slice in registers, no
// barrier in the row loop -- with one exchanged value per row (the member's
// sum of squares), which the communication wave turns into rstd.  At C3,
// three alternating runs against the two-member slice kernel (97.0 us):
// DEPTH / AHEAD 4 / 1 95.1 us, 3 / 2 95.7, 3 / 1 99.0, 2 / 2 103.0, 2 / 1
// 104.7; 16 members of 1024 vectors (VPT 2) 4 / 2 118.7, 2 / 1 110.8; 5 / 1
// and 4 / 2 at VPT 4 exceed the 168 VGPRs of a 9-wave workgroup.
//
// Rows come from a launch-wide ticket queue, so that groups which run
// faster take more rows (a group sits on one XCD, and with a fixed share
// per group the XCDs' ends were 5-10 us apart at C3, the slowest XCD
// changing from call to call).  Row step i < L takes the fixed row g + i G;
// step i >= L takes row L G + t for a ticket t that member 0's ticket wave
// (a tenth wave) draws from the counter once stage i - L - 1 is released,
// waits for and publishes in member 0's value-1 slot of stage i; every
// member's communication wave reads it at stage i - L + 2 and writes the
// row id into an LDS ring (RR entries) before it releases that stage, which
// is one stage before the data waves issue the row's loads (step i - DEPTH
// - AHEAD).  The first ticket naming no row ends the group's steps.  One
// ticket is drawn per row step processed, so a launch draws exactly `rows`
// tickets and the wave that draws value rows - 1 returns the counter to
// zero.  C3: 94.8-95.1 -> 93.8-94.1 us and 94.7-94.9 -> 94.3-94.5 us
// (alternating runs on two boxes).
template <int THREADS, int VPT, int DEPTH, int AHEAD>
__device__ __forceinline__ void rmsnorm_fwd_group_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    float* __restrict__ rstd_out, int rows, int cols, int chunk, int members,
    int rows_per_group, float eps, SplitArgs sa, uint32_t* __restrict__ queue) {
  constexpr int NW = THREADS / kWave;
  constexpr int NB = DEPTH + AHEAD + 1;
  constexpr int RING = DEPTH + 2 <= 4 ? 4 : 8;
  constexpr int L = DEPTH + AHEAD + 3;
  constexpr int RR = 16;
  static_assert(DEPTH >= 1 && AHEAD >= 1 && DEPTH + 2 <= 8, "pipeline depth");
  static_assert(2 * DEPTH + 1 < kGroupSlotRing, "device slot ring too short for DEPTH");
  static_assert(L + DEPTH < RR && L + DEPTH < kGroupSlotRing, "ticket rings");
  __shared__ double red[RING][NW];
  __shared__ float ring[RING];
  __shared__ uint32_t arrivals[RING];
  __shared__ uint32_t ready;
  __shared__ int rowid[RR];
  const int tid = threadIdx.x;
  if (tid < RING) arrivals[tid] = 0;
  if (tid == 0) ready = 0;
  const SplitGroup g = split_join(sa, members, 2);
  const int G = (rows + rows_per_group - 1) / rows_per_group;
  if (g.group >= G) return;
  // The group's fixed rows g + i G, i < n_fixed (all L of them when rows >= L G).
  const int r1 = (rows - g.group + G - 1) / G;
  const int n_fixed = r1 < L ? r1 : L;
  const int64_t first = static_cast<int64_t>(L) * G;  // the row of ticket 0
  auto row_of = [&](int i) {
    return i < L ? (i < n_fixed ? g.group + i * G : rows) : rowid[i % RR];
  };
  // Step i has a row (the steps that do are a prefix).
  auto live = [&](int i) { return row_of(i) < rows; };
  const int nvec = cols >> 3;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;
  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS + kWave) {
    if (g.member == 0) queue_ticket_wave(g, queue, &ready, n_fixed, L, first, rows, 1);
    return;
  }
  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS) {
    // ---- communication wave: stage k's total into ring, the row of step
    // k + L - 2 into rowid, then the release of stage k ----
    int n = n_fixed < L ? n_fixed : INT32_MAX;
    for (int k = 0; k < n; ++k) {
      const uint32_t bits = split_poll(g, k, 1);
      const double ssq = split_wave_sum(bits, members, 0);
      const int row = queue_take_row(g, k, L, first, rows, 1, &n);
      if (tid == THREADS) {
        if (row >= 0) rowid[(k + L - 2) % RR] = row;
        ring[k % RING] = static_cast<float>(1.0 / __builtin_sqrt(ssq / cols + eps));
        __hip_atomic_store(&ready, static_cast<uint32_t>(k + 1), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    return;
  }
  const int wid = tid / kWave;
  const bool lead = (tid & (kWave - 1)) == 0;
  const uint32_t lane_off = static_cast<uint32_t>(tid) * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  struct Row {
    u32x4 x[VPT];
  };
  Row b[NB];
  auto load_row = [&](Row& b, int r) {
    const bool on = live(r);
    const size_t off =
        static_cast<size_t>(on ? row_of(r) : 0) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t xs = make_rsrc(x + off, on ? slice_bytes : 0u);
#pragma unroll
    for (int k = 0; k < VPT; ++k) b.x[k] = buffer_load_nt(xs, lane_off + k * kStride);
  };
  const buffer_rsrc_t wrs = make_rsrc(w + 8 * static_cast<size_t>(v0), slice_bytes);
  u32x4 wk[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) wk[q] = buffer_load(wrs, lane_off + q * kStride);
  auto publish_row = [&](const Row& b, int k) {
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < VPT; ++q) ss += sumsq8(b.x[q]);
    const double v = wave_reduce_sum_f64(static_cast<double>(ss));
    const int slot = k % RING;
    if (lead) {
      red[slot][wid] = v;
      const uint32_t t = __hip_atomic_fetch_add(&arrivals[slot], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
      if (t == NW - 1) {
        double s = red[slot][0];
#pragma unroll
        for (int q = 1; q < NW; ++q) s += red[slot][q];
        split_publish_at(g, k, 0, s);
        arrivals[slot] = 0;
      }
    }
  };
  auto wait_total = [&](int i) {
    const uint32_t need = static_cast<uint32_t>(i + 1);
    while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < need)
      __builtin_amdgcn_s_sleep(1);
    return i % RING;
  };
  auto finish_row = [&](Row& b, int r, int slot) {
#pragma unroll
    for (int q = 0; q < VPT; ++q) __asm__ volatile("" : "+v"(b.x[q]));
    const float rs = ring[slot];
    const int row = row_of(r);
    const size_t off = static_cast<size_t>(row) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t out = make_rsrc(y + off, slice_bytes);
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      buffer_store_nt(out, lane_off + q * kStride, scale8(b.x[q], wk[q], rs));
    // Lane 0 of member 0 writes rstd (a 4-byte resource; other lanes fall outside it).
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(rs),
                                          make_rsrc(rstd_out + row, g.member == 0 ? 4u : 0u),
                                          static_cast<uint32_t>(tid) * 4u, 0, 0);
  };
  auto step = [&]<int S>(std::integral_constant<int, S>, int i) {
    load_row(b[(S + DEPTH + AHEAD) % NB], i + DEPTH + AHEAD);
    __builtin_amdgcn_sched_barrier(0);
    if (live(i + DEPTH)) publish_row(b[(S + DEPTH) % NB], i + DEPTH);
    finish_row(b[S], i, wait_total(i));
  };
  [&]<int... J>(std::integer_sequence<int, J...>) {
    (load_row(b[J], J), ...);
  }(std::make_integer_sequence<int, DEPTH + AHEAD>{});
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ((live(J) ? publish_row(b[J], J) : void()), ...);
  }(std::make_integer_sequence<int, DEPTH>{});
  // The group's steps end at the first step without a row; step i's row is
  // known once the data waves are past step i - DEPTH - AHEAD - 1.
  int i = 0;
  for (bool go = true; go; i += NB)
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (((go = go && live(i + S)) ? step(std::integral_constant<int, S>{}, i + S) : void()), ...);
    }(std::make_integer_sequence<int, NB>{});
}

// THREADS data lanes, the communication wave and the ticket wave.
template <int THREADS, int VPT, int DEPTH, int AHEAD>
__global__ __launch_bounds__(THREADS + 2 * kWave)
__attribute__((amdgpu_waves_per_eu(3, 8))) void rmsnorm_fwd_group_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    float* __restrict__ rstd_out, int rows, int cols, int chunk, int members,
    int rows_per_group, float eps, SplitArgs sa, uint32_t* __restrict__ queue) {
  rmsnorm_fwd_group_body<THREADS, VPT, DEPTH, AHEAD>(x, w, y, rstd_out, rows, cols, chunk,
                                                     members, rows_per_group, eps, sa, queue);
  split_leave(sa);
}

// Waves per SIMD a group kernel is compiled for: VPT 1 leaves room for two
// 8-wave workgroups per CU; VPT 2 fills one 9-wave workgroup (512 data
// lanes plus the communication wave).
template <int VPT>
constexpr int kGroupWavesPerEU = VPT == 1 ? 4 : 3;

template <int THREADS, int VPT, int DEPTH = 2, int AHEAD = 1>
__global__ __launch_bounds__(THREADS + kWave)
__attribute__((amdgpu_waves_per_eu(kGroupWavesPerEU<VPT>, 8))) void rmsnorm_bwd_group_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ rstd, uint16_t* __restrict__ dx,
    double* __restrict__ dw_part, int rows, int cols, int chunk, int members,
    int rows_per_group, SplitArgs sa) {
  rmsnorm_group_body<THREADS, VPT, false, DEPTH, AHEAD>(x, w, dy, rstd, nullptr, nullptr, dx, dw_part,
                                                 rows, cols, chunk, members, rows_per_group,
                                                 0.0f, sa);
  split_leave(sa);
}

// Forward and backward in one pass: x, dy, w in; y, rstd, dx, dweight out.
template <int THREADS, int VPT, int DEPTH = 2, int AHEAD = 1>
__global__ __launch_bounds__(THREADS + kWave)
__attribute__((amdgpu_waves_per_eu(kGroupWavesPerEU<VPT>, 8))) void rmsnorm_fused_group_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, float* __restrict__ rstd, uint16_t* __restrict__ y,
    uint16_t* __restrict__ dx, double* __restrict__ dw_part, int rows, int cols, int chunk,
    int members, int rows_per_group, float eps, SplitArgs sa) {
  rmsnorm_group_body<THREADS, VPT, true, DEPTH, AHEAD>(x, w, dy, nullptr, rstd, y, dx, dw_part, rows,
                                                cols, chunk, members, rows_per_group, eps, sa);
  split_leave(sa);
}

// READ variant pre-pass: rowdot[r] = sum_j dy*w*x over the row, streamed.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void rmsnorm_bwd_rowdot_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ dy, float* __restrict__ rowdot, int cols) {
  constexpr int NW = THREADS / kWave;
  __shared__ double red[NW];
  const int row = blockIdx.x;
  const int nvec = cols >> 3;
  const size_t off = static_cast<size_t>(row) * cols;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x + off);
  const u32x4* dv = reinterpret_cast<const u32x4*>(dy + off);
  const u32x4* wv = reinterpret_cast<const u32x4*>(w);
  double s = 0.0;
  int i = threadIdx.x;
  for (; i + THREADS < nvec; i += 2 * THREADS) {
    const u32x4 a = load_nt(xv + i), b = load_nt(xv + i + THREADS);
    const u32x4 da = load_nt(dv + i), db = load_nt(dv + i + THREADS);
    s += static_cast<double>(gx8(a, da, wv[i]) + gx8(b, db, wv[i + THREADS]));
  }
  for (; i < nvec; i += THREADS) s += static_cast<double>(gx8(load_nt(xv + i), load_nt(dv + i), wv[i]));
  const double t = block_reduce_sum_f64<NW>(s, red);
  if (threadIdx.x == 0) rowdot[row] = static_cast<float>(t);
}

// dw[c] = sum over blocks b (in order) of part[b][c], rounded once to fp32.
__global__ __launch_bounds__(256) void rmsnorm_dw_reduce_kernel(
    const double* __restrict__ part, float* __restrict__ dw, int blocks, int cols) {
  const int q = blockIdx.x * 256 + threadIdx.x;  // two columns
  const int nq = cols >> 1;
  if (q >= nq) return;
  const f64x2* p = reinterpret_cast<const f64x2*>(part) + q;
  double a0 = 0.0, a1 = 0.0;
#pragma unroll 8
  for (int b = 0; b < blocks; ++b) {
    const f64x2 v = load_nt(p + static_cast<size_t>(b) * nq);
    a0 += v.x;
    a1 += v.y;
  }
  reinterpret_cast<float2_t*>(dw)[q] = float2_t{static_cast<float>(a0), static_cast<float>(a1)};
}

// ------------------------------------------------------------ dispatch ---
using FwdSliceFn = void (*)(const uint16_t*, const uint16_t*, uint16_t*, float*, int, int,
                            int, int, float, SplitArgs);
using BwdSliceFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, const float*,
                            const float*, uint16_t*, double*, int, int, int, int, int, int,
                            SplitArgs);

struct FwdPick {
  FwdSliceFn fn;
  int threads;
  int capacity;  // dwordx4 per workgroup
};
using BwdGroupFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, const float*,
                            uint16_t*, double*, int, int, int, int, int, SplitArgs);
struct BwdPick {
  BwdSliceFn fn;
  int threads;
  int capacity;
  int lds_bytes() const { return capacity * 8 * static_cast<int>(sizeof(double)); }
};
// SPLIT: THREADS data lanes + one communication wave; per_cu is the
// residency its VGPR and LDS use allows (sizes the row groups).
struct BwdGroupPick {
  BwdGroupFn fn;
  int threads;
  int capacity;
  int per_cu;
  int lds_bytes() const { return capacity * 8 * static_cast<int>(sizeof(double)); }
};

// Smallest footprint first.  VPT stays at 4-8 dwordx4 per lane: deeper
// register staging makes the compiler hoist the weight loads of the output
// loop and spill.
const FwdPick kFwd[] = {
    {rmsnorm_fwd_slice_kernel<64, 4>, 64, 256},
    {rmsnorm_fwd_slice_kernel<128, 4>, 128, 512},
    {rmsnorm_fwd_slice_kernel<256, 4>, 256, 1024},
    {rmsnorm_fwd_slice_kernel<256, 8>, 256, 2048},
    {rmsnorm_fwd_slice_kernel<512, 8>, 512, 4096},
    {rmsnorm_fwd_slice_kernel<1024, 8>, 1024, 8192},
};
// Two row buffers of x and dy at VPT = 2 per lane; the fp64 dw accumulators
// take 16 * VPT * 8 bytes of LDS per lane (64 KiB at 512 lanes), so two
// workgroups share a CU.
const BwdPick kBwd[] = {
    {rmsnorm_bwd_slice_kernel<64, 2>, 64, 128},
    {rmsnorm_bwd_slice_kernel<128, 2>, 128, 256},
    {rmsnorm_bwd_slice_kernel<256, 2>, 256, 512},
    {rmsnorm_bwd_slice_kernel<512, 2>, 512, 1024},
};
// Group kernels: four row buffers per lane.  At one dwordx4 per lane
// (~104 VGPRs: 4 waves per SIMD, 16 per CU; 64 bytes of LDS dw
// accumulators per lane) 448 data lanes + 1 wave = 8 waves give two
// workgroups per CU and 960 + 1 = 16 waves one; two dwordx4 per lane (3
// waves per SIMD) hold the widest slice, 1024 vectors, one workgroup per CU.
const BwdGroupPick kBwdGroup[] = {
    {rmsnorm_bwd_group_kernel<64, 1>, 64, 64, 8},
    {rmsnorm_bwd_group_kernel<128, 1>, 128, 128, 5},
    {rmsnorm_bwd_group_kernel<192, 1>, 192, 192, 4},
    {rmsnorm_bwd_group_kernel<448, 1>, 448, 448, 2},
    {rmsnorm_bwd_group_kernel<960, 1>, 960, 960, 1},
    {rmsnorm_bwd_group_kernel<512, 2, 4, 2>, 512, 1024, 1},
};
// Fused forward + backward: the same shapes, the sum of squares riding in
// the same exchange (two values per member, so at most 32 members).
using FusedGroupFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, float*,
                              uint16_t*, uint16_t*, double*, int, int, int, int, int, float,
                              SplitArgs);
struct FusedGroupPick {
  FusedGroupFn fn;
  int threads;
  int capacity;
  int lds_bytes() const { return capacity * 8 * static_cast<int>(sizeof(double)); }
};
const FusedGroupPick kFusedGroup[] = {
    {rmsnorm_fused_group_kernel<64, 1>, 64, 64},
    {rmsnorm_fused_group_kernel<128, 1>, 128, 128},
    {rmsnorm_fused_group_kernel<192, 1>, 192, 192},
    {rmsnorm_fused_group_kernel<448, 1>, 448, 448},
    {rmsnorm_fused_group_kernel<960, 1>, 960, 960},
    {rmsnorm_fused_group_kernel<512, 2, 2, 2>, 512, 1024},
};
constexpr int kMaxFusedMembers = kMaxExchangeValues / 2;
constexpr int kFwdMaxCapacity = 8192;
// The forward group pipeline: 512 data lanes x 4 dwordx4; AUTO takes it for
// rows that need at most 8 such members.
constexpr int kFwdGroupThreads = 512;
constexpr int kFwdGroupVpt = 4;
constexpr int64_t kFwdGroupCapacity = kFwdGroupThreads * kFwdGroupVpt;
constexpr int kFwdGroupAutoMembers = 8;

constexpr int kBwdMaxCapacity = 1024;      // slice kernels (STAGED, READ tiles)
constexpr int kBwdGroupCapacity = 1024;    // group kernel (SPLIT): largest member slice

template <class Pick, int N>
const Pick* pick_for(const Pick (&table)[N], int64_t chunk) {
  for (const Pick& p : table)
    if (chunk <= p.capacity) return &p;
  return nullptr;
}

bool vec_ok(int64_t cols, std::initializer_list<const void*> ptrs) {
  if (cols % 8 != 0) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  return true;
}

// Split plan: members P and vectors per member.  Members are trimmed so
// that none is empty.
struct Plan {
  int variant;
  int members;
  int64_t chunk;
};

// SPLIT plans of at most 32 members holding 1025-2048 vectors each run the
// forward group pipeline; the others the slice kernel.
bool fwd_takes_group(const Plan& p) {
  return p.variant == CREDIT_VARIANT_SPLIT && p.members <= 32 &&
         p.chunk > kFwdGroupCapacity / 2 && p.chunk <= kFwdGroupCapacity;
}

Plan plan_split(int64_t nvec, int members) {
  Plan p{CREDIT_VARIANT_SPLIT, members, (nvec + members - 1) / members};
  p.members = static_cast<int>((nvec + p.chunk - 1) / p.chunk);
  return p;
}

int resolve_fwd(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  const int variant = cfg_variant(cfg);
  const int64_t nvec = cols / 8;
  if (variant == CREDIT_VARIANT_READ || (!vec && variant == CREDIT_VARIANT_AUTO)) {
    *plan = Plan{CREDIT_VARIANT_READ, 1, nvec};
    return CREDIT_OK;
  }
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd staged/split variants need cols %% 8 == 0 and 16-byte "
                     "aligned buffers");
  if (variant == CREDIT_VARIANT_STAGED || variant == CREDIT_VARIANT_AUTO) {
    if (nvec <= kFwdMaxCapacity) {
      *plan = Plan{CREDIT_VARIANT_STAGED, 1, nvec};
      return CREDIT_OK;
    }
    if (variant == CREDIT_VARIANT_STAGED)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_fwd staged variant holds at most %d columns", kFwdMaxCapacity * 8);
    // AUTO on a row wider than one workgroup: the group pipeline when at
    // most kFwdGroupAutoMembers of its slices cover the row, else the slice
    // kernel split just enough.
    const int64_t pg = (nvec + kFwdGroupCapacity - 1) / kFwdGroupCapacity;
    if (pg <= kFwdGroupAutoMembers) {
      *plan = plan_split(nvec, static_cast<int>(pg));
      return CREDIT_OK;
    }
    *plan = plan_split(nvec, static_cast<int>((nvec + kFwdMaxCapacity - 1) / kFwdMaxCapacity));
    return CREDIT_OK;
  }
  int p = cfg_split(cfg);
  if (p == 0) p = static_cast<int>((nvec + kFwdMaxCapacity - 1) / kFwdMaxCapacity);
  if (p < 2) p = 2;
  if (p > nvec) p = static_cast<int>(nvec);
  *plan = plan_split(nvec, p);
  if (plan->chunk > kFwdMaxCapacity)
    return set_error(CREDIT_ERR_UNSUPPORTED, "rmsnorm_fwd split %d leaves %lld vectors per member",
                     p, static_cast<long long>(plan->chunk));
  if (plan->members < 2) *plan = Plan{CREDIT_VARIANT_STAGED, 1, nvec};
  return CREDIT_OK;
}

// Backward plan: members P, vectors per member, rows per group R.
struct BwdPlan {
  int variant;
  int members;
  int64_t chunk;
  int rows_per_group;
  int64_t groups;
};

int rows_per_group_for(int64_t rows, int members, int cu_count, int per_cu) {
  // Slice kernels (no exchange): aim for one resident wave of groups; more
  // rows per group cut the dw partial traffic (one fp64 row per group).
  const int64_t target_groups =
      (static_cast<int64_t>(per_cu) * cu_count + members - 1) / members;
  int64_t r = (rows + target_groups - 1) / (target_groups > 0 ? target_groups : 1);
  if (r < 1) r = 1;
  if (r > 64) r = 64;
  return static_cast<int>(r);
}

// Group kernel (SPLIT): every member of every group must be running at
// once.  A member of a group waits for the others every row, and the
// hardware dispatcher does not reliably start a pending workgroup on a CU
// freed by a finished group while workgroups it would complete are
// spinning (measured: pending members started seconds late).  So the grid
// is at most one resident wave -- G groups, G a multiple of kDispensers
// (one dispenser subset per XCD) and G * P <= workgroups resident at once
// -- and each group loops over ceil(rows / G) rows.
int64_t coresident_groups(int members, int cu_count, int per_cu) {
  const int64_t resident = static_cast<int64_t>(per_cu) * cu_count;
  return resident / (static_cast<int64_t>(kDispensers) * members) * kDispensers;
}

int resolve_bwd(const credit_cfg* cfg, int64_t rows, int64_t cols, bool vec, int cu_count,
                BwdPlan* plan) {
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_bwd needs cols %% 8 == 0 and 16-byte aligned buffers");
  const int variant = cfg_variant(cfg);
  const int64_t nvec = cols / 8;
  int p = 0;
  int v = variant;
  if (v == CREDIT_VARIANT_AUTO) {
    // SPLIT when a power-of-two group of members with slices of at most
    // kBwdGroupCapacity vectors fits the device kDispensers times over.
    int p2 = 2;
    while (p2 * int64_t{kBwdGroupCapacity} < nvec) p2 *= 2;
    const int64_t chunk = (nvec + p2 - 1) / p2;
    const bool fits = p2 <= kMaxExchangeValues &&
                      coresident_groups(p2, cu_count, pick_for(kBwdGroup, chunk)->per_cu) > 0;
    v = nvec <= kBwdMaxCapacity ? CREDIT_VARIANT_STAGED
        : fits                  ? CREDIT_VARIANT_SPLIT
                                : CREDIT_VARIANT_READ;
  }
  if (v == CREDIT_VARIANT_STAGED) {
    if (nvec > kBwdMaxCapacity)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_bwd staged variant holds at most %d columns", kBwdMaxCapacity * 8);
    p = 1;
  } else if (v == CREDIT_VARIANT_SPLIT) {
    p = cfg_split(cfg);
    const int need = static_cast<int>((nvec + kBwdGroupCapacity - 1) / kBwdGroupCapacity);
    if (p == 0) {
      // A power of two: then G groups of P fill every resident slot.
      p = 2;
      while (p < need) p *= 2;
    }
    if (p < need)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_bwd split %d leaves more than %d vectors per member", p,
                       kBwdGroupCapacity);
    if (p > nvec) p = static_cast<int>(nvec);
  } else {  // READ: column tiles of the largest slice, c from the pre-pass
    p = static_cast<int>((nvec + kBwdMaxCapacity - 1) / kBwdMaxCapacity);
  }
  const Plan sp = plan_split(nvec, p);
  plan->variant = v;
  plan->members = sp.members;
  plan->chunk = sp.chunk;
  if (v == CREDIT_VARIANT_SPLIT && plan->members < 2) plan->variant = CREDIT_VARIANT_STAGED;
  if (plan->variant == CREDIT_VARIANT_SPLIT) {
    if (plan->members > kMaxExchangeValues)
      return set_error(CREDIT_ERR_UNSUPPORTED, "rmsnorm_bwd split %d exceeds %d members",
                       plan->members, kMaxExchangeValues);
    const int64_t g = coresident_groups(plan->members, cu_count,
                                        pick_for(kBwdGroup, plan->chunk)->per_cu);
    if (g == 0)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_bwd split %d: %d groups of it do not fit the device at once",
                       plan->members, kDispensers);
    const int64_t r = (rows + g - 1) / g;
    if (r > (int64_t{1} << 30))
      return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_bwd: %lld rows per group",
                       static_cast<long long>(r));
    plan->rows_per_group = static_cast<int>(r < 1 ? 1 : r);
  } else {
    plan->rows_per_group = rows_per_group_for(rows, plan->members, cu_count, 2);
  }
  plan->groups = (rows + plan->rows_per_group - 1) / plan->rows_per_group;
  return CREDIT_OK;
}

// Slot rows per group of the group kernel: a member publishes row k two
// steps before it needs row k's total, and a member reaches row k + 16 only
// after every member has polled row k, so 16 rows of slots suffice.
constexpr int kBwdRing = kGroupSlotRing;
int bwd_ring(const BwdPlan& p) { return p.variant == CREDIT_VARIANT_SPLIT ? kBwdRing : 1; }

size_t bwd_extra_bytes(const BwdPlan& p, int64_t rows, int64_t cols) {
  size_t b = align_up(static_cast<size_t>(p.groups) * cols * sizeof(double), 256);
  if (p.variant == CREDIT_VARIANT_READ) b += align_up(static_cast<size_t>(rows) * sizeof(float), 256);
  return b;
}

}  // namespace

size_t rmsnorm_fwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                             int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  if (resolve_fwd(&c, cols, cols % 8 == 0, &p) != CREDIT_OK) return 0;
  if (p.variant != CREDIT_VARIANT_SPLIT) return 0;
  int64_t groups = coresident_groups_bound(p.members, cu_count);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  return split_workspace_bytes(groups, p.members, 1, kSplitRing, 0);
}

size_t rmsnorm_fused_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int cu_count) {
  // Without a device query the group count is bounded by the resident
  // workgroups of the widest pick (one per CU): every shape's figure is an
  // upper bound of what the call acquires.
  if (cols % 8 != 0 || rows <= 0) return 0;
  const int64_t nvec = cols / 8;
  const int need = static_cast<int>((nvec + kBwdGroupCapacity - 1) / kBwdGroupCapacity);
  int p = split > 0 ? split : 1;
  while (split == 0 && p < need) p *= 2;
  if (p < need || p > kMaxFusedMembers) return 0;
  (void)variant;
  int64_t groups = coresident_groups_bound(p, cu_count);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  return split_workspace_bytes(groups, p, 2, kBwdRing,
                               align_up(static_cast<size_t>(groups) * cols * sizeof(double), 256));
}

size_t rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                             int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  BwdPlan p;
  if (resolve_bwd(&c, rows, cols, cols % 8 == 0, cu_count, &p) != CREDIT_OK) return 0;
  return split_workspace_bytes(padded_groups(p.groups), p.members, 1, bwd_ring(p),
                               bwd_extra_bytes(p, rows, cols));
}

// Fused plan: the group kernel with the fewest members (a power of two, or
// cfg->split) whose slices hold at most kBwdGroupCapacity vectors; one
// member when the row fits one workgroup.
struct FusedPlan {
  int members;
  int64_t chunk;
  int rows_per_group;
  int64_t groups;       // groups with rows
  int64_t grid_groups;  // padded to a multiple of kDispensers
  int dispensers;       // ticket subsets of the launch
};

int resolve_fused(const credit_cfg* cfg, int64_t rows, int64_t cols, int cu_count,
                  const FusedGroupPick** pick, FusedPlan* plan) {
  const int64_t nvec = cols / 8;
  const int need = static_cast<int>((nvec + kBwdGroupCapacity - 1) / kBwdGroupCapacity);
  int p = cfg_split(cfg);
  if (p == 0) {
    p = 1;
    while (p < need) p *= 2;
  }
  if (p < need)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd_bwd split %d leaves more than %d vectors per member", p,
                     kBwdGroupCapacity);
  if (p > nvec) p = static_cast<int>(nvec);
  const Plan sp = plan_split(nvec, p);
  if (sp.members > kMaxFusedMembers)
    return set_error(CREDIT_ERR_UNSUPPORTED, "rmsnorm_fwd_bwd: %d members (at most %d)",
                     sp.members, kMaxFusedMembers);
  *pick = pick_for(kFusedGroup, sp.chunk);
  int64_t fit = 0;
  CREDIT_TRY(credit::coresident_groups(reinterpret_cast<const void*>((*pick)->fn),
                                       (*pick)->threads + kWave, (*pick)->lds_bytes(),
                                       sp.members, &fit, &plan->dispensers));
  (void)cu_count;
  if (fit == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd_bwd: %d groups of %d members do not fit the device at once",
                     kDispensers, sp.members);
  const int64_t g = fit < padded_groups(rows) ? fit : padded_groups(rows);
  const int64_t r = (rows + g - 1) / g;
  if (r > (int64_t{1} << 30))
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_fwd_bwd: %lld rows per group",
                     static_cast<long long>(r));
  plan->members = sp.members;
  plan->chunk = sp.chunk;
  plan->rows_per_group = static_cast<int>(r);
  plan->groups = (rows + r - 1) / r;
  plan->grid_groups = padded_groups(plan->groups);
  return CREDIT_OK;
}

// ----------------------------------------------- allocation-free variant --
// credit_rmsnorm_bwd_bf16_noalloc runs the backward with its workspace (the
// layout of api_internal.hpp: watchdog header, counters, exchange slots,
// then the dweight partials) in this fixed device array instead of a
// hipMalloc'd buffer.  40 MiB covers the BASELINE shape (1024 x 131072:
// 5 MiB of header, counters and slots plus 16 MiB of fp64 partials) and any
// width up to 262144 at that grouping.  The array is zero at module load,
// which is the state the header, counters and slots need; every completed
// call leaves them so (dispensers return to zero, slot tags are fresh per
// launch), and the partials are written before they are read.
constexpr size_t kNoAllocScratchBytes = size_t{40} << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
char* g_noalloc_base[kNoAllocMaxDevices] = {};  // per device: scratch's device address

// The device address of `scratch` on the current device, looked up once
// per device.  The host-side name is only a handle for the lookup, never an
// address to pass to a kernel.
int noalloc_scratch(char** out) {
  int dev = 0;
  CREDIT_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(CREDIT_ERR_UNSUPPORTED, "allocation-free calls support devices 0..%d",
                     kNoAllocMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_base[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_failure(err, "hipGetSymbolAddress(scratch)");
    if (p == nullptr || reinterpret_cast<uintptr_t>(p) % 256 != 0)
      return set_error(CREDIT_ERR_HIP, "scratch has no 256-byte aligned device address");
    g_noalloc_base[dev] = static_cast<char*>(p);
  }
  *out = g_noalloc_base[dev];
  return CREDIT_OK;
}
}  // namespace

char* noalloc_scratch_base(int device) {
  if (device < 0 || device >= kNoAllocMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  return g_noalloc_base[device];
}

}  // namespace credit

using namespace credit;

extern "C" int credit_rmsnorm_fwd_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y,
                                       float* rstd, int64_t rows, int64_t cols, float eps,
                                       const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w, "w"));
  CREDIT_TRY(check_row_ptr(y, "y", rows));
  CREDIT_TRY(check_row_ptr(rstd, "rstd", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, 2, "x"));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (rows == 0) return CREDIT_OK;
  const bool vec = vec_ok(cols, {x, w, y});
  Plan plan;
  CREDIT_TRY(resolve_fwd(cfg, cols, vec, &plan));
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  if (plan.variant == CREDIT_VARIANT_READ) {
    if (vec)
      rmsnorm_fwd_read_kernel<256, true>
          <<<dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream>>>(x, w, y, rstd, c, eps);
    else
      rmsnorm_fwd_read_kernel<256, false>
          <<<dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream>>>(x, w, y, rstd, c, eps);
    return check_launch("rmsnorm_fwd_read_kernel");
  }
  if (fwd_takes_group(plan)) {
    static_assert(kFwdGroupThreads == 512 && kFwdGroupVpt == 4, "the instance below");
    auto fn = rmsnorm_fwd_group_kernel<512, 4, 4, 1>;
    const int threads = kFwdGroupThreads + 2 * kWave;
    int64_t fit = 0;
    int dispensers = 0;
    CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(fn), threads, 0,
                                 plan.members, &fit, &dispensers));
    if (fit == 0)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_fwd: %d groups of %d members do not fit the device", kDispensers,
                       plan.members);
    const int64_t g = fit < padded_groups(rows) ? fit : padded_groups(rows);
    const int64_t rows_per_group = (rows + g - 1) / g;
    const int64_t grid_groups = padded_groups((rows + rows_per_group - 1) / rows_per_group);
    // A group may take every row (the queue); its tags run L < 16 steps
    // past its last.
    const int64_t stages = rows + 16;
    if (stages > int64_t{credit::plan::kMaxLaunchStages})
      return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_fwd: %lld rows",
                       static_cast<long long>(rows));
    SplitWorkspace ws;
    CREDIT_TRY(acquire_split_workspace(cfg, grid_groups, plan.members, 2, kGroupSlotRing, 0, &ws));
    const uint32_t total = static_cast<uint32_t>(grid_groups * plan.members);
    hipLaunchKernelGGL(fn, dim3(total), dim3(threads), 0, stream, x, w, y, rstd,
                       static_cast<int>(rows), c, static_cast<int>(plan.chunk), plan.members,
                       static_cast<int>(rows_per_group), eps,
                       make_split_args(ws, total, static_cast<uint32_t>(stages), kGroupSlotRing,
                                       dispensers),
                       ws.counters + kQueueWord);
    return check_launch("rmsnorm_fwd_group_kernel");
  }
  const FwdPick* pick = pick_for(kFwd, plan.chunk);
  if (plan.variant == CREDIT_VARIANT_STAGED) {
    hipLaunchKernelGGL(pick->fn, dim3(static_cast<unsigned>(rows)), dim3(pick->threads), 0,
                       stream, x, w, y, rstd, c, static_cast<int>(plan.chunk), 1,
                       static_cast<int>(rows), eps, SplitArgs{});
    return check_launch("rmsnorm_fwd_slice_kernel");
  }
  int64_t groups = 0;
  int dispensers = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(pick->fn), pick->threads, 0,
                               plan.members, &groups, &dispensers));
  if (groups == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd: %d groups of %d members do not fit the device", kDispensers,
                     plan.members);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  const int64_t per_group = (rows + groups - 1) / groups;
  if (per_group > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_fwd: %lld rows per group",
                     static_cast<long long>(per_group));
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, 1, kSplitRing, 0, &ws));
  const uint32_t total = static_cast<uint32_t>(groups * plan.members);
  const SplitArgs sa =
      make_split_args(ws, total, static_cast<uint32_t>(per_group), kSplitRing, dispensers);
  hipLaunchKernelGGL(pick->fn, dim3(total), dim3(pick->threads), 0, stream, x, w, y, rstd, c,
                     static_cast<int>(plan.chunk), plan.members, static_cast<int>(rows), eps,
                     sa);
  return check_launch("rmsnorm_fwd_slice_kernel(split)");
}

extern "C" int credit_rmsnorm_bwd_bf16(const uint16_t* x, const uint16_t* w,
                                       const uint16_t* dy, const float* rstd, uint16_t* dx,
                                       float* dw, int64_t rows, int64_t cols,
                                       const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w, "w"));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_row_ptr(rstd, "rstd", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_ptr(dw, "dw"));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_cfg(cfg));
  if (rows > (int64_t{1} << 24))
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_bwd supports at most 2^24 rows");
  const bool vec = vec_ok(cols, {x, w, dy, dx, dw});
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  BwdPlan plan;
  CREDIT_TRY(resolve_bwd(cfg, rows, cols, vec, props->cu_count, &plan));
  hipStream_t stream = cfg_stream(cfg);
  if (rows == 0) {
    // No rows: dw is a sum over nothing.  A fill kernel, not a memset node,
    // so the call stays correct under stream capture.
    fill_f32_kernel<<<dim3(static_cast<unsigned>((cols + 255) / 256)), dim3(256), 0, stream>>>(
        dw, 0.0f, cols);
    return check_launch("fill_f32_kernel");
  }
  if (padded_groups(plan.groups) > kMaxGroupsPerLaunch)
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_bwd: %lld row groups exceed %d",
                     static_cast<long long>(plan.groups), kMaxGroupsPerLaunch);
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(cfg, padded_groups(plan.groups), plan.members, 1,
                                     bwd_ring(plan), bwd_extra_bytes(plan, rows, cols), &ws));
  double* dw_part = reinterpret_cast<double*>(ws.extra);
  float* rowdot = reinterpret_cast<float*>(
      ws.extra + align_up(static_cast<size_t>(plan.groups) * cols * sizeof(double), 256));
  const int c = static_cast<int>(cols);
  int mode = kBwdWhole;
  if (plan.variant == CREDIT_VARIANT_SPLIT) mode = kBwdExchange;
  // Ticketed launches cover whole dispenser subsets (padding groups exit).
  const int64_t grid_groups = mode == kBwdExchange ? padded_groups(plan.groups) : plan.groups;
  const uint32_t total = static_cast<uint32_t>(grid_groups * plan.members);
  if (plan.variant == CREDIT_VARIANT_READ) {
    mode = kBwdGiven;
    rmsnorm_bwd_rowdot_kernel<256>
        <<<dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream>>>(x, w, dy, rowdot, c);
    CREDIT_TRY(check_launch("rmsnorm_bwd_rowdot_kernel"));
  }
  if (mode == kBwdExchange) {
    const BwdGroupPick* pick = pick_for(kBwdGroup, plan.chunk);
    int64_t fit = 0;
    int dispensers = 0;
    CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(pick->fn), pick->threads + kWave,
                                 pick->lds_bytes(), plan.members, &fit, &dispensers));
    if (padded_groups(plan.groups) > fit)
      return set_error(CREDIT_ERR_UNSUPPORTED,
                       "rmsnorm_bwd: %lld groups of %d members exceed the %lld resident at once",
                       static_cast<long long>(padded_groups(plan.groups)), plan.members,
                       static_cast<long long>(fit));
    hipLaunchKernelGGL(pick->fn, dim3(total), dim3(pick->threads + kWave),
                       pick->lds_bytes(), stream, x, w, dy, rstd, dx, dw_part,
                       static_cast<int>(rows), c, static_cast<int>(plan.chunk), plan.members,
                       plan.rows_per_group,
                       make_split_args(ws, total, static_cast<uint32_t>(plan.rows_per_group),
                                       kBwdRing, dispensers));
    CREDIT_TRY(check_launch("rmsnorm_bwd_group_kernel"));
  } else {
    const BwdPick* pick = pick_for(kBwd, plan.chunk);
    hipLaunchKernelGGL(pick->fn, dim3(total), dim3(pick->threads), pick->lds_bytes(), stream, x,
                       w, dy, rstd, rowdot, dx, dw_part, static_cast<int>(rows), c,
                       static_cast<int>(plan.chunk), plan.members, plan.rows_per_group, mode,
                       SplitArgs{});
    CREDIT_TRY(check_launch("rmsnorm_bwd_slice_kernel"));
  }
  const unsigned reduce_blocks = static_cast<unsigned>((cols / 2 + 255) / 256);
  rmsnorm_dw_reduce_kernel<<<dim3(reduce_blocks), dim3(256), 0, stream>>>(
      dw_part, dw, static_cast<int>(plan.groups), c);
  return check_launch("rmsnorm_dw_reduce_kernel");
}

extern "C" int credit_rmsnorm_bwd_bf16_noalloc(const uint16_t* x, const uint16_t* w,
                                               const uint16_t* dy, const float* rstd,
                                               uint16_t* dx, float* dw, int64_t rows,
                                               int64_t cols, const credit_cfg* cfg) {
  CREDIT_TRY(check_cfg(cfg));
  if (cfg != nullptr && cfg->workspace != nullptr)
    return set_error(CREDIT_ERR_BAD_CONFIG,
                     "rmsnorm_bwd_noalloc takes no cfg->workspace (it uses the library's fixed "
                     "scratch array); pass the workspace to credit_rmsnorm_bwd_bf16 instead");
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  const size_t body = rmsnorm_bwd_workspace(rows, cols, cfg_variant(cfg), cfg_split(cfg),
                                            props->cu_count);
  const size_t need = kScratchOffset + body;
  if (need > kNoAllocScratchBytes)
    return set_error(CREDIT_ERR_WORKSPACE,
                     "rmsnorm_bwd_noalloc: %lld x %lld needs %zu bytes of scratch, more than "
                     "the fixed %zu-byte array; use credit_rmsnorm_bwd_bf16",
                     static_cast<long long>(rows), static_cast<long long>(cols), need,
                     kNoAllocScratchBytes);
  char* base = nullptr;
  CREDIT_TRY(noalloc_scratch(&base));
  credit_cfg c = cfg != nullptr ? *cfg : credit_cfg{nullptr, CREDIT_VARIANT_AUTO, 0, nullptr, 0};
  c.workspace = base;
  c.workspace_bytes = kNoAllocScratchBytes;
  const NoAllocScope no_alloc;  // no host-mapped watchdog word is allocated for it
  return credit_rmsnorm_bwd_bf16(x, w, dy, rstd, dx, dw, rows, cols, &c);
}

extern "C" int credit_rmsnorm_fwd_bwd_bf16(const uint16_t* x, const uint16_t* w,
                                           const uint16_t* dy, uint16_t* y, float* rstd,
                                           uint16_t* dx, float* dw, int64_t rows, int64_t cols,
                                           float eps, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w, "w"));
  CREDIT_TRY(check_row_ptr(dy, "dy", rows));
  CREDIT_TRY(check_row_ptr(y, "y", rows));
  CREDIT_TRY(check_row_ptr(rstd, "rstd", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_ptr(dw, "dw"));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_cfg(cfg));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (rows > (int64_t{1} << 24))
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_fwd_bwd supports at most 2^24 rows");
  const int variant = cfg_variant(cfg);
  if (variant == CREDIT_VARIANT_STAGED)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd_bwd: STAGED is not a variant of the fused call (AUTO, SPLIT, "
                     "or READ = the forward then the backward)");
  const bool vec = vec_ok(cols, {x, w, dy, y, dx, dw});
  if (variant == CREDIT_VARIANT_READ || (!vec && variant == CREDIT_VARIANT_AUTO) || rows == 0) {
    // The two passes: the forward's rstd feeds the backward.
    credit_cfg c = cfg != nullptr ? *cfg : credit_cfg{nullptr, 0, 0, nullptr, 0};
    c.variant = CREDIT_VARIANT_AUTO;
    c.split = 0;
    if (rows > 0) CREDIT_TRY(credit_rmsnorm_fwd_bf16(x, w, y, rstd, rows, cols, eps, &c));
    if (variant == CREDIT_VARIANT_READ) c.variant = CREDIT_VARIANT_READ;
    return credit_rmsnorm_bwd_bf16(x, w, dy, rstd, dx, dw, rows, cols, &c);
  }
  if (!vec)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "rmsnorm_fwd_bwd SPLIT needs cols %% 8 == 0 and 16-byte aligned buffers");
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  const FusedGroupPick* pick = nullptr;
  FusedPlan plan;
  CREDIT_TRY(resolve_fused(cfg, rows, cols, props->cu_count, &pick, &plan));
  if (plan.grid_groups > kMaxGroupsPerLaunch)
    return set_error(CREDIT_ERR_BAD_SHAPE, "rmsnorm_fwd_bwd: %lld row groups exceed %d",
                     static_cast<long long>(plan.groups), kMaxGroupsPerLaunch);
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(
      cfg, plan.grid_groups, plan.members, 2, kBwdRing,
      align_up(static_cast<size_t>(plan.groups) * cols * sizeof(double), 256), &ws));
  double* dw_part = reinterpret_cast<double*>(ws.extra);
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  const uint32_t total = static_cast<uint32_t>(plan.grid_groups * plan.members);
  hipLaunchKernelGGL(pick->fn, dim3(total), dim3(pick->threads + kWave), pick->lds_bytes(),
                     stream, x, w, dy, rstd, y, dx, dw_part, static_cast<int>(rows), c,
                     static_cast<int>(plan.chunk), plan.members, plan.rows_per_group, eps,
                     make_split_args(ws, total, static_cast<uint32_t>(plan.rows_per_group),
                                     kBwdRing, plan.dispensers));
  CREDIT_TRY(check_launch("rmsnorm_fused_group_kernel"));
  const unsigned reduce_blocks = static_cast<unsigned>((cols / 2 + 255) / 256);
  rmsnorm_dw_reduce_kernel<<<dim3(reduce_blocks), dim3(256), 0, stream>>>(
      dw_part, dw, static_cast<int>(plan.groups), c);
  return check_launch("rmsnorm_dw_reduce_kernel");
}
