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
__device__ __forceinline__ void softmax_fwd_slice_kernel_body(
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

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_fwd_slice_kernel(
    const float* __restrict__ x, float* __restrict__ p, float* __restrict__ rowmax,
    float* __restrict__ lse, int cols, int chunk, int members, int rows, SplitArgs sa) {
  softmax_fwd_slice_kernel_body<THREADS, VPT>(x, p, rowmax, lse, cols, chunk, members, rows, sa);
  split_leave(sa);
}

// One wave merges up to 64 (max, sum) partials, one per lane (`has`
// false: no partial): M = max m_l, S = sum s_l e^(m_l - M), each term an
// fp32 rescale summed in fp64 by a fixed tree; S rounded to fp32 once.  The
// maximum propagates NaN; a lane with s = 0 adds nothing (also when its m
// is -inf).  Every lane gets the result.
__device__ __forceinline__ void merge_maxsum_lanes(bool has, float m, float s, float* M_out,
                                                   float* S_out) {
  const float M = wave_reduce(has ? m : kNegInf, MaxOp{});
  const double term = has && s != 0.0f ? static_cast<double>(s) * exp_accurate(m - M) : 0.0;
  *M_out = M;
  *S_out = static_cast<float>(wave_reduce_sum_f64(term));
}

// SPLIT variant for rows wider than one workgroup: a co-resident wave of G
// row groups, each group P members that hold 1/P of every one of its rows
// (group g: rows g, g + G, g + 2G, ...), pipelined four rows deep.  The workgroup is THREADS data lanes (VPT
// f32x4 of the member's slice per lane and row) plus one communication wave.
//
// In the step of row i each data wave issues the loads of row i+3, reduces
// row i+2 (loaded a step earlier) to its wave partial (m_w, s_w) -- m_w the
// wave maximum, s_w = sum e^(x - m_w) -- replacing the row's values by
// e^(x - m_w) in registers, and counts itself in with an LDS atomic; the
// wave that arrives last merges the wave partials in wave order and
// publishes the member's (m, s) of row i+2.  The communication wave polls
// each row's exchange in order, merges the members' partials in member
// order into the row's (M, S), writes them into a 4-entry LDS ring and
// advances an LDS ready count.  A data wave then waits (LDS spin) for row
// i's (M, S) and writes p = e^(x - m_w) * (e^(m_w - M) / S): one exponential
// per element, the second pass a multiply.  Row i is published two steps
// before it is needed, so the exchange round trip overlaps the loads and
// stores of the rows around it, and no wave ever waits for another wave's
// loads (vmcnt is per wave: the polling wave issues no row traffic).  LDS
// slots of row k are reused by row k+4 only, which a wave reaches after row
// k+3's total is ready, i.e. after every access to them for row k.  Every
// wait ends: the poll is bounded (watchdog), and the ready count then still
// advances.
//
// Row traffic goes through buffer resources whose num_records covers the
// member's slice (0 for a row beyond the group): out-of-range lanes read
// zeros, masked to -inf / 0, and drop their stores; no branch surrounds a
// load or store, so the waitcnt pass keeps rows i+1..i+3 in flight.
// Buffer J of four statically named row buffers (J a constant, so the
// rotation stays in registers).
template <int J, typename T>
__device__ __forceinline__ T& pick4(T& a, T& b, T& c, T& d) {
  if constexpr (J == 0) return a;
  else if constexpr (J == 1) return b;
  else if constexpr (J == 2) return c;
  else return d;
}

template <int THREADS, int VPT, bool PARK = false>
__device__ __forceinline__ void softmax_fwd_group_kernel_body(
    const float* __restrict__ x, float* __restrict__ p, float* __restrict__ rowmax,
    float* __restrict__ lse, int rows, int cols, int chunk, int members, int rows_per_group,
    SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  // Rows between their publish and their finish: 2, or 4 with PARK (two of
  // them parked in LDS).  The per-row LDS rings hold every row from the
  // slowest wave's finish to the comm wave's newest total: RING entries.
  constexpr int RING = PARK ? 8 : 4;
  __shared__ float wmax[RING][NW];    // wave partials of row k at [(k - r0) % RING]
  __shared__ double wsum[RING][NW];
  __shared__ float ring_m[RING];      // group (M, S) of row k at [(k - r0) % RING]
  __shared__ float ring_s[RING];
  __shared__ uint32_t arrivals[RING];
  __shared__ uint32_t ready;          // rows r0 .. r0 + ready - 1 have (M, S)
  // PARK: two published rows of e^(x - m_w), lane-private ([slot][q][lane]):
  // each lane reads back only what it wrote, so no barrier guards a slot.
  __shared__ f32x4 parked[PARK ? 2 * VPT * THREADS : 1];
  const int tid = threadIdx.x;
  if (tid < RING) arrivals[tid] = 0;
  if (tid == 0) ready = 0;
  const SplitGroup g = split_join(sa, members, 2);  // its barrier covers the stores above
  // Rows are dealt to the G groups round-robin (group g's i-th row is
  // g + i G), so the rows in flight at any moment are adjacent in memory;
  // i below counts the group's rows and row_of(i) is the tensor row.
  // G: the groups that take rows (the launch pads the grid to a multiple
  // of the dispensers; padding groups, and their dweight partial rows where
  // there are any, stay out).  Each takes at most rows_per_group rows, the
  // host's bound on its exchange tags.
  const int G = (rows + rows_per_group - 1) / rows_per_group;
  if (g.group >= G) return;  // padding group
  const int r0 = 0;
  const int r1 = (rows - g.group + G - 1) / G;
  auto row_of = [&](int i) { return g.group + i * G; };
  const int nvec = cols >> 2;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;

  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS) {
    // ---- communication wave: merge every row's member partials ----
    const int lane = tid & (kWave - 1);
    for (int k = r0; k < r1; ++k) {
      const uint32_t bits = split_poll(g, k - r0, 2);
      // Lane m < P holds member m's (m, s): s sits P lanes up.
      const uint32_t sbits = static_cast<uint32_t>(__shfl(static_cast<int>(bits), lane + members));
      float M, S;
      merge_maxsum_lanes(lane < members, __builtin_bit_cast(float, bits),
                         __builtin_bit_cast(float, sbits), &M, &S);
      if (tid == THREADS) {
        ring_m[(k - r0) & (RING - 1)] = M;
        ring_s[(k - r0) & (RING - 1)] = S;
        __hip_atomic_store(&ready, static_cast<uint32_t>(k - r0 + 1), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
        if (g.member == 0) {
          rowmax[row_of(k)] = M;
          lse[row_of(k)] = static_cast<float>(static_cast<double>(M) + ::log(static_cast<double>(S)));
        }
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
    f32x4 v[VPT];
  };
  Row b0, b1, b2, b3;
  auto load_row = [&](Row& b, int r) {
    const bool live = r < r1;
    const size_t off =
        static_cast<size_t>(row_of(live ? r : r0)) * cols + 4 * static_cast<size_t>(v0);
    const buffer_rsrc_t xs = make_rsrc(x + off, live ? slice_bytes : 0u);
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      b.v[q] = __builtin_bit_cast(f32x4, buffer_load_nt(xs, lane_off + q * kStride));
  };
  // Row k -> e^(x - m_w) in place; the last wave in publishes the member's
  // (m, s) of row k.
  auto publish_row = [&](Row& b, int k) {
    float lm = kNegInf;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      lm = lane_off + q * kStride < slice_bytes ? fmax_nan(lm, max4(b.v[q])) : lm;
    const float wm = wave_reduce(lm, MaxOp{});
    float ls = 0.0f;
    if (wm != kNegInf) {
#pragma unroll
      for (int q = 0; q < VPT; ++q) {
        const f32x4 e = prob4(b.v[q], wm, 1.0f);
        b.v[q] = lane_off + q * kStride < slice_bytes ? e : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        ls += (b.v[q].x + b.v[q].y) + (b.v[q].z + b.v[q].w);
      }
    } else {
#pragma unroll
      for (int q = 0; q < VPT; ++q) b.v[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const double ws = wave_reduce_sum_f64(static_cast<double>(ls));
    const int slot = (k - r0) & (RING - 1);
    uint32_t t = 0;
    if (lead) {
      wmax[slot][wid] = wm;
      wsum[slot][wid] = ws;
      t = __hip_atomic_fetch_add(&arrivals[slot], 1u, __ATOMIC_ACQ_REL,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (__builtin_amdgcn_readfirstlane(t) == NW - 1) {
      // Last wave in: lane w merges wave w's partial.
      const int lane = tid & (kWave - 1);
      const bool has = lane < NW;
      float M, S;
      merge_maxsum_lanes(has, has ? wmax[slot][lane] : kNegInf,
                         has ? static_cast<float>(wsum[slot][lane]) : 0.0f, &M, &S);
      if (lead) {
        arrivals[slot] = 0;
        split_publish_at(g, k - r0, 0, M);
        split_publish_at(g, k - r0, 1, S);
      }
    }
  };
  // Waits for row r's (M, S); returns the wave's output scale for it.
  auto row_scale = [&](int r) {
    const int slot = (r - r0) & (RING - 1);
    const uint32_t need = static_cast<uint32_t>(r - r0 + 1);
    while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < need)
      __builtin_amdgcn_s_sleep(1);
    const float M = ring_m[slot];
    const float S = ring_s[slot];
    // e^(m_w - M) / S; 0/0 (NaN) for a row of -inf, as torch.softmax.
    const float mw = wmax[slot][wid];
    return (mw == kNegInf ? 0.0f : exp_accurate(mw - M)) / S;
  };
  auto out_rsrc = [&](int r) {
    const size_t off = static_cast<size_t>(row_of(r)) * cols + 4 * static_cast<size_t>(v0);
    return make_rsrc(p + off, slice_bytes);
  };
  auto finish_row = [&](const Row& b, int r) {
    const float f = row_scale(r);
    const buffer_rsrc_t out = out_rsrc(r);
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      buffer_store_nt(out, lane_off + q * kStride, __builtin_bit_cast(u32x4, b.v[q] * f));
  };
  if constexpr (PARK) {
    // Row k lives in buffer k % 4 from its load to its park.  Step i: load
    // row i+5, publish row i+4, finish row i from LDS slot i % 2, park row
    // i+2 there: a row is published four steps before its total is needed.
    auto park = [&](const Row& b, int slot) {
#pragma unroll
      for (int q = 0; q < VPT; ++q) parked[(slot * VPT + q) * THREADS + tid] = b.v[q];
    };
    auto finish_parked = [&](int r, int slot) {
      const float f = row_scale(r);
      const buffer_rsrc_t out = out_rsrc(r);
#pragma unroll
      for (int q = 0; q < VPT; ++q)
        buffer_store_nt(out, lane_off + q * kStride,
                        __builtin_bit_cast(u32x4, parked[(slot * VPT + q) * THREADS + tid] * f));
    };
    auto step = [&]<int S>(std::integral_constant<int, S>, int i) {
      load_row(pick4<(S + 1) & 3>(b0, b1, b2, b3), i + 5);
      __builtin_amdgcn_sched_barrier(0);
      if (i + 4 < r1) publish_row(pick4<S>(b0, b1, b2, b3), i + 4);
      finish_parked(i, S & 1);
      park(pick4<(S + 2) & 3>(b0, b1, b2, b3), S & 1);
    };
    load_row(b0, r0);
    load_row(b1, r0 + 1);
    load_row(b2, r0 + 2);
    load_row(b3, r0 + 3);
    publish_row(b0, r0);
    park(b0, 0);
    load_row(b0, r0 + 4);
    if (r0 + 1 < r1) publish_row(b1, r0 + 1);
    park(b1, 1);
    if (r0 + 2 < r1) publish_row(b2, r0 + 2);
    if (r0 + 3 < r1) publish_row(b3, r0 + 3);
    int i = r0;
    for (; i + 3 < r1; i += 4) {
      step(std::integral_constant<int, 0>{}, i);
      step(std::integral_constant<int, 1>{}, i + 1);
      step(std::integral_constant<int, 2>{}, i + 2);
      step(std::integral_constant<int, 3>{}, i + 3);
    }
    if (i < r1) step(std::integral_constant<int, 0>{}, i);
    if (i + 1 < r1) step(std::integral_constant<int, 1>{}, i + 1);
    if (i + 2 < r1) step(std::integral_constant<int, 2>{}, i + 2);
    return;
  }
  auto step = [&](Row& cur, Row& r2, Row& fut, int i) {
    load_row(fut, i + 3);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < r1) publish_row(r2, i + 2);
    finish_row(cur, i);
  };

  load_row(b0, r0);
  load_row(b1, r0 + 1);
  load_row(b2, r0 + 2);
  publish_row(b0, r0);
  if (r0 + 1 < r1) publish_row(b1, r0 + 1);
  // Rotate the four buffers through statically named registers.
  int i = r0;
  for (; i + 3 < r1; i += 4) {
    step(b0, b2, b3, i);
    step(b1, b3, b0, i + 1);
    step(b2, b0, b1, i + 2);
    step(b3, b1, b2, i + 3);
  }
  if (i < r1) step(b0, b2, b3, i);
  if (i + 1 < r1) step(b1, b3, b0, i + 1);
  if (i + 2 < r1) step(b2, b0, b1, i + 2);
}

template <int THREADS, int VPT, bool PARK = false>
__global__ __launch_bounds__(THREADS + kWave)
__attribute__((amdgpu_waves_per_eu(THREADS <= 512 && VPT <= 4 ? 4 : 3, 8))) void softmax_fwd_group_kernel(
    const float* __restrict__ x, float* __restrict__ p, float* __restrict__ rowmax,
    float* __restrict__ lse, int rows, int cols, int chunk, int members, int rows_per_group,
    SplitArgs sa) {
  softmax_fwd_group_kernel_body<THREADS, VPT, PARK>(x, p, rowmax, lse, rows, cols, chunk, members, rows_per_group, sa);
  split_leave(sa);
}

// Backward group kernel (SPLIT on rows wider than one workgroup): the row
// pipeline of softmax_fwd_group_kernel with one exchanged value per row,
// c = sum_j p*dy.  THREADS data lanes hold VPT f32x4 of p and of dy per row
// in four rotating row buffers; one extra communication wave polls each
// row's exchange into a 4-entry LDS ring.  At step i a data wave issues the
// loads of row i+3, reduces row i+2 to its wave partial (the last wave in
// adds the wave partials in wave order and publishes the member's), then
// waits for row i's group total and writes dx = p * (dy - c): the exchange
// round trip has two steps to complete and no workgroup barrier sits in the
// loop.  Buffer resources cover the member's slice (0 for a row beyond the
// group), so no load or store is under a branch.  PARK moves two published
// rows into LDS, so each row is published four steps before its total is
// needed, with the same four register buffers (the forward's scheme).
template <int THREADS, int VPT, bool PARK = false>
__device__ __forceinline__ void softmax_bwd_group_kernel_body(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int rows,
    int cols, int chunk, int members, int rows_per_group, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  // Rows between publish and finish: 2, or 4 with PARK (two parked in LDS);
  // the per-row LDS rings hold RING entries.
  constexpr int RING = PARK ? 8 : 4;
  __shared__ double red[RING][NW];  // wave partials of row k at [(k - r0) % RING]
  __shared__ double ring[RING];     // group totals of row k at [(k - r0) % RING]
  __shared__ uint32_t arrivals[RING];
  // PARK: p and dy of two published rows, lane-private ([slot][p/dy][q][lane]).
  __shared__ f32x4 parked[PARK ? 2 * 2 * VPT * THREADS : 1];
  __shared__ uint32_t ready;     // rows r0 .. r0 + ready - 1 have totals
  const int tid = threadIdx.x;
  if (tid < RING) arrivals[tid] = 0;
  if (tid == 0) ready = 0;
  const SplitGroup g = split_join(sa, members, 1);  // its barrier covers the stores above
  // Rows are dealt to the G groups round-robin (group g's i-th row is
  // g + i G), so the rows in flight at any moment are adjacent in memory;
  // i below counts the group's rows and row_of(i) is the tensor row.
  // G: the groups that take rows (the launch pads the grid to a multiple
  // of the dispensers; padding groups, and their dweight partial rows where
  // there are any, stay out).  Each takes at most rows_per_group rows, the
  // host's bound on its exchange tags.
  const int G = (rows + rows_per_group - 1) / rows_per_group;
  if (g.group >= G) return;  // padding group
  const int r0 = 0;
  const int r1 = (rows - g.group + G - 1) / G;
  auto row_of = [&](int i) { return g.group + i * G; };
  const int nvec = cols >> 2;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;

  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS) {
    // ---- communication wave: every row's group total, in row order ----
    for (int k = r0; k < r1; ++k) {
      const uint32_t bits = split_poll(g, k - r0, 1);
      const double dot = split_wave_sum(bits, members, 0);
      if (tid == THREADS) {
        ring[(k - r0) & (RING - 1)] = dot;
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
    f32x4 p[VPT], d[VPT];
  };
  Row b0, b1, b2, b3;
  auto load_row = [&](Row& b, int r) {
    const bool live = r < r1;
    const size_t off =
        static_cast<size_t>(row_of(live ? r : r0)) * cols + 4 * static_cast<size_t>(v0);
    const buffer_rsrc_t ps = make_rsrc(p + off, live ? slice_bytes : 0u);
    const buffer_rsrc_t ds = make_rsrc(dy + off, live ? slice_bytes : 0u);
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      b.p[q] = slice_load(ps, lane_off + q * kStride);
      b.d[q] = slice_load(ds, lane_off + q * kStride);
    }
  };
  auto publish_row = [&](const Row& b, int k) {
    float part = 0.0f;  // lanes beyond the slice hold zeros
#pragma unroll
    for (int q = 0; q < VPT; ++q) part += dot4(b.p[q], b.d[q]);
    const double v = wave_reduce_sum_f64(static_cast<double>(part));
    const int slot = (k - r0) & (RING - 1);
    if (lead) {
      red[slot][wid] = v;
      const uint32_t t = __hip_atomic_fetch_add(&arrivals[slot], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
      if (t == NW - 1) {
        double s = red[slot][0];
#pragma unroll
        for (int q = 1; q < NW; ++q) s += red[slot][q];
        arrivals[slot] = 0;
        split_publish_at(g, k - r0, 0, s);
      }
    }
  };
  auto wait_total = [&](int i) {
    const uint32_t need = static_cast<uint32_t>(i - r0 + 1);
    while (__hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < need)
      __builtin_amdgcn_s_sleep(1);
    return ring[(i - r0) & (RING - 1)];
  };
  auto finish_row = [&](const Row& b, int r, double dot) {
    const float c = static_cast<float>(dot);
    const size_t off = static_cast<size_t>(row_of(r)) * cols + 4 * static_cast<size_t>(v0);
    const buffer_rsrc_t out = make_rsrc(dx + off, slice_bytes);
#pragma unroll
    for (int q = 0; q < VPT; ++q) slice_store(out, lane_off + q * kStride, grad4(b.p[q], b.d[q], c));
  };
  if constexpr (PARK) {
    // Row k lives in buffer k % 4 from its load to its park.  Step i: load
    // row i+5, publish row i+4, finish row i from LDS slot i % 2, park row
    // i+2 there: a row is published four steps before its total is needed.
    auto park = [&](const Row& b, int slot) {
#pragma unroll
      for (int q = 0; q < VPT; ++q) {
        parked[((slot * 2 + 0) * VPT + q) * THREADS + tid] = b.p[q];
        parked[((slot * 2 + 1) * VPT + q) * THREADS + tid] = b.d[q];
      }
    };
    auto step = [&]<int S>(std::integral_constant<int, S>, int i) {
      load_row(pick4<(S + 1) & 3>(b0, b1, b2, b3), i + 5);
      __builtin_amdgcn_sched_barrier(0);
      if (i + 4 < r1) publish_row(pick4<S>(b0, b1, b2, b3), i + 4);
      const float c = static_cast<float>(wait_total(i));
      const size_t off = static_cast<size_t>(row_of(i)) * cols + 4 * static_cast<size_t>(v0);
      const buffer_rsrc_t out = make_rsrc(dx + off, slice_bytes);
#pragma unroll
      for (int q = 0; q < VPT; ++q)
        slice_store(out, lane_off + q * kStride,
                    grad4(parked[(((S & 1) * 2 + 0) * VPT + q) * THREADS + tid],
                          parked[(((S & 1) * 2 + 1) * VPT + q) * THREADS + tid], c));
      park(pick4<(S + 2) & 3>(b0, b1, b2, b3), S & 1);
    };
    load_row(b0, r0);
    load_row(b1, r0 + 1);
    load_row(b2, r0 + 2);
    load_row(b3, r0 + 3);
    publish_row(b0, r0);
    park(b0, 0);
    load_row(b0, r0 + 4);
    if (r0 + 1 < r1) publish_row(b1, r0 + 1);
    park(b1, 1);
    if (r0 + 2 < r1) publish_row(b2, r0 + 2);
    if (r0 + 3 < r1) publish_row(b3, r0 + 3);
    int i = r0;
    for (; i + 3 < r1; i += 4) {
      step(std::integral_constant<int, 0>{}, i);
      step(std::integral_constant<int, 1>{}, i + 1);
      step(std::integral_constant<int, 2>{}, i + 2);
      step(std::integral_constant<int, 3>{}, i + 3);
    }
    if (i < r1) step(std::integral_constant<int, 0>{}, i);
    if (i + 1 < r1) step(std::integral_constant<int, 1>{}, i + 1);
    if (i + 2 < r1) step(std::integral_constant<int, 2>{}, i + 2);
    return;
  }
  // Step of row i: cur = row i, r2 = row i+2 (loaded), fut receives row i+3.
  auto step = [&](Row& cur, Row& r2, Row& fut, int i) {
    load_row(fut, i + 3);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < r1) publish_row(r2, i + 2);
    finish_row(cur, i, wait_total(i));
  };

  load_row(b0, r0);
  load_row(b1, r0 + 1);
  load_row(b2, r0 + 2);
  publish_row(b0, r0);
  if (r0 + 1 < r1) publish_row(b1, r0 + 1);
  // Rotate the four buffers through statically named registers.
  int i = r0;
  for (; i + 3 < r1; i += 4) {
    step(b0, b2, b3, i);
    step(b1, b3, b0, i + 1);
    step(b2, b0, b1, i + 2);
    step(b3, b1, b2, i + 3);
  }
  if (i < r1) step(b0, b2, b3, i);
  if (i + 1 < r1) step(b1, b3, b0, i + 1);
  if (i + 2 < r1) step(b2, b0, b1, i + 2);
}

template <int THREADS, int VPT, bool PARK = false>
__global__ __launch_bounds__(THREADS + kWave)
__attribute__((amdgpu_waves_per_eu(3, 8))) void softmax_bwd_group_kernel(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int rows,
    int cols, int chunk, int members, int rows_per_group, SplitArgs sa) {
  softmax_bwd_group_kernel_body<THREADS, VPT, PARK>(p, dy, dx, rows, cols, chunk, members, rows_per_group, sa);
  split_leave(sa);
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
__device__ __forceinline__ void softmax_bwd_slice_kernel_body(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int cols,
    int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ double sred[1][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 1, chunk, cols >> 2, sa);
  const uint32_t lane_off = threadIdx.x * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  for (int row = sl.row; row < rows; row += sl.step) {
    const size_t off = static_cast<size_t>(row) * cols;
    const buffer_rsrc_t pr = slice_rsrc(p + off, sl);
    const buffer_rsrc_t dr = slice_rsrc(dy + off, sl);
    f32x4 pv[VPT], dv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      pv[k] = slice_load(pr, lane_off + k * kStride);
      dv[k] = slice_load(dr, lane_off + k * kStride);
    }
    float ld = 0.0f;  // beyond the slice p = dy = 0
#pragma unroll
    for (int k = 0; k < VPT; ++k) ld += dot4(pv[k], dv[k]);
    double dot[1] = {ld};
    block_reduce_sum_f64_multi<NW, 1>(dot, sred);
    if (members > 1) {
      if (threadIdx.x == 0) split_publish(g, 0, dot[0]);
      split_exchange(g);
      dot[0] = split_sum(g, 0);
    }
    const float d = static_cast<float>(dot[0]);
    const buffer_rsrc_t xr = slice_rsrc(dx + off, sl);
#pragma unroll
    for (int k = 0; k < VPT; ++k) slice_store(xr, lane_off + k * kStride, grad4(pv[k], dv[k], d));
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_bwd_slice_kernel(
    const float* __restrict__ p, const float* __restrict__ dy, float* __restrict__ dx, int cols,
    int chunk, int members, int rows, SplitArgs sa) {
  softmax_bwd_slice_kernel_body<THREADS, VPT>(p, dy, dx, cols, chunk, members, rows, sa);
  split_leave(sa);
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
__device__ __forceinline__ void softmax_logits_bwd_slice_kernel_body(
    const float* __restrict__ logits, const float* __restrict__ dy, float* __restrict__ dx,
    int cols, int chunk, int members, int rows, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  __shared__ float wmax[NW];
  __shared__ float wsum[NW];
  __shared__ double dred[1][NW];
  SplitGroup g;
  const Slice sl = slice_of(&g, members, 2, chunk, cols >> 2, sa);
  const uint32_t lane_off = threadIdx.x * 16u;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  constexpr uint32_t kStride = THREADS * 16u;
  const uint32_t slice_bytes = static_cast<uint32_t>(sl.vlen) * 16u;
  for (int row = sl.row; row < rows; row += sl.step) {
    const size_t off = static_cast<size_t>(row) * cols;
    const buffer_rsrc_t lr = slice_rsrc(logits + off, sl);
    const buffer_rsrc_t dr = slice_rsrc(dy + off, sl);
    f32x4 v[VPT], dv[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      v[k] = slice_load(lr, lane_off + k * kStride);
      dv[k] = slice_load(dr, lane_off + k * kStride);
    }
    // Wave partial (m_w, s_w); the row's values become e^(x - m_w) in place
    // (zeros beyond the slice), so p costs one exponential per element.
    float lm = kNegInf;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
      lm = lane_off + k * kStride < slice_bytes ? fmax_nan(lm, max4(v[k])) : lm;
    const float wm = wave_reduce(lm, MaxOp{});
    float ls = 0.0f;
    if (wm != kNegInf) {
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const f32x4 e = prob4(v[k], wm, 1.0f);
        v[k] = lane_off + k * kStride < slice_bytes ? e : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        ls += (v[k].x + v[k].y) + (v[k].z + v[k].w);
      }
    } else {
#pragma unroll
      for (int k = 0; k < VPT; ++k) v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const double ws = wave_reduce_sum_f64(static_cast<double>(ls));
    if (lane == 0) {
      wmax[wid] = wm;
      wsum[wid] = static_cast<float>(ws);
    }
    __syncthreads();
    float M, S;
    merge_maxsum_lanes(lane < NW, lane < NW ? wmax[lane] : kNegInf,
                       lane < NW ? wsum[lane] : 0.0f, &M, &S);
    double Sd = S;
    if (members > 1) {
      if (threadIdx.x == 0) {
        split_publish(g, 0, static_cast<double>(M));
        split_publish(g, 1, Sd);
      }
      split_exchange(g);
      split_merge_maxsum(g, &M, &Sd);
    }
    // p = e^(x - m_w) * e^(m_w - M) / S; 0/0 (NaN) on a row of -inf.
    const float f = (wm == kNegInf ? 0.0f : exp_accurate(wm - M)) / static_cast<float>(Sd);
    float ld = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      v[k] = v[k] * f;
      ld += dot4(v[k], dv[k]);
    }
    double dot[1] = {ld};
    block_reduce_sum_f64_multi<NW, 1>(dot, dred);
    if (members > 1) {
      if (threadIdx.x == 0) split_publish(g, 0, dot[0]);
      split_exchange(g, 1);  // stage 2 carries the dot only
      dot[0] = split_sum(g, 0);
    }
    const float d = static_cast<float>(dot[0]);
    const buffer_rsrc_t xr = slice_rsrc(dx + off, sl);
#pragma unroll
    for (int k = 0; k < VPT; ++k) slice_store(xr, lane_off + k * kStride, grad4(v[k], dv[k], d));
  }
}

template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void softmax_logits_bwd_slice_kernel(
    const float* __restrict__ logits, const float* __restrict__ dy, float* __restrict__ dx,
    int cols, int chunk, int members, int rows, SplitArgs sa) {
  softmax_logits_bwd_slice_kernel_body<THREADS, VPT>(logits, dy, dx, cols, chunk, members, rows, sa);
  split_leave(sa);
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

using BwdGroupFn = void (*)(const float*, const float*, float*, int, int, int, int, int,
                            SplitArgs);
const Pick<BwdGroupFn> kBwdGroup[] = {
    {softmax_bwd_group_kernel<64, 4>, 64, 256},
    {softmax_bwd_group_kernel<128, 4>, 128, 512},
    {softmax_bwd_group_kernel<256, 4>, 256, 1024},
    {softmax_bwd_group_kernel<512, 4, true>, 512, 2048},
};
constexpr int64_t kBwdGroupCapacity = 2048;

constexpr int64_t kFwdCapacity = 16384;
constexpr int64_t kBwdCapacity = 8192;
// AUTO slices of the softmax backward on rows wider than one workgroup:
// 512-lane members, two per CU (at 512 x 262144: 16 members 5.18 TB/s,
// 8 members of 8192 vectors 4.89 TB/s).
constexpr int64_t kBwdAutoSlice = 4096;

// Forward group kernel (SPLIT on rows wider than one workgroup): four row
// buffers of VPT f32x4 per lane; 448-512 data lanes + 1 wave give two
// workgroups per CU, 960 + 1 one.
using FwdGroupFn = void (*)(const float*, float*, float*, float*, int, int, int, int, int,
                            SplitArgs);
const Pick<FwdGroupFn> kFwdGroup[] = {
    {softmax_fwd_group_kernel<64, 4>, 64, 256},
    {softmax_fwd_group_kernel<128, 4>, 128, 512},
    {softmax_fwd_group_kernel<192, 4>, 192, 768},
    {softmax_fwd_group_kernel<448, 4>, 448, 1792},
    {softmax_fwd_group_kernel<512, 4>, 512, 2048},
    {softmax_fwd_group_kernel<960, 4>, 960, 3840},
    {softmax_fwd_group_kernel<512, 8, true>, 512, 4096},
};
constexpr int64_t kFwdGroupCapacity = 4096;
// Slot rows per group: a member publishes row k two steps before it needs
// row k's total and reaches row k + 16 only after every member has polled
// row k.
constexpr int kGroupRing = 16;
constexpr int kMaxGroupMembers = kMaxExchangeValues / 2;  // (m, s) per member

bool fwd_group_ok(const Plan& plan) {
  return plan.variant == CREDIT_VARIANT_SPLIT && plan.members <= kMaxGroupMembers &&
         plan.chunk <= kFwdGroupCapacity;
}

// Forward plan.  AUTO on a row wider than one workgroup takes the group
// kernel with the fewest members (a power of two) whose slices fit it:
// fewer members wait for fewer stragglers at every row (measured at
// 512 x 262144: 16 members 212 us, 32 members 239 us, the 4-member slice
// kernel without the pipeline 249 us).
int resolve_fwd(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  const int64_t nvec = cols / 4;
  if (cfg_variant(cfg) == CREDIT_VARIANT_AUTO && vec && nvec > kFwdCapacity) {
    int p = 2;
    while (p * kFwdGroupCapacity < nvec) p *= 2;
    if (p <= kMaxGroupMembers) {
      const int64_t chunk = (nvec + p - 1) / p;
      *plan = Plan{CREDIT_VARIANT_SPLIT, static_cast<int>((nvec + chunk - 1) / chunk), chunk};
      return CREDIT_OK;
    }
  }
  return resolve(cfg, cols, vec, kFwdCapacity, "softmax_fwd", plan);
}

// At most 32 members, as the forward; wider groups take the slice kernel.
// A 64-member launch of the 256-lane kernel ran into the exchange watchdog
// at 9 x 262144 when the launch sizing still put one group across every
// slot of each 8-way ticket subset (two workgroups per CU, G*P equal to the
// resident count): one slot withheld from such a launch strands that group
// (tests/cpp/split_protocol_model.cpp, withheld_old).  The sizing now keeps
// two groups per subset (split_plan.hpp, dispensers_for); the 64-member
// group kernel is not needed by any shape AUTO picks and stays off.
constexpr int kMaxBwdGroupMembers = 32;

bool bwd_group_ok(const Plan& plan) {
  return plan.variant == CREDIT_VARIANT_SPLIT && plan.members <= kMaxBwdGroupMembers &&
         plan.chunk <= kBwdGroupCapacity;
}

// Backward plan.  AUTO on a row wider than one workgroup takes the group
// kernel with the fewest members (a power of two) whose slices fit it, as
// the forward does; rows wider than 32 such members cover take slices.
int resolve_bwd(const credit_cfg* cfg, int64_t cols, bool vec, Plan* plan) {
  const int64_t nvec = cols / 4;
  if (cfg_variant(cfg) == CREDIT_VARIANT_AUTO && vec && nvec > kBwdCapacity) {
    int p = 2;
    while (p * kBwdGroupCapacity < nvec) p *= 2;
    if (p <= kMaxBwdGroupMembers) {
      const int64_t chunk = (nvec + p - 1) / p;
      *plan = Plan{CREDIT_VARIANT_SPLIT, static_cast<int>((nvec + chunk - 1) / chunk), chunk};
      return CREDIT_OK;
    }
  }
  return resolve(cfg, cols, vec, kBwdCapacity, "softmax_bwd", plan, kBwdAutoSlice);
}

// Rows per group and groups of a group-kernel launch: as many groups as
// fit the device at once (a multiple of kDispensers); the kernels deal the
// rows to them round-robin, at most rows_per_group each.
int plan_row_groups(const void* fn, int threads, int members, int64_t rows, int* rows_per_group,
                    int64_t* groups, int* dispensers, const char* name) {
  int64_t fit = 0;
  CREDIT_TRY(coresident_groups(fn, threads, 0, members, &fit, dispensers));
  if (fit == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED, "%s: %d groups of %d members do not fit the device",
                     name, kDispensers, members);
  const int64_t g = fit < padded_groups(rows) ? fit : padded_groups(rows);
  const int64_t r = (rows + g - 1) / g;
  if (r > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_SHAPE, "%s: %lld rows per group", name,
                     static_cast<long long>(r));
  *rows_per_group = static_cast<int>(r);
  *groups = padded_groups((rows + r - 1) / r);
  return CREDIT_OK;
}

}  // namespace

size_t softmax_workspace(int op, int64_t rows, int64_t cols, int variant, int split,
                         int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  Plan p;
  const int64_t cap = op == CREDIT_OP_SOFTMAX_FWD ? kFwdCapacity : kBwdCapacity;
  const int st = op == CREDIT_OP_SOFTMAX_FWD   ? resolve_fwd(&c, cols, cols % 4 == 0, &p)
                 : op == CREDIT_OP_SOFTMAX_BWD ? resolve_bwd(&c, cols, cols % 4 == 0, &p)
                                               : resolve(&c, cols, cols % 4 == 0, cap, "softmax", &p);
  if (st != CREDIT_OK) return 0;
  const int k = op == CREDIT_OP_SOFTMAX_BWD ? 1 : 2;
  if ((op == CREDIT_OP_SOFTMAX_FWD && fwd_group_ok(p)) ||
      (op == CREDIT_OP_SOFTMAX_BWD && bwd_group_ok(p))) {
    int64_t groups = coresident_groups_bound(p.members, cu_count);
    if (groups > padded_groups(rows)) groups = padded_groups(rows);
    return split_workspace_bytes(groups, p.members, k, kGroupRing, 0);
  }
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
  CREDIT_TRY(resolve_fwd(cfg, cols, vec_ok(cols, {x, p}), &plan));
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
  if (fwd_group_ok(plan)) {
    const Pick<FwdGroupFn>* gk = pick_for(kFwdGroup, plan.chunk);
    const int threads = gk->threads + kWave;
    int rpg = 0;
    int64_t groups = 0;
    int dispensers = 0;
    CREDIT_TRY(plan_row_groups(reinterpret_cast<const void*>(gk->fn), threads, plan.members, rows,
                               &rpg, &groups, &dispensers, "softmax_fwd_group_kernel"));
    SplitWorkspace ws;
    CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, 2, kGroupRing, 0, &ws));
    const uint32_t total = static_cast<uint32_t>(groups * plan.members);
    hipLaunchKernelGGL(gk->fn, dim3(total), dim3(threads), 0, stream, x, p, rowmax, lse,
                       static_cast<int>(rows), c, static_cast<int>(plan.chunk), plan.members, rpg,
                       make_split_args(ws, total, static_cast<uint32_t>(rpg), kGroupRing,
                                       dispensers));
    return check_launch("softmax_fwd_group_kernel");
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
  CREDIT_TRY(resolve_bwd(cfg, cols, vec, &plan));
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
  if (bwd_group_ok(plan)) {
    const Pick<BwdGroupFn>* gk = pick_for(kBwdGroup, plan.chunk);
    const int threads = gk->threads + kWave;
    int rpg = 0;
    int64_t groups = 0;
    int dispensers = 0;
    CREDIT_TRY(plan_row_groups(reinterpret_cast<const void*>(gk->fn), threads, plan.members, rows,
                               &rpg, &groups, &dispensers, "softmax_bwd_group_kernel"));
    SplitWorkspace ws;
    CREDIT_TRY(acquire_split_workspace(cfg, groups, plan.members, 1, kGroupRing, 0, &ws));
    const uint32_t total = static_cast<uint32_t>(groups * plan.members);
    hipLaunchKernelGGL(gk->fn, dim3(total), dim3(threads), 0, stream, p, dy, dx,
                       static_cast<int>(rows), c, static_cast<int>(plan.chunk), plan.members, rpg,
                       make_split_args(ws, total, static_cast<uint32_t>(rpg), kGroupRing,
                                       dispensers));
    return check_launch("softmax_bwd_group_kernel");
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
