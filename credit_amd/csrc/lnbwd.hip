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
#include <type_traits>
#include <utility>

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

// ------------------------------------------------ bf16 group pipeline ---
// SPLIT for bf16 rows: the barrier-free row pipeline of the RMSNorm backward
// group kernel (credit_amd/csrc/rmsnorm.hip, rmsnorm_group_body) with the
// LayerNorm statistics in the same single exchange.  Each member publishes
// four partials of a row, about the row's first element x0:
//   S1 = sum(x - x0), S2 = sum((x - x0)^2), S3 = sum(g), S4 = sum(g (x - x0))
// with g = dy * gamma.  From the group totals d = S1/N (= mean - x0),
// var = S2/N - d^2, rstd, mean(g) = S3/N and
// mean(g xhat) = rstd (S4 - d S3) / N, so one exchange per row carries what
// the slice kernel exchanges in two stages.  The communication wave turns
// the totals into (d, rstd, mean(g), mean(g xhat)); a data wave then writes
// dx = (g - mean(g) - xhat mean(g xhat)) rstd with xhat = ((x - x0) - d) rstd.
// The shifted product sum S4 - d S3 cancels where |mean - x0| |S3| is far
// above |sum(g xhat)| / rstd; fp32 lane sums over 16 elements, fp64 beyond,
// leave that well inside bf16 output precision (the fp32 variant keeps the
// two-stage slice kernel).  THREADS data lanes hold VPT vectors of x and dy
// per row in DEPTH + AHEAD + 1 rotating buffers, gamma's slice in registers,
// one extra communication wave polls; rows are published DEPTH steps before
// their totals are needed and loaded AHEAD steps before that.
constexpr int kLnGroupRing = 16;  // device slot rows per group (> 2 DEPTH + 1)
constexpr int kLnValues = 4;      // partials per member and row

template <int THREADS, int VPT, int DEPTH, int AHEAD>
__device__ __forceinline__ void layernorm_bwd_group_body(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ dx, int rows, int cols, int chunk,
    int members, int rows_per_group, float eps, SplitArgs sa) {
  constexpr int NW = THREADS / kWave;
  constexpr int K = kLnValues;
  constexpr int NB = DEPTH + AHEAD + 1;
  constexpr int RING = DEPTH + 2 <= 4 ? 4 : 8;
  static_assert(DEPTH >= 1 && AHEAD >= 1 && DEPTH + 2 <= 8, "pipeline depth");
  static_assert(2 * DEPTH + 1 < kLnGroupRing, "device slot ring too short for DEPTH");
  __shared__ double red[RING][K][NW];  // wave partials of row k at [k % RING]
  __shared__ float ring[RING][4];      // (d, rstd, mean g, mean g xhat) of row k
  __shared__ uint32_t arrivals[RING];
  __shared__ uint32_t ready;           // rows 0 .. ready - 1 have totals
  const int tid = threadIdx.x;
  if (tid < RING) arrivals[tid] = 0;
  if (tid == 0) ready = 0;
  const SplitGroup g = split_join(sa, members, K);  // its barrier covers the stores above
  // Rows dealt round-robin to the G groups that take rows (padding groups
  // of the dispenser-multiple grid exit); i counts the group's rows.
  const int G = (rows + rows_per_group - 1) / rows_per_group;
  if (g.group >= G) return;
  const int r1 = (rows - g.group + G - 1) / G;
  auto row_of = [&](int i) { return g.group + i * G; };
  const int nvec = cols >> 3;
  const int v0 = g.member * chunk;
  const int vlen = nvec - v0 < chunk ? nvec - v0 : chunk;
  const uint32_t slice_bytes = static_cast<uint32_t>(vlen) * 16u;
  const double inv_n = 1.0 / cols;

  if (__builtin_amdgcn_readfirstlane(tid) >= THREADS) {
    // ---- communication wave: every row's totals, in row order ----
    for (int k = 0; k < r1; ++k) {
      const uint32_t bits = split_poll(g, k, K);
      const double s1 = split_wave_sum(bits, members, 0);
      const double s2 = split_wave_sum(bits, members, 1);
      const double s3 = split_wave_sum(bits, members, 2);
      const double s4 = split_wave_sum(bits, members, 3);
      if (tid == THREADS) {
        const double d = s1 * inv_n;
        const double var = s2 * inv_n - d * d;
        const double rs = 1.0 / __builtin_sqrt((var > 0.0 ? var : 0.0) + eps);
        float* e = ring[k % RING];
        e[0] = static_cast<float>(d);
        e[1] = static_cast<float>(rs);
        e[2] = static_cast<float>(s3 * inv_n);
        e[3] = static_cast<float>(rs * (s4 - d * s3) * inv_n);
        __hip_atomic_store(&ready, static_cast<uint32_t>(k + 1), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    return;
  }

  // ---- data waves ----
  const int wid = tid / kWave;
  const bool lead = (tid & (kWave - 1)) == 0;
  const uint32_t lane_off = static_cast<uint32_t>(tid) * 16u;
  constexpr uint32_t kStride = THREADS * 16u;
  struct Row {
    u32x4 x[VPT], d[VPT];
    uint32_t x0;  // the row's first two bf16 (x0 in the low half), every lane
  };
  Row b[NB];
  // Row r's slice and its first element, or zeros (no traffic) beyond the
  // group: every load goes through a buffer resource, none under a branch.
  auto load_row = [&](Row& b, int r) {
    const bool live = r < r1;
    const size_t row_off = static_cast<size_t>(row_of(live ? r : 0)) * cols;
    const size_t off = row_off + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t xs = make_rsrc(x + off, live ? slice_bytes : 0u);
    const buffer_rsrc_t ds = make_rsrc(dy + off, live ? slice_bytes : 0u);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      b.x[k] = buffer_load_nt(xs, lane_off + k * kStride);
      b.d[k] = buffer_load_nt(ds, lane_off + k * kStride);
    }
    b.x0 = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(x + row_off, live ? 4u : 0u), 0, 0, 0);
  };
  const buffer_rsrc_t grs = make_rsrc(gamma + 8 * static_cast<size_t>(v0), slice_bytes);
  u32x4 gk[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) gk[q] = buffer_load(grs, lane_off + q * kStride);
  // Row k's four lane sums -> wave partials; the last wave in publishes the
  // member's four partials (wave order, fp64).
  auto publish_row = [&](const Row& b, int k) {
    const float x0 = bf16_lo(b.x0);
    float a[K] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      float p1 = 0.0f, p2 = 0.0f, p3 = 0.0f, p4 = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xc = Vec<uint16_t>::get(b.x[q], e) - x0;
        const float gg = Vec<uint16_t>::get(b.d[q], e) * Vec<uint16_t>::get(gk[q], e);
        p1 += xc;
        p2 += xc * xc;
        p3 += gg;
        p4 += gg * xc;
      }
      // Beyond the slice x reads 0: its shifted value -x0 must add nothing
      // (g is 0 there, since dy reads 0).
      const bool in = lane_off + q * kStride < slice_bytes;
      a[0] += in ? p1 : 0.0f;
      a[1] += in ? p2 : 0.0f;
      a[2] += p3;
      a[3] += p4;
    }
    double v[K];
#pragma unroll
    for (int e = 0; e < K; ++e) v[e] = wave_reduce_sum_f64(static_cast<double>(a[e]));
    const int slot = k % RING;
    if (lead) {
#pragma unroll
      for (int e = 0; e < K; ++e) red[slot][e][wid] = v[e];
      const uint32_t t = __hip_atomic_fetch_add(&arrivals[slot], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
      if (t == NW - 1) {
#pragma unroll
        for (int e = 0; e < K; ++e) {
          double s = red[slot][e][0];
#pragma unroll
          for (int q = 1; q < NW; ++q) s += red[slot][e][q];
          split_publish_at(g, k, e, s);
        }
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
    // The packed row stays in registers across the DEPTH steps; unpacked
    // copies would double it (opaque: recompute from the packed values).
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      __asm__ volatile("" : "+v"(b.x[q]));
      __asm__ volatile("" : "+v"(b.d[q]));
    }
    const float x0 = bf16_lo(b.x0);
    const float d = ring[slot][0], rs = ring[slot][1], mg = ring[slot][2], mgx = ring[slot][3];
    const size_t off = static_cast<size_t>(row_of(r)) * cols + 8 * static_cast<size_t>(v0);
    const buffer_rsrc_t out = make_rsrc(dx + off, slice_bytes);
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = ((Vec<uint16_t>::get(b.x[q], e) - x0) - d) * rs;
        const float gg = Vec<uint16_t>::get(b.d[q], e) * Vec<uint16_t>::get(gk[q], e);
        o[e] = (gg - mg - xh * mgx) * rs;
      }
      buffer_store_nt(out, lane_off + q * kStride, Vec<uint16_t>::pack(o));
    }
  };
  auto step = [&]<int S>(std::integral_constant<int, S>, int i) {
    load_row(b[(S + DEPTH + AHEAD) % NB], i + DEPTH + AHEAD);
    __builtin_amdgcn_sched_barrier(0);
    if (i + DEPTH < r1) publish_row(b[(S + DEPTH) % NB], i + DEPTH);
    finish_row(b[S], i, wait_total(i));
  };
  [&]<int... J>(std::integer_sequence<int, J...>) {
    (load_row(b[J], J), ...);
  }(std::make_integer_sequence<int, DEPTH + AHEAD>{});
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ((J < r1 ? publish_row(b[J], J) : void()), ...);
  }(std::make_integer_sequence<int, DEPTH>{});
  int i = 0;
  for (; i + NB - 1 < r1; i += NB)
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (step(std::integral_constant<int, S>{}, i + S), ...);
    }(std::make_integer_sequence<int, NB>{});
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((i + S < r1 ? step(std::integral_constant<int, S>{}, i + S) : void()), ...);
  }(std::make_integer_sequence<int, NB - 1>{});
}

template <int THREADS, int VPT, int DEPTH, int AHEAD>
__global__ __launch_bounds__(THREADS + kWave)
__attribute__((amdgpu_waves_per_eu(3, 8))) void layernorm_bwd_group_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ dx, int rows, int cols, int chunk,
    int members, int rows_per_group, float eps, SplitArgs sa) {
  layernorm_bwd_group_body<THREADS, VPT, DEPTH, AHEAD>(x, dy, gamma, dx, rows, cols, chunk,
                                                       members, rows_per_group, eps, sa);
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

// The bf16 group pipeline: members of at most kLnGroupCapacity vectors, at
// most kMaxExchangeValues / 4 of them (four partials each per row).
using LnGroupFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int,
                           int, int, int, float, SplitArgs);
struct LnGroupPick {
  LnGroupFn fn;
  int threads;   // data lanes (plus one communication wave)
  int capacity;  // vectors per member
};
// One shape: 512 lanes x 2 vectors, one workgroup per CU.  A 256-lane form
// (three workgroups per CU, 16 members of 512 vectors at 2048 x 65536) ran
// at 2.7 TB/s against 5.0 for this one at 8 members; narrower slices leave
// lanes of this shape idle instead.
// DEPTH 4 / AHEAD 2: seven row buffers (168 VGPRs, no spill).  At
// 2048 x 65536, two GPU sessions of three alternating runs: 160.0 us at 3 / 2,
// 157.6 at 4 / 1, 157.7 at 2 / 2, 153.9 at 3 / 1 and 3 / 3, 152.1 at 2 / 1,
// 151.8 at 4 / 2 (5 / 1 spills).
const LnGroupPick kLnGroup[] = {
    {layernorm_bwd_group_kernel<512, 2, 4, 2>, 512, 1024},
};
constexpr int64_t kLnGroupCapacity = 1024;
constexpr int kLnGroupMaxMembers = kMaxExchangeValues / kLnValues;

// Members of the bf16 group pipeline for this call, or 0 when it does not
// apply: AUTO on rows wider than the STAGED capacity (the fewest power-of-two
// members whose slices fit), SPLIT with a split factor whose slices fit.
int ln_group_members(const credit_cfg* cfg, int64_t nvec, bool vec) {
  if (!vec) return 0;
  const int variant = cfg_variant(cfg);
  int p = 0;
  if (variant == CREDIT_VARIANT_AUTO && nvec > Slices<uint16_t>::capacity) {
    p = 2;
    while (p * kLnGroupCapacity < nvec) p *= 2;
  } else if (variant == CREDIT_VARIANT_SPLIT && cfg_split(cfg) > 1) {
    p = cfg_split(cfg);
  }
  if (p < 2 || p > kLnGroupMaxMembers || p > nvec) return 0;
  const int64_t chunk = (nvec + p - 1) / p;
  if (chunk > kLnGroupCapacity || (nvec + chunk - 1) / chunk != p) return 0;
  return p;
}

int layernorm_bwd_group(const uint16_t* x, const uint16_t* dy, const uint16_t* gamma,
                        uint16_t* dx, int64_t rows, int64_t cols, float eps, int members,
                        const credit_cfg* cfg) {
  const int64_t nvec = cols / 8;
  const int64_t chunk = (nvec + members - 1) / members;
  const LnGroupPick* pk = &kLnGroup[0];
  int64_t fit = 0;
  int dispensers = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(pk->fn), pk->threads + kWave, 0,
                               members, &fit, &dispensers));
  if (fit == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "layernorm_bwd: %d groups of %d members do not fit the device", kDispensers,
                     members);
  const int64_t g = fit < padded_groups(rows) ? fit : padded_groups(rows);
  const int64_t rpg = (rows + g - 1) / g;
  if (rpg > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_SHAPE, "layernorm_bwd: %lld rows per group",
                     static_cast<long long>(rpg));
  const int64_t groups = padded_groups((rows + rpg - 1) / rpg);
  SplitWorkspace ws;
  CREDIT_TRY(acquire_split_workspace(cfg, groups, members, kLnValues, kLnGroupRing, 0, &ws));
  const uint32_t total = static_cast<uint32_t>(groups * members);
  hipLaunchKernelGGL(pk->fn, dim3(total), dim3(pk->threads + kWave), 0, cfg_stream(cfg), x, dy,
                     gamma, dx, static_cast<int>(rows), static_cast<int>(cols),
                     static_cast<int>(chunk), members, static_cast<int>(rpg), eps,
                     make_split_args(ws, total, static_cast<uint32_t>(rpg), kLnGroupRing,
                                     dispensers));
  return check_launch("layernorm_bwd_group_kernel");
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
  if constexpr (std::is_same_v<T, uint16_t>) {
    if (const int p = ln_group_members(cfg, cols / E, vec))
      return layernorm_bwd_group(x, dy, gamma, dx, rows, cols, eps, p, cfg);
  }
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
  if (elem_bytes == 2) {
    if (const int m = ln_group_members(&c, cols / e, cols % e == 0)) {
      int64_t groups = coresident_groups_bound(m, cu_count);
      if (groups > padded_groups(rows)) groups = padded_groups(rows);
      return split_workspace_bytes(groups, m, kLnValues, kLnGroupRing, 0);
    }
  }
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
