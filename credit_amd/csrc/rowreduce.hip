// C1: fused row sum + row max over fp32 rows.
//
// The reference has no standalone sum/max workload; its row max is the
// max-abs pass of src/workloads/rowwise_quant.cu:260-363 (block_read,
// block_smem and cluster_smem variants) and its row sums live inside the
// LayerNorm statistics (src/workloads/layernorm_backward.cu:286-292).  A pure
// reduction needs no staging, so the gfx950 variants are:
//  - READ  : one workgroup streams one row with dwordx4 loads, UNROLL loads
//            in flight per lane; sum in fp64, max with v_maximum3_f32.
//  - SPLIT : P workgroups per row each reduce a 1/P slice and deposit a
//            partial in the workspace; the last to arrive (device-scope
//            counter) folds the P partials in slice order and resets the
//            counter.  No workgroup ever waits on another, so the split
//            needs no co-residency guarantee and stays deterministic.
// Algorithmic traffic per row: 4*cols bytes read + 8 bytes written.
#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

constexpr int kRowThreads = 256;
constexpr int kRowUnroll = 8;

struct SumMax {
  double s;
  float m;
};

__device__ __forceinline__ void fold4(f32x4 v, double& s, float& m) {
  const double a = static_cast<double>(v.x) + static_cast<double>(v.y);
  const double b = static_cast<double>(v.z) + static_cast<double>(v.w);
  s += a + b;
  m = fmax_nan(m, fmax_nan(fmax_nan(v.x, v.y), fmax_nan(v.z, v.w)));
}

// Reduce x[c0, c1) of one row held by THREADS threads.  The aligned body is
// read as f32x4; up to three head and three tail elements go scalar.
template <int THREADS>
__device__ __forceinline__ SumMax reduce_range(const float* __restrict__ row,
                                               int c0, int c1) {
  double s = 0.0;
  float m = -__builtin_inff();
  const int tid = threadIdx.x;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(row + c0);
  int head = static_cast<int>(((16 - (addr & 15)) & 15) >> 2);
  if (head > c1 - c0) head = c1 - c0;
  if (tid < head) {
    const float v = row[c0 + tid];
    s += static_cast<double>(v);
    m = fmax_nan(m, v);
  }
  const int b0 = c0 + head;
  const int n4 = (c1 - b0) >> 2;
  const f32x4* p = reinterpret_cast<const f32x4*>(row + b0);
  int i = tid;
  for (; i + (kRowUnroll - 1) * THREADS < n4; i += kRowUnroll * THREADS) {
    f32x4 v[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) v[u] = load_nt(p + i + u * THREADS);
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) fold4(v[u], s, m);
  }
  for (; i < n4; i += THREADS) fold4(load_nt(p + i), s, m);
  const int t0 = b0 + (n4 << 2);
  if (t0 + tid < c1) {
    const float v = row[t0 + tid];
    s += static_cast<double>(v);
    m = fmax_nan(m, v);
  }
  return {s, m};
}

template <int THREADS>
__device__ __forceinline__ SumMax block_sum_max(SumMax v) {
  constexpr int NW = THREADS / kWave;
  __shared__ double s_slots[NW];
  __shared__ float m_slots[NW];
  const double s = block_reduce_sum_f64<NW>(v.s, s_slots);
  const float m = block_reduce<NW>(v.m, MaxOp{}, m_slots);
  return {s, m};
}

template <int THREADS>
__global__ __launch_bounds__(THREADS) void row_sum_max_read_kernel(
    const float* __restrict__ x, float* __restrict__ sum_out,
    float* __restrict__ max_out, int cols) {
  const int row = blockIdx.x;
  const float* xr = x + static_cast<size_t>(row) * cols;
  const SumMax r = block_sum_max<THREADS>(reduce_range<THREADS>(xr, 0, cols));
  if (threadIdx.x == 0) {
    sum_out[row] = static_cast<float>(r.s);
    max_out[row] = r.m;
  }
}

template <int THREADS>
__global__ __launch_bounds__(THREADS) void row_sum_max_split_kernel(
    const float* __restrict__ x, float* __restrict__ sum_out,
    float* __restrict__ max_out, int cols, int split, int chunk,
    double* __restrict__ part_sum, float* __restrict__ part_max,
    uint32_t* __restrict__ arrivals) {
  const int row = blockIdx.x / split;
  const int slice = blockIdx.x - row * split;
  const int c0 = slice * chunk;
  const int c1 = c0 + chunk < cols ? c0 + chunk : cols;
  const float* xr = x + static_cast<size_t>(row) * cols;
  SumMax local{0.0, -__builtin_inff()};
  if (c0 < c1) local = reduce_range<THREADS>(xr, c0, c1);
  const SumMax r = block_sum_max<THREADS>(local);
  __shared__ int is_last;
  if (threadIdx.x == 0) {
    const size_t slot = static_cast<size_t>(row) * split + slice;
    publish(part_sum + slot, r.s);
    publish(part_max + slot, r.m);
    publish_wait();
    is_last = arrive(arrivals + row) == static_cast<uint32_t>(split - 1);
  }
  __syncthreads();
  if (is_last && threadIdx.x == 0) {
    const size_t base = static_cast<size_t>(row) * split;
    double s = 0.0;
    float m = -__builtin_inff();
    for (int k = 0; k < split; ++k) {
      s += fetch(part_sum + base + k);
      m = fmax_nan(m, fetch(part_max + base + k));
    }
    sum_out[row] = static_cast<float>(s);
    max_out[row] = m;
    counter_reset(arrivals + row);
  }
}

struct SplitLayout {
  size_t part_sum_off, part_max_off, bytes;
};

// Arrival counters live in the workspace's counter area, one per row of a
// launch, after the ticket dispenser's slots; a launch covers at most
// kLaunchRows rows and the partials are sized for one launch.
constexpr int64_t kLaunchRows = kCounterSlots - kGroupCounterBase;

SplitLayout split_layout(int64_t rows, int split) {
  SplitLayout l;
  const int64_t launch_rows = rows < kLaunchRows ? rows : kLaunchRows;
  const size_t slots = static_cast<size_t>(launch_rows) * split;
  l.part_sum_off = 0;
  l.part_max_off = align_up(slots * sizeof(double), 256);
  l.bytes = l.part_max_off + align_up(slots * sizeof(float), 256);
  return l;
}

int choose_split(int64_t rows, int64_t cols, int cu_count) {
  // Enough workgroups to give every CU four, but never slices under 16 KiB.
  const int64_t want = (4 * static_cast<int64_t>(cu_count) + rows - 1) / rows;
  int64_t p = want < 1 ? 1 : want;
  const int64_t max_by_width = cols / 4096 > 0 ? cols / 4096 : 1;
  if (p > max_by_width) p = max_by_width;
  if (p > 16) p = 16;
  return static_cast<int>(p);
}

int resolve_variant(const credit_cfg* cfg, int64_t rows, int64_t cols,
                    int cu_count, int* split) {
  int variant = cfg_variant(cfg);
  int p = cfg_split(cfg);
  if (variant == CREDIT_VARIANT_AUTO) {
    p = choose_split(rows, cols, cu_count);
    variant = p > 1 ? CREDIT_VARIANT_SPLIT : CREDIT_VARIANT_READ;
  } else if (variant == CREDIT_VARIANT_STAGED) {
    // A pure reduction reads every element once; staging adds nothing.
    variant = CREDIT_VARIANT_READ;
  }
  if (variant == CREDIT_VARIANT_SPLIT) {
    if (p == 0) p = choose_split(rows, cols, cu_count);
    if (p < 1) p = 1;
  }
  *split = p;
  return variant;
}

}  // namespace

size_t row_sum_max_workspace(int64_t rows, int64_t cols, int variant,
                             int split, int cu_count) {
  credit_cfg c{nullptr, variant, split, nullptr, 0};
  int p = 1;
  const int v = resolve_variant(&c, rows, cols, cu_count, &p);
  if (v != CREDIT_VARIANT_SPLIT || p <= 1) return 0;
  return split_layout(rows, p).bytes;
}

}  // namespace credit

using namespace credit;

extern "C" int credit_row_sum_max_f32(const float* x, float* sum, float* max,
                                      int64_t rows, int64_t cols,
                                      const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_row_ptr(sum, "sum", rows));
  CREDIT_TRY(check_row_ptr(max, "max", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_aligned(x, 4, "x"));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  int split = 1;
  const int variant = resolve_variant(cfg, rows, cols, props->cu_count, &split);
  hipStream_t stream = cfg_stream(cfg);
  const int c = static_cast<int>(cols);
  if (variant == CREDIT_VARIANT_READ || split == 1) {
    row_sum_max_read_kernel<kRowThreads>
        <<<dim3(static_cast<unsigned>(rows)), dim3(kRowThreads), 0, stream>>>(
            x, sum, max, c);
    return check_launch("row_sum_max_read_kernel");
  }
  if (split > cols) split = static_cast<int>(cols);
  // Slices are whole f32x4s so every slice but the first starts aligned
  // whenever the row does.
  int chunk = static_cast<int>((cols + split - 1) / split);
  chunk = (chunk + 3) & ~3;
  split = static_cast<int>((cols + chunk - 1) / chunk);
  const SplitLayout l = split_layout(rows, split);
  // The grid is not co-resident (no member waits), but its shape is what
  // credit_last_split_shape reports for this call: plan it the same way.
  int64_t resident_groups = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(row_sum_max_split_kernel<kRowThreads>),
                               kRowThreads, 0, split, &resident_groups));
  char* ws = nullptr;
  CREDIT_TRY(acquire_workspace(cfg, l.bytes, &ws));
  char* scratch = ws_scratch(ws);
  for (int64_t r0 = 0; r0 < rows; r0 += kLaunchRows) {
    const int64_t n = rows - r0 < kLaunchRows ? rows - r0 : kLaunchRows;
    row_sum_max_split_kernel<kRowThreads>
        <<<dim3(static_cast<unsigned>(n * split)), dim3(kRowThreads), 0, stream>>>(
            x + r0 * cols, sum + r0, max + r0, c, split, chunk,
            reinterpret_cast<double*>(scratch + l.part_sum_off),
            reinterpret_cast<float*>(scratch + l.part_max_off),
            ws_counters(ws) + kGroupCounterBase);
    CREDIT_TRY(check_launch("row_sum_max_split_kernel"));
  }
  return CREDIT_OK;
}
