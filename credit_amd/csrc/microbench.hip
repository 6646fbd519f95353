// gfx950 calibration microbenchmarks.
//
// Replaces the reference's src/primitive_benchmark.cu (pointer-chase
// latencies :58-115, L1/L2/DRAM bandwidth :118-171, DSMEM sync/latency/
// throughput/visibility :236-566) and src/cluster_control.cu (cluster launch +
// k barriers minus a plain launch, :69-89,114-180).  CDNA4 has no DSMEM, so
// the cluster measurements become the costs of the split-row exchange this
// library uses instead: device-scope atomic round trips between two
// workgroups on the same / on different XCDs, and the cost of a P-member
// arrival barrier inside a cooperative persistent grid.
//
// Every kernel here is bounded: spin loops carry an iteration limit and
// report a timeout instead of hanging.
#include <string.h>

#include <vector>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

// --------------------------------------------------------- HBM streams ---
template <int UNROLL>
__global__ __launch_bounds__(256) void mb_read_kernel(const f32x4* __restrict__ src,
                                                      int64_t n4, float* __restrict__ sink) {
  float acc = 0.0f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  for (; i + (UNROLL - 1) * stride < n4; i += UNROLL * stride) {
    f32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = load_nt(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  for (; i < n4; i += stride) {
    const f32x4 v = load_nt(src + i);
    acc += (v.x + v.y) + (v.z + v.w);
  }
  if (acc == 1.2345e-30f) sink[0] = acc;  // keeps the loads alive
}

__global__ __launch_bounds__(256) void mb_write_kernel(f32x4* __restrict__ dst, int64_t n4) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const f32x4 v = {1.0f, 2.0f, 3.0f, 4.0f};
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += stride)
    store_nt(dst + i, v);
}

template <int UNROLL, bool NT_STORE>
__global__ __launch_bounds__(256) void mb_copy_kernel(const f32x4* __restrict__ src,
                                                      f32x4* __restrict__ dst, int64_t n4) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  for (; i + (UNROLL - 1) * stride < n4; i += UNROLL * stride) {
    f32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = load_nt(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (NT_STORE)
        store_nt(dst + i + u * stride, v[u]);
      else
        dst[i + u * stride] = v[u];
    }
  }
  for (; i < n4; i += stride) {
    if (NT_STORE)
      store_nt(dst + i, load_nt(src + i));
    else
      dst[i] = load_nt(src + i);
  }
}

// One contiguous chunk per workgroup (the access shape of the row kernels:
// a workgroup owns a row, reads it whole, then writes it whole).
template <int VPT>
__global__ __launch_bounds__(256) void mb_copy_rows_kernel(const f32x4* __restrict__ src,
                                                           f32x4* __restrict__ dst) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * VPT;
  f32x4 v[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) v[k] = load_nt(src + base + k * 256 + threadIdx.x);
#pragma unroll
  for (int k = 0; k < VPT; ++k) store_nt(dst + base + k * 256 + threadIdx.x, v[k]);
}

// ------------------------------------------------------------- latency ---
// Single-lane pointer chase; the chain is laid out with a fixed stride so a
// working set of `bytes` is walked.  Cycles come from s_memtime.
__global__ void mb_chase_kernel(const uint32_t* __restrict__ chain, int iters,
                                uint64_t* __restrict__ out) {
  uint32_t p = 0;
  // warm pass over the chain
  for (int i = 0; i < iters; ++i) p = __hip_atomic_load(chain + p, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_WORKGROUP);
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int i = 0; i < iters; ++i) p = __hip_atomic_load(chain + p, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_WORKGROUP);
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  out[0] = t1 - t0;
  out[1] = p;
}

__global__ void mb_chase_init(uint32_t* chain, int64_t n, int64_t stride) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) chain[i] = static_cast<uint32_t>((i + stride) % n);
}

// Shader clock against the 100 MHz constant clock.
__global__ void mb_clock_kernel(uint64_t* out) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  uint64_t r1 = r0;
  while (r1 - r0 < 1000000) r1 = __builtin_amdgcn_s_memrealtime();  // 10 ms
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  out[0] = c1 - c0;
  out[1] = r1 - r0;
}

// ------------------------------------------------------ LDS bandwidth ---
template <bool WRITE>
__global__ __launch_bounds__(256) void mb_lds_kernel(int iters, float* sink, uint64_t* cycles) {
  __shared__ f32x4 tile[4096];  // 64 KiB
  const int t = threadIdx.x;
  for (int k = t; k < 4096; k += 256) tile[k] = f32x4{1.0f, 2.0f, 3.0f, static_cast<float>(k)};
  __syncthreads();
  f32x4 acc = {0, 0, 0, 0};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int idx = (k * 256 + t + i) & 4095;
      if (WRITE)
        tile[idx] = acc;
      else
        acc += tile[idx];
    }
    if (WRITE) acc.x += 1.0f;
  }
  __syncthreads();
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  if (t == 0) cycles[blockIdx.x] = t1 - t0;
  if (acc.x == 1.2345e-30f) sink[0] = acc.y + tile[t].z;
}

// ------------------------------------------- exchange round trip (H3) ----
// Workgroups 0 and `peer` bounce a token `rounds` times through device-scope
// atomics; workgroup 0 times the loop with s_memtime.  All other
// workgroups exit at once.  With blockIdx -> XCD assigned round-robin,
// peer = 8 shares workgroup 0's XCD and peer = 1 does not.
__global__ void mb_pingpong_kernel(uint32_t* flag, int peer, int rounds, uint64_t* out,
                                   uint32_t* timeout) {
  const int me = blockIdx.x == 0 ? 0 : (static_cast<int>(blockIdx.x) == peer ? 1 : -1);
  if (me < 0 || threadIdx.x != 0) return;
  uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int r = 0; r < rounds; ++r) {
    const uint32_t want = 2u * r + me;
    uint32_t spins = 0;
    while (counter_read(flag) != want) {
      if (++spins > (1u << 24)) {
        __hip_atomic_store(timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
    __hip_atomic_store(flag, want + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (me == 0) out[0] = __builtin_amdgcn_s_memtime() - t0;
}

// ------------------------------------------ arrival barrier cost (H3/H4) --
// A co-resident grid of ticketed groups of `members` workgroups, shaped
// like the split kernels' launches: each group takes rows group, group + G,
// ... of `rows` and meets `barriers` times per row (publish, poll, read the
// partials): the un-overlapped cost of the exchange the split kernels use.
__global__ __launch_bounds__(256) void mb_barrier_kernel(SplitArgs sa, int members,
                                                         int barriers, int rows,
                                                         double* sink) {
  SplitGroup g = split_join(sa, members, 1);
  const int step = static_cast<int>(sa.grid) / members;
  double acc = 0.0;
  for (int row = g.group; row < rows; row += step) {
    for (int k = 0; k < barriers; ++k) {
      if (threadIdx.x == 0) split_publish(g, 0, static_cast<double>(g.member + k));
      split_exchange(g);
      acc += split_sum(g, 0);
    }
  }
  if (acc == -1.0 && threadIdx.x == 0) sink[0] = acc;  // keeps the reads alive
}

__global__ __launch_bounds__(256) void mb_plain_kernel(int* sink) {
  if (threadIdx.x == 0 && blockIdx.x == 0x7fffffff) sink[0] = 1;
}

struct Events {
  hipEvent_t a = nullptr, b = nullptr;
  ~Events() {
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
  }
};

template <class F>
int time_ms(F&& launch, int warmup, int iters, double* ms) {
  Events ev;
  CREDIT_HIP(hipEventCreate(&ev.a));
  CREDIT_HIP(hipEventCreate(&ev.b));
  for (int i = 0; i < warmup; ++i) CREDIT_TRY(launch(i));
  CREDIT_HIP(hipEventRecord(ev.a, nullptr));
  for (int i = 0; i < iters; ++i) CREDIT_TRY(launch(i));
  CREDIT_HIP(hipEventRecord(ev.b, nullptr));
  CREDIT_HIP(hipEventSynchronize(ev.b));
  float t = 0.0f;
  CREDIT_HIP(hipEventElapsedTime(&t, ev.a, ev.b));
  *ms = static_cast<double>(t) / iters;
  return CREDIT_OK;
}

struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  int alloc(size_t bytes) {
    CREDIT_HIP(hipMalloc(&p, bytes));
    CREDIT_HIP(hipMemset(p, 0, bytes));
    return CREDIT_OK;
  }
};

int bench_stream(int which, int64_t bytes, int iters, double* results, int n) {
  if (bytes < (int64_t{1} << 20)) bytes = int64_t{1} << 30;
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  // Three source/destination pairs rotate so the 256 MB MALL cannot serve a
  // repeated working set.
  DevBuf src[3], dst[3], sink;
  for (int k = 0; k < 3; ++k) {
    CREDIT_TRY(src[k].alloc(bytes));
    if (which != CREDIT_MB_HBM_READ) CREDIT_TRY(dst[k].alloc(bytes));
  }
  CREDIT_TRY(sink.alloc(256));
  const int64_t n4 = bytes / 16;
  const int grids[] = {props->cu_count * 4, props->cu_count * 8, props->cu_count * 16,
                       props->cu_count * 32};
  double best = 0.0;
  int slot = 0;
  for (int gi = 0; gi < 4; ++gi) {
    const int grid = grids[gi];
    for (int variant = 0; variant < 3; ++variant) {
      double ms = 0.0;
      auto launch = [&](int i) -> int {
        const f32x4* s = static_cast<const f32x4*>(src[i % 3].p);
        f32x4* d = static_cast<f32x4*>(dst[i % 3].p);
        if (which == CREDIT_MB_HBM_READ) {
          if (variant == 0) mb_read_kernel<4><<<grid, 256>>>(s, n4, static_cast<float*>(sink.p));
          else if (variant == 1) mb_read_kernel<8><<<grid, 256>>>(s, n4, static_cast<float*>(sink.p));
          else mb_read_kernel<16><<<grid, 256>>>(s, n4, static_cast<float*>(sink.p));
        } else if (which == CREDIT_MB_HBM_WRITE) {
          mb_write_kernel<<<grid, 256>>>(d, n4);
        } else {
          if (variant == 0) mb_copy_kernel<4, true><<<grid, 256>>>(s, d, n4);
          else if (variant == 1) mb_copy_kernel<8, true><<<grid, 256>>>(s, d, n4);
          else mb_copy_kernel<8, false><<<grid, 256>>>(s, d, n4);
        }
        return check_launch("microbench stream");
      };
      CREDIT_TRY(time_ms(launch, 3, iters, &ms));
      const double moved = (which == CREDIT_MB_HBM_COPY ? 2.0 : 1.0) * static_cast<double>(bytes);
      const double gbps = moved / (ms * 1e-3) / 1e9;
      if (slot + 1 < n) results[1 + slot] = gbps;
      ++slot;
      if (gbps > best) best = gbps;
      if (which == CREDIT_MB_HBM_WRITE) break;
    }
  }
  // Row-shaped copy: workgroups own contiguous 16*VPT KiB chunks.
  if (which == CREDIT_MB_HBM_COPY) {
    const int vpts[] = {4, 8, 16};
    for (int vi = 0; vi < 3; ++vi) {
      const int vpt = vpts[vi];
      const int64_t grid = n4 / (256 * vpt);
      double ms = 0.0;
      auto launch = [&](int i) -> int {
        const f32x4* s = static_cast<const f32x4*>(src[i % 3].p);
        f32x4* d = static_cast<f32x4*>(dst[i % 3].p);
        if (vpt == 4) mb_copy_rows_kernel<4><<<static_cast<unsigned>(grid), 256>>>(s, d);
        else if (vpt == 8) mb_copy_rows_kernel<8><<<static_cast<unsigned>(grid), 256>>>(s, d);
        else mb_copy_rows_kernel<16><<<static_cast<unsigned>(grid), 256>>>(s, d);
        return check_launch("microbench copy rows");
      };
      CREDIT_TRY(time_ms(launch, 3, iters, &ms));
      const double gbps = 2.0 * static_cast<double>(grid * 256 * vpt * 16) / (ms * 1e-3) / 1e9;
      if (slot + 1 < n) results[1 + slot] = gbps;
      ++slot;
      if (gbps > best) best = gbps;
    }
  }
  results[0] = best;
  return CREDIT_OK;
}

int bench_clock(double* results, int n) {
  DevBuf out;
  CREDIT_TRY(out.alloc(64));
  mb_clock_kernel<<<1, 64>>>(static_cast<uint64_t*>(out.p));
  CREDIT_TRY(check_launch("mb_clock_kernel"));
  uint64_t h[2];
  CREDIT_HIP(hipMemcpy(h, out.p, sizeof(h), hipMemcpyDeviceToHost));
  // s_memrealtime runs at 100 MHz.
  results[0] = static_cast<double>(h[0]) / (static_cast<double>(h[1]) / 100.0);  // MHz
  (void)n;
  return CREDIT_OK;
}

int bench_chase(int iters, double* results, int n) {
  // Working sets: 16 KiB (L1), 2 MiB (L2), 64 MiB (MALL), 1 GiB (HBM).
  const int64_t sets[] = {int64_t{16} << 10, int64_t{2} << 20, int64_t{64} << 20, int64_t{1} << 30};
  if (iters <= 0) iters = 20000;
  DevBuf chain, out;
  CREDIT_TRY(chain.alloc(sets[3]));
  CREDIT_TRY(out.alloc(64));
  for (int k = 0; k < 4 && k < n; ++k) {
    const int64_t elems = sets[k] / 4;
    // 4 KiB + 64 B stride: every step a new cache line, spread over
    // channels, and the chain covers the whole working set.
    int64_t stride = (4096 + 64) / 4;
    if (stride >= elems) stride = 16 + 1;
    mb_chase_init<<<static_cast<unsigned>((elems + 255) / 256), 256>>>(
        static_cast<uint32_t*>(chain.p), elems, stride);
    CREDIT_TRY(check_launch("mb_chase_init"));
    mb_chase_kernel<<<1, 1>>>(static_cast<const uint32_t*>(chain.p), iters,
                              static_cast<uint64_t*>(out.p));
    CREDIT_TRY(check_launch("mb_chase_kernel"));
    uint64_t h[2];
    CREDIT_HIP(hipMemcpy(h, out.p, sizeof(h), hipMemcpyDeviceToHost));
    results[k] = static_cast<double>(h[0]) / iters;  // shader cycles per load
  }
  return CREDIT_OK;
}

int bench_lds(bool write, int iters, double* results, int n) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (iters <= 0) iters = 4096;
  DevBuf cyc, sink;
  CREDIT_TRY(cyc.alloc(sizeof(uint64_t) * props->cu_count));
  CREDIT_TRY(sink.alloc(256));
  // One workgroup per CU.
  if (write)
    mb_lds_kernel<true><<<props->cu_count, 256>>>(iters, static_cast<float*>(sink.p),
                                                 static_cast<uint64_t*>(cyc.p));
  else
    mb_lds_kernel<false><<<props->cu_count, 256>>>(iters, static_cast<float*>(sink.p),
                                                  static_cast<uint64_t*>(cyc.p));
  CREDIT_TRY(check_launch("mb_lds_kernel"));
  std::vector<uint64_t> h(props->cu_count);
  CREDIT_HIP(hipMemcpy(h.data(), cyc.p, sizeof(uint64_t) * h.size(), hipMemcpyDeviceToHost));
  uint64_t worst = 1;
  for (uint64_t v : h) worst = v > worst ? v : worst;
  // bytes moved per workgroup / cycles of the slowest
  results[0] = 256.0 * 16 * 16 * iters / static_cast<double>(worst);
  (void)n;
  return CREDIT_OK;
}

int bench_pingpong(int rounds, double* results, int n) {
  if (rounds <= 0) rounds = 2000;
  DevBuf flag, out, tmo;
  CREDIT_TRY(flag.alloc(256));
  CREDIT_TRY(out.alloc(64));
  CREDIT_TRY(tmo.alloc(64));
  const int peers[] = {8, 1};  // same XCD, neighbouring XCD
  for (int k = 0; k < 2 && k < n; ++k) {
    CREDIT_HIP(hipMemset(flag.p, 0, 256));
    mb_pingpong_kernel<<<16, 64>>>(static_cast<uint32_t*>(flag.p), peers[k], rounds,
                                   static_cast<uint64_t*>(out.p), static_cast<uint32_t*>(tmo.p));
    CREDIT_TRY(check_launch("mb_pingpong_kernel"));
    uint64_t h = 0;
    uint32_t t = 0;
    CREDIT_HIP(hipMemcpy(&h, out.p, sizeof(h), hipMemcpyDeviceToHost));
    CREDIT_HIP(hipMemcpy(&t, tmo.p, sizeof(t), hipMemcpyDeviceToHost));
    if (t != 0) return set_error(CREDIT_ERR_WATCHDOG, "ping-pong partner never answered");
    results[k] = static_cast<double>(h) / rounds;  // shader cycles per round trip
  }
  return CREDIT_OK;
}

}  // namespace

int control_overhead(int64_t rows, int split, int barriers, int warmup, int iters,
                     double* plain_ms, double* split_ms, int cooperative) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (split < 1 || split > 64) return set_error(CREDIT_ERR_BAD_CONFIG, "split %d", split);
  if (rows < 1) return set_error(CREDIT_ERR_BAD_CONFIG, "rows must be >= 1");
  int64_t groups = 0;
  CREDIT_TRY(coresident_groups(reinterpret_cast<const void*>(mb_barrier_kernel), 256, 0, split,
                               &groups));
  if (groups < 1) return set_error(CREDIT_ERR_UNSUPPORTED, "split %d does not fit", split);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  const int64_t per_group = (rows + groups - 1) / groups;
  DevBuf ws, sink;
  CREDIT_TRY(ws.alloc(kScratchOffset + split_slot_bytes(groups, split, 1, kSplitRing)));
  CREDIT_TRY(sink.alloc(256));
  char* base = static_cast<char*>(ws.p);
  uint32_t* counters = ws_counters(base);
  uint32_t* watchdog = ws_watchdog(base);
  uint64_t* slots = reinterpret_cast<uint64_t*>(ws_scratch(base));
  double* sinkp = static_cast<double*>(sink.p);
  const unsigned grid = static_cast<unsigned>(groups * split);
  // The plain reference launches one workgroup per (row, member): the work
  // items a split launch covers, with no exchange.
  const unsigned plain_grid = static_cast<unsigned>(rows * split);
  const uint32_t total = grid;
  int valid = static_cast<int>(rows);
  const uint32_t stages = static_cast<uint32_t>(per_group * (barriers > 0 ? barriers : 1));
  auto plain = [&](int) -> int {
    mb_plain_kernel<<<plain_grid, 256>>>(static_cast<int*>(sink.p));
    return check_launch("mb_plain_kernel");
  };
  int members = split;
  auto timed = [&](int) -> int {
    SplitArgs sa{counters, slots, watchdog, total, next_split_epoch(stages), kSplitRing};
    if (cooperative) {
      void* args[] = {&sa, &members, &barriers, &valid, &sinkp};
      CREDIT_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(mb_barrier_kernel),
                                            dim3(grid), dim3(256), args, 0, nullptr));
      return CREDIT_OK;
    }
    mb_barrier_kernel<<<grid, 256>>>(sa, members, barriers, valid, sinkp);
    return check_launch("mb_barrier_kernel");
  };
  CREDIT_TRY(time_ms(plain, warmup, iters, plain_ms));
  CREDIT_TRY(time_ms(timed, warmup, iters, split_ms));
  uint32_t flag = 0;
  CREDIT_HIP(hipMemcpy(&flag, watchdog, sizeof(flag), hipMemcpyDeviceToHost));
  if (flag != 0) return set_error(CREDIT_ERR_WATCHDOG, "barrier benchmark timed out");
  return CREDIT_OK;
}

}  // namespace credit

using namespace credit;

extern "C" int credit_microbench(int32_t which, int64_t bytes, int32_t iters, double* results,
                                 int32_t n_results) {
  CREDIT_TRY(check_ptr(results, "results"));
  if (n_results < 1) return set_error(CREDIT_ERR_BAD_CONFIG, "n_results must be >= 1");
  if (iters < 0) return set_error(CREDIT_ERR_BAD_CONFIG, "iters must be >= 0");
  for (int i = 0; i < n_results; ++i) results[i] = 0.0;
  switch (which) {
    case CREDIT_MB_HBM_READ:
    case CREDIT_MB_HBM_WRITE:
    case CREDIT_MB_HBM_COPY:
      return bench_stream(which, bytes, iters > 0 ? iters : 20, results, n_results);
    case CREDIT_MB_CLOCK:
      return bench_clock(results, n_results);
    case CREDIT_MB_LATENCY:
      return bench_chase(iters, results, n_results);
    case CREDIT_MB_LDS_READ:
      return bench_lds(false, iters, results, n_results);
    case CREDIT_MB_LDS_WRITE:
      return bench_lds(true, iters, results, n_results);
    case CREDIT_MB_EXCHANGE_ROUNDTRIP:
      return bench_pingpong(iters, results, n_results);
    default:
      return set_error(CREDIT_ERR_BAD_CONFIG, "unknown microbenchmark %d", which);
  }
}

extern "C" int credit_control_overhead(int64_t rows, int32_t split, int32_t barriers,
                                       int32_t warmup, int32_t iters, int32_t cooperative,
                                       double* plain_ms, double* split_ms) {
  CREDIT_TRY(check_ptr(plain_ms, "plain_ms"));
  CREDIT_TRY(check_ptr(split_ms, "split_ms"));
  if (rows < 1 || barriers < 0 || warmup < 0 || iters < 1)
    return set_error(CREDIT_ERR_BAD_CONFIG, "rows >= 1, barriers >= 0, iters >= 1 required");
  return control_overhead(rows, split, barriers, warmup, iters, plain_ms, split_ms, cooperative);
}
