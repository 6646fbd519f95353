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

#include <algorithm>
#include <chrono>
#include <vector>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

// --------------------------------------------------------- HBM streams ---
// R source and W destination streams of equal length: a read:write byte mix
// of R:W.  Every workgroup of T lanes moves chunks of T*U 16-byte vectors
// per stream (each lane U vectors per stream), chunk c = blockIdx.x + k*grid:
// the whole grid advances through the streams as one narrow front, which is
// the access order the settled measurements found fastest (one large
// contiguous region per workgroup ran 10% slower at 1:1).  Loads are
// nontemporal; stores nontemporal (SP = kBufferNt) or plain (SP = 0).  The
// destination value depends on every source vector, so no load is dead.
struct StreamArgs {
  const void* src[4];
  void* dst[2];
  uint32_t bytes;  // per stream, a multiple of T * U * 16
};

template <int R, int W, int U, int SP>
__global__ __launch_bounds__(512) void mb_stream_kernel(StreamArgs a, uint32_t* sink) {
  const uint32_t lanes = blockDim.x;
  const uint32_t chunk = lanes * U * 16u;
  const uint32_t nchunks = a.bytes / chunk;
  buffer_rsrc_t rs[R > 0 ? R : 1];
  buffer_rsrc_t ws[W > 0 ? W : 1];
#pragma unroll
  for (int i = 0; i < R; ++i) rs[i] = make_rsrc(a.src[i], a.bytes);
#pragma unroll
  for (int i = 0; i < W; ++i) ws[i] = make_rsrc(a.dst[i], a.bytes);
  u32x4 acc = {0, 0, 0, 0};
  for (uint32_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const uint32_t base = c * chunk + threadIdx.x * 16u;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = u32x4{c, c, c, c};
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u)
        v[u] += __builtin_amdgcn_raw_buffer_load_b128(rs[i], base + u * lanes * 16u, 0, kBufferNt);
#pragma unroll
    for (int i = 0; i < W; ++i)
#pragma unroll
      for (int u = 0; u < U; ++u)
        __builtin_amdgcn_raw_buffer_store_b128(v[u] + static_cast<uint32_t>(i), ws[i],
                                               base + u * lanes * 16u, 0, SP);
    if (W == 0)
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  // Read-only streams: a data-dependent store that never fires keeps the
  // loads alive.
  if (W == 0 && acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u) sink[0] = acc.z;
}

using StreamFn = void (*)(StreamArgs, uint32_t*);

template <int R, int W, int U>
StreamFn stream_fn(bool nt_store) {
  return nt_store ? mb_stream_kernel<R, W, U, kBufferNt> : mb_stream_kernel<R, W, U, 0>;
}

template <int R, int W>
StreamFn stream_fn_u(int u, bool nt_store) {
  switch (u) {
    case 1: return stream_fn<R, W, 1>(nt_store);
    case 2: return stream_fn<R, W, 2>(nt_store);
    case 4: return stream_fn<R, W, 4>(nt_store);
    default: return stream_fn<R, W, 8>(nt_store);
  }
}

StreamFn stream_kernel_for(int reads, int writes, int u, bool nt_store) {
  const int mix = reads * 10 + writes;
  switch (mix) {
    case 10: return stream_fn_u<1, 0>(u, nt_store);
    case 1: return stream_fn_u<0, 1>(u, nt_store);
    case 11: return stream_fn_u<1, 1>(u, nt_store);
    case 21: return stream_fn_u<2, 1>(u, nt_store);
    case 31: return stream_fn_u<3, 1>(u, nt_store);
    case 41: return stream_fn_u<4, 1>(u, nt_store);
    case 32: return stream_fn_u<3, 2>(u, nt_store);
    case 22: return stream_fn_u<2, 2>(u, nt_store);
    case 12: return stream_fn_u<1, 2>(u, nt_store);
    default: return nullptr;
  }
}

// Launch shapes tried per mix: lanes per workgroup, vectors per lane and
// stream, workgroups per CU.  Each stays under 48 KiB of loads in flight
// per CU; the settled sweep over 64..1024 lanes, 1..16 vectors and 1..8
// workgroups per CU put every mix's best among these.
struct StreamShape {
  int lanes, u, per_cu;
};
constexpr StreamShape kStreamShapes[] = {
    {64, 4, 4}, {128, 2, 4}, {256, 4, 1}, {256, 2, 1}, {512, 1, 2}, {512, 2, 1}, {256, 8, 1},
};
constexpr int kStreamShapeCount = sizeof(kStreamShapes) / sizeof(kStreamShapes[0]);
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
// The workgroup has the block size and the dynamic LDS of the split launch
// it prices (src/cluster_control.cu:76-88 sizes its cluster kernel's shared
// memory the same way), so it holds the same workgroups per CU; thread 0
// touches the LDS, as there.
__global__ __launch_bounds__(1024) void mb_barrier_kernel(SplitArgs sa, int members,
                                                          int barriers, int rows,
                                                          double* sink, int lds_bytes) {
  extern __shared__ unsigned char mb_lds[];
  if (threadIdx.x == 0 && lds_bytes > 0) mb_lds[0] = 1;
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
  if (lds_bytes > 0 && threadIdx.x == 0) acc += mb_lds[0];
  if (acc == -1.0 && threadIdx.x == 0) sink[0] = acc;  // keeps the reads alive
  split_leave(sa);
}

__global__ __launch_bounds__(256) void mb_plain_kernel(int* sink) {
  if (threadIdx.x == 0 && blockIdx.x == 0x7fffffff) sink[0] = 1;
}

// ------------------------------------------------- L1 / L2 bandwidth (H2) -
// Every workgroup reads a `bytes`-long buffer `passes` times with plain
// dwordx4 loads, starting at a rotated offset so concurrent workgroups hit
// different channels.  Sized to fit the CU's vector L1 (16 KiB, one
// workgroup per CU) the loads hit L1; sized far above L1 and below one XCD's
// 4 MiB L2 (2 MiB) they miss L1 and hit L2.  Thread 0 records s_memtime
// cycles around the passes.
template <int U>
__global__ __launch_bounds__(1024) void mb_cache_read_kernel(const u32x4* __restrict__ buf,
                                                             uint32_t nvec, int passes,
                                                             uint32_t* sink, uint64_t* cycles) {
  const uint32_t lanes = blockDim.x;
  const uint32_t rot = (blockIdx.x * 2048u) % nvec;
  u32x4 acc = {0, 0, 0, 0};
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int p = 0; p < passes; ++p) {
    // An index the compiler cannot prove the same every pass: no load is
    // hoisted out of the pass loop.
    uint32_t first = threadIdx.x;
    __asm__ volatile("" : "+v"(first));
    for (uint32_t i = first; i < nvec; i += lanes * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t j = i + u * lanes + rot;
        j = j >= nvec ? j - nvec : j;
        v[u] = buf[j];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u];
    }
  }
  __syncthreads();
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
  if (acc.x == 0x9e3779b9u && acc.w == 0x7f4a7c15u) sink[0] = acc.y;
}

// ----------------------------------------- exchange slot throughput (H3) --
// One workgroup per CU; its first wave stores 64 tagged 64-bit slots per
// round to its own 512-byte row with device-scope atomic stores (the
// publish of the split kernels, all lanes at once), `rounds` rounds, then
// waits for every store to be acknowledged.  s_memtime cycles of wave 0.
__global__ __launch_bounds__(64) void mb_slot_store_kernel(uint64_t* slots, int rounds,
                                                           uint64_t* cycles) {
  uint64_t* row = slots + static_cast<size_t>(blockIdx.x) * kWave;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int r = 0; r < rounds; ++r)
    __hip_atomic_store(row + threadIdx.x,
                       (static_cast<uint64_t>(r + 1) << 32) | threadIdx.x, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  publish_wait();
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
}

// Ticket draws: lane 0 of every workgroup takes `draws` tickets one after
// another (each waits for the returned value, as split_join does) from its
// own 64-byte line (shared == 0) or from one line every workgroup uses.
__global__ __launch_bounds__(64) void mb_ticket_kernel(uint32_t* lines, int draws, int shared,
                                                       uint64_t* cycles) {
  if (threadIdx.x != 0) return;
  uint32_t* line = lines + (shared ? 0 : (static_cast<size_t>(blockIdx.x) + 1) * 16);
  uint32_t t = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  // Each draw's operand depends on the previous ticket (the sum stays far
  // below 2^31, so the increment is always 1).
  for (int d = 0; d < draws; ++d)
    t += __hip_atomic_fetch_add(line, 1u + (t >> 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  cycles[blockIdx.x] = t1 - t0 + (t >> 31);
}

// ------------------------------------------------------ MFMA rate ---
// Dense bf16 MFMA issue rate: every wave runs `iters` rounds of CHAINS
// independent v_mfma_f32_32x32x16_bf16 (no memory traffic in the loop), and
// records its shader-clock and 100 MHz constant-clock deltas.  Operands are
// small constants so the accumulators stay finite; the sums are stored so
// the chains are not dead code.
typedef __bf16 mb_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mb_f32x16 __attribute__((ext_vector_type(16)));
constexpr int kMfmaChains = 8;

__global__ __launch_bounds__(512) void mb_mfma_kernel(int iters, float* sink, uint64_t* clocks) {
  extern __shared__ char hold[];  // sized by the launch to keep one workgroup per CU
  const int lane = threadIdx.x & 63;
  mb_bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = static_cast<__bf16>(1.0f / 1024.0f * static_cast<float>((lane + e) & 7));
    b[e] = static_cast<__bf16>(1.0f / 4096.0f * static_cast<float>((lane * 3 + e) & 7));
  }
  mb_f32x16 acc[kMfmaChains];
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c)
      acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s + static_cast<float>(hold[0] & 0);
  if (lane == 0) {
    clocks[2 * wave] = t1 - t0;
    clocks[2 * wave + 1] = r1 - r0;
  }
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

// Settle the HBM clocks with `settle_ms` of back-to-back launches
// (synchronised every 8), then `trials` timed blocks of `iters` launches;
// *median_ms = the median block's time per launch.  After an idle period
// the first 10-20 ms of HBM traffic on the MI355X run slow.
template <class F>
int settled_median_ms(F&& launch, double settle_ms, int trials, int iters, double* median_ms) {
  int i = 0;
  const auto t_end = std::chrono::steady_clock::now() +
                     std::chrono::microseconds(static_cast<int64_t>(settle_ms * 1e3));
  while (std::chrono::steady_clock::now() < t_end) {
    for (int k = 0; k < 8; ++k) CREDIT_TRY(launch(i++));
    CREDIT_HIP(hipDeviceSynchronize());
  }
  Events ev;
  CREDIT_HIP(hipEventCreate(&ev.a));
  CREDIT_HIP(hipEventCreate(&ev.b));
  std::vector<double> per_call;
  for (int t = 0; t < trials; ++t) {
    CREDIT_HIP(hipEventRecord(ev.a, nullptr));
    for (int k = 0; k < iters; ++k) CREDIT_TRY(launch(i++));
    CREDIT_HIP(hipEventRecord(ev.b, nullptr));
    CREDIT_HIP(hipEventSynchronize(ev.b));
    float ms = 0.0f;
    CREDIT_HIP(hipEventElapsedTime(&ms, ev.a, ev.b));
    per_call.push_back(static_cast<double>(ms) / iters);
  }
  std::sort(per_call.begin(), per_call.end());
  *median_ms = per_call[per_call.size() / 2];
  return CREDIT_OK;
}

}  // namespace

// The stream ceiling of a read:write mix: every shape of kStreamShapes with
// nontemporal and with plain stores over three rotating buffer sets.
// results: [0] best GB/s (bytes moved / median time per call), [1] its
// median ms per call, [2] lanes, [3] vectors per lane, [4] workgroups per
// CU, [5] 1 for nontemporal stores, [6] bytes moved per call, then GB/s of
// each (shape, store policy) in table order, nontemporal first.
int stream_ceiling(int reads, int writes, int64_t call_bytes, int trials, int iters,
                   double settle_ms, double* results, int n) {
  if (reads < 0 || writes < 0 || reads > 4 || writes > 2 || reads + writes == 0 ||
      stream_kernel_for(reads, writes, 1, true) == nullptr)
    return set_error(CREDIT_ERR_BAD_CONFIG,
                     "stream mix %d:%d not built (reads 0..4, writes 0..2: 1:0 0:1 1:1 2:1 "
                     "3:1 4:1 3:2 2:2 1:2)", reads, writes);
  if (trials < 1 || iters < 1) return set_error(CREDIT_ERR_BAD_CONFIG, "trials, iters >= 1");
  const int streams = reads + writes;
  constexpr int64_t kGranule = int64_t{512} * 8 * 16;  // the largest chunk, 64 KiB
  const int64_t per = call_bytes / streams / kGranule * kGranule;
  if (per < kGranule || per > (int64_t{1} << 32) - kGranule)
    return set_error(CREDIT_ERR_BAD_CONFIG,
                     "%lld bytes per call over %d streams: each stream must hold 64 KiB to 4 GiB",
                     static_cast<long long>(call_bytes), streams);
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  constexpr int kSets = 3;
  std::vector<DevBuf> bufs(static_cast<size_t>(kSets) * streams);
  for (DevBuf& b : bufs) CREDIT_TRY(b.alloc(static_cast<size_t>(per)));
  DevBuf sink;
  CREDIT_TRY(sink.alloc(256));
  StreamArgs sets[kSets];
  for (int k = 0; k < kSets; ++k) {
    sets[k] = StreamArgs{};
    sets[k].bytes = static_cast<uint32_t>(per);
    for (int i = 0; i < reads; ++i) sets[k].src[i] = bufs[k * streams + i].p;
    for (int i = 0; i < writes; ++i) sets[k].dst[i] = bufs[k * streams + reads + i].p;
  }
  const double moved = static_cast<double>(per) * streams;
  double best = 0.0;
  int slot = 7;
  for (int i = 0; i < 7 && i < n; ++i) results[i] = 0.0;
  for (int nt = 1; nt >= 0; --nt) {
    if (writes == 0 && nt == 0) break;  // no stores to vary
    for (const StreamShape& sh : kStreamShapes) {
      const StreamFn fn = stream_kernel_for(reads, writes, sh.u, nt != 0);
      const unsigned grid = static_cast<unsigned>(props->cu_count * sh.per_cu);
      auto launch = [&](int i) -> int {
        hipLaunchKernelGGL(fn, dim3(grid), dim3(sh.lanes), 0, nullptr, sets[i % kSets],
                           static_cast<uint32_t*>(sink.p));
        return check_launch("mb_stream_kernel");
      };
      double ms = 0.0;
      CREDIT_TRY(settled_median_ms(launch, settle_ms, trials, iters, &ms));
      const double gbps = moved / (ms * 1e-3) / 1e9;
      if (slot < n) results[slot] = gbps;
      ++slot;
      if (gbps > best) {
        best = gbps;
        const double rec[7] = {gbps, ms, static_cast<double>(sh.lanes), static_cast<double>(sh.u),
                               static_cast<double>(sh.per_cu), static_cast<double>(nt), moved};
        for (int i = 0; i < 7 && i < n; ++i) results[i] = rec[i];
      }
    }
  }
  return CREDIT_OK;
}

namespace {

// The runtime's own device-to-device copy (hipMemcpyAsync on the null
// stream) of `bytes` per call, over the stream ceiling's three rotating
// buffer sets, settle phase and trial blocks: an independent 1:1 ceiling
// beside the library's stream kernels.  results: [0] GB/s (read + write
// bytes over the median call time), [1] ms per call.
int bench_runtime_copy(int64_t bytes, int iters, double* results, int n) {
  if (bytes < (int64_t{1} << 20)) bytes = int64_t{128} << 20;
  if (iters <= 0) iters = 20;
  constexpr int kSets = 3;
  std::vector<DevBuf> src(kSets), dst(kSets);
  for (int k = 0; k < kSets; ++k) {
    CREDIT_TRY(src[k].alloc(static_cast<size_t>(bytes)));
    CREDIT_TRY(dst[k].alloc(static_cast<size_t>(bytes)));
  }
  auto launch = [&](int i) -> int {
    CREDIT_HIP(hipMemcpyAsync(dst[i % kSets].p, src[i % kSets].p, static_cast<size_t>(bytes),
                              hipMemcpyDeviceToDevice, nullptr));
    return CREDIT_OK;
  };
  double ms = 0.0;
  CREDIT_TRY(settled_median_ms(launch, 20.0, 5, iters, &ms));
  results[0] = 2.0 * static_cast<double>(bytes) / (ms * 1e-3) / 1e9;
  if (n > 1) results[1] = ms;
  return CREDIT_OK;
}

int bench_stream(int which, int64_t bytes, int iters, double* results, int n) {
  if (bytes < (int64_t{1} << 20)) bytes = int64_t{1} << 30;
  const int reads = which == CREDIT_MB_HBM_WRITE ? 0 : 1;
  const int writes = which == CREDIT_MB_HBM_READ ? 0 : 1;
  // results[0] = best GB/s, then the per-shape figures of stream_ceiling.
  std::vector<double> r(7 + 2 * kStreamShapeCount, 0.0);
  CREDIT_TRY(stream_ceiling(reads, writes, bytes * (reads + writes), 5, iters, 20.0, r.data(),
                            static_cast<int>(r.size())));
  results[0] = r[0];
  for (int i = 0; i + 1 < n && 7 + i < static_cast<int>(r.size()); ++i) results[1 + i] = r[7 + i];
  return CREDIT_OK;
}

// XCC of every workgroup of a grid (hardware register XCC_ID, read with
// s_getreg): the dispatch order the split launches' dispenser subsets rely
// on (workgroup b on XCC b % 8).
__global__ __launch_bounds__(64) void mb_xcc_kernel(uint32_t* out) {
  // hwreg(HW_REG_XCC_ID = 20, offset 0, size 4): size-1 in [15:11], id in [5:0].
  const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xfu;
  if (threadIdx.x == 0) out[blockIdx.x] = xcc;
}

// results[b] = XCC of workgroup b of a grid of n workgroups (n <= 65536).
int bench_xcc_map(double* results, int n) {
  if (n < 1 || n > 65536) return set_error(CREDIT_ERR_BAD_CONFIG, "n_results %d (1..65536)", n);
  DevBuf out;
  CREDIT_TRY(out.alloc(static_cast<size_t>(n) * 4));
  mb_xcc_kernel<<<static_cast<unsigned>(n), 64>>>(static_cast<uint32_t*>(out.p));
  CREDIT_TRY(check_launch("mb_xcc_kernel"));
  std::vector<uint32_t> h(static_cast<size_t>(n));
  CREDIT_HIP(hipMemcpy(h.data(), out.p, h.size() * 4, hipMemcpyDeviceToHost));
  for (int i = 0; i < n; ++i) results[i] = static_cast<double>(h[static_cast<size_t>(i)]);
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

uint64_t max_of(const std::vector<uint64_t>& v) {
  uint64_t worst = 1;
  for (uint64_t c : v) worst = c > worst ? c : worst;
  return worst;
}

// [0] B/cycle per CU from its vector L1: one 1024-lane workgroup per CU
// (its 96 KiB LDS allocation keeps a second one off the CU) re-reading
// 16 KiB, s_memtime cycles of the slowest.  [1] B/cycle per XCD from L2:
// two 1024-lane workgroups per CU re-reading a 2 MiB buffer, timed with
// events over the launch and converted at the measured shader clock; [2]
// that L2 rate as device GB/s.
int bench_cache(int passes, double* results, int n) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (passes <= 0) passes = 64;
  DevBuf buf, sink, cyc;
  CREDIT_TRY(buf.alloc(size_t{2} << 20));
  CREDIT_TRY(sink.alloc(256));
  CREDIT_TRY(cyc.alloc(sizeof(uint64_t) * props->cu_count * 2));
  std::vector<uint64_t> h(props->cu_count);
  const u32x4* b = static_cast<const u32x4*>(buf.p);
  constexpr size_t kHoldCu = size_t{96} << 10;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(mb_cache_read_kernel<1>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kHoldCu));
  if (attr != hipSuccess) return hip_failure(attr, "hipFuncSetAttribute(mb_cache_read_kernel)");
  // L1: 16 KiB = 1024 vectors, one vector per lane per pass.
  mb_cache_read_kernel<1><<<props->cu_count, 1024, kHoldCu>>>(
      b, 1024u, passes * 16, static_cast<uint32_t*>(sink.p), static_cast<uint64_t*>(cyc.p));
  CREDIT_TRY(check_launch("mb_cache_read_kernel"));
  CREDIT_HIP(hipMemcpy(h.data(), cyc.p, sizeof(uint64_t) * props->cu_count,
                       hipMemcpyDeviceToHost));
  results[0] = 16384.0 * passes * 16 / static_cast<double>(max_of(h));
  // L2: 2 MiB = 131072 vectors per workgroup pass.
  const int grid = props->cu_count * 2;
  const int l2_passes = passes / 4 > 0 ? passes / 4 : 1;
  auto launch = [&](int) -> int {
    mb_cache_read_kernel<4><<<grid, 1024>>>(b, 131072u, l2_passes,
                                            static_cast<uint32_t*>(sink.p),
                                            static_cast<uint64_t*>(cyc.p));
    return check_launch("mb_cache_read_kernel");
  };
  double ms = 0.0;
  CREDIT_TRY(time_ms(launch, 2, 5, &ms));
  const double bytes = (double{2} * (1 << 20)) * l2_passes * grid;
  const double gbps = bytes / (ms * 1e-3) / 1e9;
  double clk[1] = {0.0};
  CREDIT_TRY(bench_clock(clk, 1));
  if (n > 1) results[1] = gbps * 1e9 / (clk[0] * 1e6) / props->xcd_count;
  if (n > 2) results[2] = gbps;
  return CREDIT_OK;
}

// Dense bf16 MFMA rate with one workgroup per CU of 4 waves (one per
// SIMD) and of 8 waves (two per SIMD), each settled for about 100 ms and
// timed as the median of five launches of about 5 ms.  results: [0] best
// TFLOP/s, [1] the mean shader clock of its waves during the MFMA loop
// (MHz, from s_memtime against the 100 MHz s_memrealtime), [2] its flops per
// shader cycle per CU, [3] waves per SIMD of the best, [4] TFLOP/s with 4
// waves, [5] with 8.
int bench_mfma(int iters, double* results, int n) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (iters <= 0) iters = 20000;
  constexpr int kHold = 96 << 10;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(mb_mfma_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kHold);
  if (attr != hipSuccess) return hip_failure(attr, "hipFuncSetAttribute(mb_mfma_kernel)");
  const int cus = props->cu_count;
  DevBuf sink, clk;
  CREDIT_TRY(sink.alloc(sizeof(float) * cus * 512));
  CREDIT_TRY(clk.alloc(sizeof(uint64_t) * 2 * cus * 8));
  double best = 0.0, best_mhz = 0.0, best_waves = 0.0, rate[2] = {0.0, 0.0};
  for (int v = 0; v < 2; ++v) {
    const int threads = 256 << v;
    auto launch = [&](int) -> int {
      mb_mfma_kernel<<<cus, threads, kHold>>>(iters, static_cast<float*>(sink.p),
                                              static_cast<uint64_t*>(clk.p));
      return check_launch("mb_mfma_kernel");
    };
    double ms = 0.0;
    CREDIT_TRY(settled_median_ms(launch, 100.0, 5, 1, &ms));
    const double flops = 2.0 * 32 * 32 * 16 * kMfmaChains * static_cast<double>(iters) *
                         (threads / 64) * cus;
    rate[v] = flops / (ms * 1e-3) / 1e12;
    const int waves = cus * threads / 64;
    std::vector<uint64_t> h(static_cast<size_t>(2) * waves);
    CREDIT_HIP(hipMemcpy(h.data(), clk.p, sizeof(uint64_t) * h.size(), hipMemcpyDeviceToHost));
    double mhz = 0.0;
    for (int w = 0; w < waves; ++w)
      mhz += static_cast<double>(h[2 * w]) / (static_cast<double>(h[2 * w + 1]) / 100.0);
    mhz /= waves;
    if (rate[v] > best) {
      best = rate[v];
      best_mhz = mhz;
      best_waves = (threads / 64) / 4;
    }
  }
  results[0] = best;
  if (n > 1) results[1] = best_mhz;
  if (n > 2) results[2] = best * 1e12 / (best_mhz * 1e6) / cus;
  if (n > 3) results[3] = best_waves;
  if (n > 4) results[4] = rate[0];
  if (n > 5) results[5] = rate[1];
  return CREDIT_OK;
}

// [0] bytes per cycle per workgroup of device-scope slot stores with one
// workgroup per CU, [1] the same stores as GB/s over the device, [2] cycles
// per ticket draw on a workgroup's own line, [3] cycles per draw when one
// workgroup per CU draws from one shared line.
int bench_exchange_throughput(int rounds, double* results, int n) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (rounds <= 0) rounds = 4096;
  const int grid = props->cu_count;
  DevBuf slots, lines, cyc;
  CREDIT_TRY(slots.alloc(sizeof(uint64_t) * kWave * grid));
  CREDIT_TRY(lines.alloc(size_t{64} * (grid + 1)));
  CREDIT_TRY(cyc.alloc(sizeof(uint64_t) * grid));
  std::vector<uint64_t> h(grid);
  mb_slot_store_kernel<<<grid, 64>>>(static_cast<uint64_t*>(slots.p), rounds,
                                     static_cast<uint64_t*>(cyc.p));
  CREDIT_TRY(check_launch("mb_slot_store_kernel"));
  CREDIT_HIP(hipMemcpy(h.data(), cyc.p, sizeof(uint64_t) * grid, hipMemcpyDeviceToHost));
  const double store_cycles = static_cast<double>(max_of(h));
  const double per_wg = 8.0 * kWave * rounds;
  results[0] = per_wg / store_cycles;
  double clk[1] = {0.0};
  CREDIT_TRY(bench_clock(clk, 1));
  if (n > 1) results[1] = per_wg * grid / (store_cycles / (clk[0] * 1e6)) / 1e9;
  const int draws = rounds / 4 > 0 ? rounds / 4 : 1;
  for (int shared = 0; shared <= 1; ++shared) {
    CREDIT_HIP(hipMemset(lines.p, 0, size_t{64} * (grid + 1)));
    mb_ticket_kernel<<<grid, 64>>>(static_cast<uint32_t*>(lines.p), draws, shared,
                                   static_cast<uint64_t*>(cyc.p));
    CREDIT_TRY(check_launch("mb_ticket_kernel"));
    CREDIT_HIP(hipMemcpy(h.data(), cyc.p, sizeof(uint64_t) * grid, hipMemcpyDeviceToHost));
    if (n > 2 + shared) results[2 + shared] = static_cast<double>(max_of(h)) / draws;
  }
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

int control_overhead(int64_t rows, int split, int barriers, int lds_bytes, int threads,
                     int warmup, int iters, double* plain_ms, double* split_ms, int cooperative) {
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  if (split < 1 || split > 64) return set_error(CREDIT_ERR_BAD_CONFIG, "split %d", split);
  if (rows < 1) return set_error(CREDIT_ERR_BAD_CONFIG, "rows must be >= 1");
  if (threads == 0) threads = 256;
  if (threads < kWave || threads > 1024 || threads % kWave != 0)
    return set_error(CREDIT_ERR_BAD_CONFIG, "threads %d (a multiple of 64 up to 1024)", threads);
  if (lds_bytes < 0 || lds_bytes > props->max_lds_per_block)
    return set_error(CREDIT_ERR_BAD_CONFIG, "lds_bytes %d (at most %d)", lds_bytes,
                     props->max_lds_per_block);
  const void* fn = reinterpret_cast<const void*>(mb_barrier_kernel);
  const size_t lds = static_cast<size_t>(lds_bytes);
  if (lds > 65536) CREDIT_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  static_cast<int>(lds)));
  int64_t groups = 0;
  int dispensers = 0;
  CREDIT_TRY(coresident_groups(fn, threads, lds, split, &groups, &dispensers));
  if (groups < 1) return set_error(CREDIT_ERR_UNSUPPORTED, "split %d does not fit", split);
  if (groups > padded_groups(rows)) groups = padded_groups(rows);
  const int64_t per_group = (rows + groups - 1) / groups;
  const int64_t stages64 = per_group * (barriers > 0 ? barriers : 1);
  if (stages64 > int64_t{credit::plan::kMaxLaunchStages})
    return set_error(CREDIT_ERR_BAD_CONFIG, "%lld barriers per group", static_cast<long long>(stages64));
  DevBuf ws, sink;
  if (split_slot_bytes(groups, split, 1, kSplitRing) > kSlotAreaBytes)
    return set_error(CREDIT_ERR_UNSUPPORTED, "barrier benchmark slots exceed the slot area");
  CREDIT_TRY(ws.alloc(kScratchOffset));
  CREDIT_TRY(sink.alloc(256));
  char* base = static_cast<char*>(ws.p);
  uint32_t* counters = ws_counters(base);
  uint32_t* watchdog = ws_watchdog(base);
  uint64_t* slots = ws_slots(base);
  double* sinkp = static_cast<double*>(sink.p);
  const unsigned grid = static_cast<unsigned>(groups * split);
  // The plain reference launches one workgroup per (row, member): the work
  // items a split launch covers, with no exchange.
  const unsigned plain_grid = static_cast<unsigned>(rows * split);
  const uint32_t total = grid;
  int valid = static_cast<int>(rows);
  int lds_arg = lds_bytes;
  SplitArgs sa{counters, slots, watchdog, total, static_cast<uint32_t>(stages64), kSplitRing};
  sa.dispensers = static_cast<uint32_t>(dispensers);
  auto plain = [&](int) -> int {
    mb_plain_kernel<<<plain_grid, 256>>>(static_cast<int*>(sink.p));
    return check_launch("mb_plain_kernel");
  };
  int members = split;
  auto timed = [&](int) -> int {
    if (cooperative) {
      void* args[] = {&sa, &members, &barriers, &valid, &sinkp, &lds_arg};
      CREDIT_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(threads), args, lds, nullptr));
      return CREDIT_OK;
    }
    mb_barrier_kernel<<<grid, threads, lds>>>(sa, members, barriers, valid, sinkp, lds_arg);
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
    case CREDIT_MB_CACHE_READ:
      return bench_cache(iters, results, n_results);
    case CREDIT_MB_EXCHANGE_THROUGHPUT:
      return bench_exchange_throughput(iters, results, n_results);
    case CREDIT_MB_MFMA_BF16:
      return bench_mfma(iters, results, n_results);
    case CREDIT_MB_XCC_MAP:
      return bench_xcc_map(results, n_results);
    case CREDIT_MB_RUNTIME_COPY:
      return bench_runtime_copy(bytes, iters, results, n_results);
    default:
      return set_error(CREDIT_ERR_BAD_CONFIG, "unknown microbenchmark %d", which);
  }
}

extern "C" int credit_stream_ceiling(int32_t reads, int32_t writes, int64_t call_bytes,
                                     int32_t trials, int32_t iters, double settle_ms,
                                     double* results, int32_t n_results) {
  CREDIT_TRY(check_ptr(results, "results"));
  if (n_results < 1) return set_error(CREDIT_ERR_BAD_CONFIG, "n_results must be >= 1");
  if (!(settle_ms >= 0.0) || settle_ms > 10000.0)
    return set_error(CREDIT_ERR_BAD_CONFIG, "settle_ms must lie in [0, 10000]");
  for (int i = 0; i < n_results; ++i) results[i] = 0.0;
  return stream_ceiling(reads, writes, call_bytes, trials, iters, settle_ms, results, n_results);
}

extern "C" int credit_control_overhead(int64_t rows, int32_t split, int32_t barriers,
                                       int32_t lds_bytes, int32_t threads, int32_t warmup,
                                       int32_t iters, int32_t cooperative, double* plain_ms,
                                       double* split_ms) {
  CREDIT_TRY(check_ptr(plain_ms, "plain_ms"));
  CREDIT_TRY(check_ptr(split_ms, "split_ms"));
  if (rows < 1 || barriers < 0 || warmup < 0 || iters < 1)
    return set_error(CREDIT_ERR_BAD_CONFIG, "rows >= 1, barriers >= 0, iters >= 1 required");
  return control_overhead(rows, split, barriers, lds_bytes, threads, warmup, iters, plain_ms,
                          split_ms, cooperative);
}
