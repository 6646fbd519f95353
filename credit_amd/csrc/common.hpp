// Device-side building blocks shared by every wide-row kernel (gfx950 / CDNA4).
//
// The reference duplicates its reduction helpers in every workload file
// (warp shuffle -> 8-slot shared array -> warp 0, e.g.
// src/workloads/layernorm_backward.cu:177-251).  On CDNA4 a wavefront is 64
// lanes, so the in-wave part is four DPP steps inside each 16-lane row plus
// four v_readlane reads across rows; the cross-wave part is one LDS round; the
// cross-workgroup part (the reference's DSMEM cluster exchange) is an
// L2/MALL-resident scratch exchange through device-scope atomics.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "api_internal.hpp"

namespace credit {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 ----
// bf16 is carried as raw uint16 bits in memory.  Widening is a shift; the
// narrowing conversion is round-to-nearest-even with NaN kept quiet, which is
// what torch's float->bfloat16 cast does.  gfx950 has a packed hardware
// conversion (v_cvt_pk_bf16_f32), reached through the __bf16 vector cast.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __builtin_bit_cast(float, packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __builtin_bit_cast(float, packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  float2_t f = {lo, hi};
  bf16x2_t b = __builtin_convertvector(f, bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  return static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xffffu);
}
// a.lo * b.lo + a.hi * b.hi + c on two packed bf16 pairs (v_dot2_f32_bf16):
// the bf16 products are exact in fp32.  With b = (1, 1) it sums a pair, with
// b = a it sums a pair's squares, one instruction per two elements.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ---------------------------------------------------------- max with NaN --
// torch.amax propagates NaN.  v_maximum3_f32 (IEEE 754-2019 maximum) does the
// same in one instruction, so the row max stays bit-exact with torch,
// including NaN rows.
__device__ __forceinline__ float fmax_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// ------------------------------------------------------- wave reductions --
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, 0xf,
                                             0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(
      0, static_cast<int>(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(
      double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                  static_cast<uint32_t>(lo));
}

// DPP controls: quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_half_mirror,
// row_mirror.  After the four steps every lane of a 16-lane row holds the
// row's total; the four row totals are then combined through v_readlane in a
// fixed order, so the result is wave-uniform and deterministic.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

struct SumOp {
  template <class T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return fmax_nan(a, b);
  }
};

template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_f32<kDppXor1>(v));
  v = op(v, dpp_f32<kDppXor2>(v));
  v = op(v, dpp_f32<kDppHalfMirror>(v));
  v = op(v, dpp_f32<kDppMirror>(v));
  const float a = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return op(op(a, b), op(c, d));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(u), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ double wave_reduce_sum_f64(double v) {
  v += dpp_f64<kDppXor1>(v);
  v += dpp_f64<kDppXor2>(v);
  v += dpp_f64<kDppHalfMirror>(v);
  v += dpp_f64<kDppMirror>(v);
  const double a = readlane_f64(v, 0), b = readlane_f64(v, 16);
  const double c = readlane_f64(v, 32), d = readlane_f64(v, 48);
  return (a + b) + (c + d);
}

// ------------------------------------------------------ block reductions --
// One LDS round: each wave deposits its wave-uniform value, one barrier, then
// every thread folds the NW slots in slot order.  Callers pass a distinct
// slot array per reduction that is live at the same time (or separate two
// uses of one array with a barrier), so no trailing barrier is needed.
template <int NW, class Op>
__device__ __forceinline__ float block_reduce(float v, Op op, float* slots) {
  v = wave_reduce(v, op);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = v;
  __syncthreads();
  float r = slots[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r = op(r, slots[w]);
  return r;
}

template <int NW>
__device__ __forceinline__ double block_reduce_sum_f64(double v, double* slots) {
  v = wave_reduce_sum_f64(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = v;
  __syncthreads();
  double r = slots[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r += slots[w];
  return r;
}

// K sums over the workgroup in one LDS round (one barrier): each wave
// deposits its K wave sums, then lane w < NW of every wave loads wave w's
// sum of value k and a second wave reduction folds them -- K LDS reads per
// lane instead of K*NW, which keeps the register footprint of several
// simultaneous sums flat in the workgroup size.  Fixed order: the result is
// deterministic and the same in every lane.  `slots` is [K][NW] and must not
// be reused before a later barrier.
template <int NW, int K>
__device__ __forceinline__ void block_reduce_sum_f64_multi(double (&v)[K], double (*slots)[NW]) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = wave_reduce_sum_f64(v[k]);
  if (lane == 0)
#pragma unroll
    for (int k = 0; k < K; ++k) slots[k][wave] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = wave_reduce_sum_f64(lane < NW ? slots[k][lane] : 0.0);
}

// --------------------------------------------------- memory access helpers
// Native clang vectors: the nontemporal builtins (global_load/store with the
// nt bit) accept these, not HIP's struct-wrapped float4/uint4.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 load_nt(const f32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ u32x4 load_nt(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ f64x2 load_nt(const f64x2* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void store_nt(f32x4* p, f32x4 v) {
  __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_nt(u32x4* p, u32x4 v) {
  __builtin_nontemporal_store(v, p);
}

// Raw buffer access (gfx9 buffer resource: base, stride 0, num_records
// bytes, dword3 = DATA_FORMAT 32).  A load beyond num_records returns 0
// and a store beyond it is dropped, in hardware: bounds and tail conditions
// fold into the resource (scalar registers) instead of branches, which
// matters for the waitcnt pass -- a load or store under a branch makes the
// number of operations in flight path-dependent, and the wait after the
// join then drains everything (vmcnt(0)).
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kBufferNt = 2;  // cache-policy operand: nontemporal ("nt")
using buffer_rsrc_t = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           kBufferRsrcWord3);
}
__device__ __forceinline__ u32x4 buffer_load_nt(buffer_rsrc_t r, uint32_t offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kBufferNt);
}
__device__ __forceinline__ u32x4 buffer_load(buffer_rsrc_t r, uint32_t offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
}
__device__ __forceinline__ void buffer_store_nt(buffer_rsrc_t r, uint32_t offset, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, offset, 0, kBufferNt);
}
// Atomic add through a buffer resource, returning the old value; lanes
// whose offset falls outside the resource change nothing (and read 0).
__device__ __forceinline__ uint32_t queue_add(buffer_rsrc_t q, uint32_t off, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(static_cast<int>(v), q, off, 0, 0));
}
__device__ __forceinline__ void buffer_store(buffer_rsrc_t r, uint32_t offset, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, offset, 0, 0);
}

// The lane index, re-defined opaquely: per-lane addresses and predicates
// derived from it inside a loop cannot be hoisted out of the loop (where
// they would stay live across iterations and raise register pressure).
__device__ __forceinline__ int opaque_lane_index() {
  int t = static_cast<int>(threadIdx.x);
  __asm__ volatile("" : "+v"(t));
  return t;
}

// *p += v on an LDS double that only this lane updates (ds_add_f64).
__device__ __forceinline__ void lds_add(double* p, double v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__global__ void fill_f32_kernel(float* __restrict__ p, float v, int64_t n);

// ------------------------------------- cross-workgroup exchange (L2/MALL) --
// CDNA4 has no distributed shared memory; workgroups exchange partials
// through device memory.  The L2 of each XCD is not coherent with the other
// seven, and the compiler's agent-scope acquire/release fences are whole-L2
// maintenance operations (buffer_wbl2 / buffer_inv), far too costly to issue
// once per workgroup.  The exchange therefore never relies on fences:
//  - partials are published with device-scope relaxed atomic stores
//    (global_store ... sc1: written through to the coherent level);
//  - publish_wait() is an explicit s_waitcnt vmcnt(0): every store of this
//    wave has been acknowledged before the arrival atomic issues;
//  - arrival counters are device-scope atomics, performed at the coherent
//    level for every XCD;
//  - waiting and reading partials use device-scope relaxed atomic loads
//    (global_load ... sc1: never served by a stale L2 line), and a wave
//    cannot issue a load that depends on the loop exit before the spin load
//    has returned.
__device__ __forceinline__ void publish_wait() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish(double* p, double v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch(const float* p) {
  return __builtin_bit_cast(
      float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ double fetch(const double* p) {
  return __builtin_bit_cast(
      double, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ uint32_t arrive(uint32_t* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_reset(uint32_t* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t counter_read(const uint32_t* counter) {
  return __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------ ticketed split groups ---
// P workgroups ("members") that share a row -- or a block of rows -- form a
// group and exchange partial results to combine them.
//
// Membership comes from a ticket, not from blockIdx.  The grid is split into
// D subsets by blockIdx % D (D = SplitArgs::dispensers: 8, one subset per
// XCD, or fewer when an XCD's slots hold fewer than two groups), each with
// its own device-scope ticket dispenser; thread 0 of every workgroup draws
// the next ticket of its subset as the workgroup starts, and ticket t of
// subset d makes it member t % P of group d * (subset size / P) + t / P
// (plan::seat_of).  The grid is a multiple of D * P, so every subset holds
// whole groups.  Within a subset a group's members hold consecutive tickets,
// so every group whose P tickets are drawn has all P members running, and at
// most one group per subset (the newest) is incomplete.  Split launches are
// sized to what the device holds at once (coresident_groups), and every
// subset's slots hold at least two groups, so no group needs every slot of
// its subset: a slot withheld from the launch delays a group until another
// group of the subset exits rather than stranding it.  One dispenser per
// subset keeps the same-address atomics off a single serialisation point.
// The workgroup that draws a subset's last ticket returns that dispenser to
// zero.  tests/cpp/split_protocol_model.cpp runs these rules on host threads.
//
// Exchange protocol: tagged slots, no counters.  Every (group, stage, value
// k, member) has its own 64-bit slot: the partial's fp32 bits in the low
// word and a tag in the high word, written by ONE device-scope atomic store.
// The tag of stage s is seq + 1 + s, where seq is the workspace header's
// sequence word as the launch starts; the launch's last workgroup to exit
// advances it by the launch's stage count (split_leave), so every launch --
// a replayed graph too -- owns tags no slot holds yet, and a publisher never
// waits for anything (no fence, no vmcnt drain of its own loads and stores):
// a reader that sees the tag in a slot sees that launch's value of that
// stage.  Stages use slot rows modulo `ring`: a kernel whose members run many
// stages reuses a slot row only once every member has polled it (the kernels
// guarantee that by their step structure).  One wave of each member polls
// the group's P*K slots of the stage (contiguous: one request per poll)
// until every tag matches, puts the values in LDS, and after a barrier every
// thread combines them in member order: all members, and every run, get
// bit-identical results.  Partials travel as fp32 (the block reductions
// before them are fp64); the combination is fp64.  The poll is bounded: on
// expiry it raises *watchdog (and the device's host-mapped watchdog word)
// and continues, so a broken launch ends with a reported error instead of a
// hung GPU.
constexpr uint32_t kSpinLimit = 1u << 21;  // ~1 s of s_sleep polling
constexpr int kMaxExchange = kMaxExchangeValues;  // members * values per stage
static_assert(kMaxExchange <= kWave, "one wave polls a stage's slots");

// Split-launch arguments, passed by value to every split kernel.  grid == 0
// marks a launch without groups (members == 1): no join, no leave.
struct SplitArgs {
  uint32_t* counters;  // workspace counter area (dispensers)
  uint64_t* slots;     // workspace slots, [group][stage % ring][k][member]
  uint32_t* header;    // workspace header: watchdog, sequence, exit count
  uint32_t grid;       // gridDim.x, a multiple of dispensers * members
  uint32_t stages;     // exchange tags the launch uses (<= plan::kMaxLaunchStages)
  int ring;            // slot rows per group (stages modulo ring)
  uint32_t dispensers = kDispensers;  // ticket subsets (blockIdx % dispensers)
  uint32_t spin_limit = kSpinLimit;   // polls before a wait gives up
  uint32_t* host_flag = nullptr;      // host-mapped word raised with the watchdog
};

// The product launches' arguments: the process-wide spin limit and the
// device's host-mapped watchdog word (credit_set_spin_limit, api.hip).
inline SplitArgs make_split_args(const SplitWorkspace& ws, uint32_t grid, uint32_t stages,
                                 int ring, int dispensers) {
  SplitArgs a{ws.counters, ws.slots, ws.watchdog, grid, stages, ring};
  a.dispensers = static_cast<uint32_t>(dispensers);
  a.spin_limit = split_spin_limit();
  a.host_flag = ws.host_flag;
  return a;
}

struct SplitGroup {
  int group;
  int member;
  int members;
  int k_values;
  int stage;
  int ring;
  uint32_t epoch;
  uint64_t* slots;    // this group's slots
  uint32_t* watchdog;
  uint32_t spin_limit;
  uint32_t* host_flag;
};

// What split_leave needs, stashed in LDS by split_join so that the launch
// arguments need not stay live in registers across the kernel.
struct SplitExit {
  uint32_t* subset_out;  // the subset's exited-workgroup count
  uint32_t* header;
  uint64_t* slots;
  uint32_t per_subset;
  uint32_t dispensers;
  uint32_t stages;
  uint32_t seq;          // the sequence word as the launch started
  uint32_t waves_out;    // waves of this workgroup that have left
};
__device__ __forceinline__ SplitExit* split_exit_lds() {
  __shared__ SplitExit exit_info;
  return &exit_info;
}

// Draw a ticket, read the launch's tag sequence and derive (group, member).
// Every thread calls it; it contains one __syncthreads.
__device__ __forceinline__ SplitGroup split_join(const SplitArgs& a, int members, int k_values) {
  __shared__ uint32_t join_s[2];  // ticket, sequence
  const uint32_t subset = blockIdx.x % a.dispensers;
  const uint32_t per_subset = a.grid / a.dispensers;
  if (threadIdx.x == 0) {
    uint32_t* dispenser = a.counters + subset * kDispenserStride;
    const uint32_t t = __hip_atomic_fetch_add(dispenser, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    if (t == per_subset - 1) counter_reset(dispenser);
    const uint32_t seq = __hip_atomic_load(a.header + kHeaderSeqWord, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    join_s[0] = t;
    join_s[1] = seq;
    *split_exit_lds() = SplitExit{a.counters + subset * kDispenserStride + 1, a.header, a.slots,
                                  per_subset, a.dispensers, a.stages, seq, 0u};
  }
  __syncthreads();
  // readfirstlane: the ticket is workgroup-uniform, and saying so keeps the
  // group/member arithmetic (and everything addressed by it) scalar.
  const uint32_t t = __builtin_amdgcn_readfirstlane(join_s[0]);
  const plan::Seat seat = plan::seat_of(blockIdx.x, t, a.grid, a.dispensers,
                                        static_cast<uint32_t>(members));
  SplitGroup g;
  g.group = seat.group;
  g.member = seat.member;
  g.members = members;
  g.k_values = k_values;
  g.stage = 0;
  g.ring = a.ring;
  g.epoch = plan::launch_epoch(__builtin_amdgcn_readfirstlane(join_s[1]));
  g.slots = a.slots + static_cast<size_t>(g.group) * a.ring * k_values * members;
  g.watchdog = a.header;
  g.spin_limit = a.spin_limit;
  g.host_flag = a.host_flag;
  return g;
}

// Every thread of a workgroup that joined (split_join), once, at the end of
// the kernel, with each wave's threads converged.  Each wave counts itself
// out in LDS; the last wave of the workgroup counts the workgroup out of its
// dispenser subset, the last workgroup of a subset counts the subset out of
// the launch, and the last subset's wave stores the advanced tag sequence
// (every workgroup read the old value in split_join, before it counted
// out).  When the advance takes the sequence past plan::kSeqLimit, every
// wave first waits for its own stores (slot stores included) and the last
// one returns the whole slot area to zero before the sequence restarts: every
// other workgroup has exited by then, and the next launch starts after this
// one ends.  The counters return to zero.  Only the launch's last workgroup
// waits on anything here: two device-scope atomics.
__device__ __forceinline__ void split_leave(const SplitArgs& a) {
  if (a.grid == 0) return;
  SplitExit* ex = split_exit_lds();
  bool clear = false;
  const uint32_t next = plan::advance_seq(ex->seq, ex->stages, &clear);
  if (clear) publish_wait();  // this wave's slot stores land before the area is cleared
  const uint64_t exec = __builtin_amdgcn_read_exec();
  const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(exec >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(
                                                      static_cast<uint32_t>(exec), 0u));
  const uint32_t nwaves = (blockDim.x + kWave - 1) / kWave;
  uint32_t last = 0;
  if (rank == 0)
    last = __hip_atomic_fetch_add(&ex->waves_out, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP) == nwaves - 1;
  if (__builtin_amdgcn_readfirstlane(last) == 0) return;
  uint32_t* header = ex->header;
  uint32_t done = 0;
  if (rank == 0) {
    uint32_t* out = ex->subset_out;
    if (__hip_atomic_fetch_add(out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        ex->per_subset - 1) {
      counter_reset(out);
      uint32_t* launch_out = header + kHeaderExitWord;
      if (__hip_atomic_fetch_add(launch_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          ex->dispensers - 1) {
        counter_reset(launch_out);
        done = 1;
      }
    }
  }
  if (__builtin_amdgcn_readfirstlane(done) == 0) return;
  if (clear) {
    const uint32_t lanes = static_cast<uint32_t>(__builtin_popcountll(exec));
    u32x4* area = reinterpret_cast<u32x4*>(ex->slots);
    for (size_t i = rank; i < kSlotAreaBytes / sizeof(u32x4); i += lanes)
      area[i] = u32x4{0, 0, 0, 0};
    publish_wait();
  }
  if (rank == 0)
    __hip_atomic_store(header + kHeaderSeqWord, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One thread: publish this member's k-th partial of exchange stage `stage`.
__device__ __forceinline__ void split_publish_at(const SplitGroup& g, int stage, int k, double v) {
  const uint64_t word = (static_cast<uint64_t>(plan::stage_tag(g.epoch, stage)) << 32) |
                        __builtin_bit_cast(uint32_t, static_cast<float>(v));
  const int row = stage % g.ring;
  uint64_t* slot = g.slots + (static_cast<size_t>(row) * g.k_values + k) * g.members + g.member;
  __hip_atomic_store(slot, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 only: publish this member's k-th partial of the current stage.
__device__ __forceinline__ void split_publish(const SplitGroup& g, int k, double v) {
  split_publish_at(g, g.stage, k, v);
}

// One whole wave: wait until partials 0..values-1 of every member at
// exchange stage `stage` carry this launch's epoch.  Lane k*P + m returns
// member m's partial k as fp32 bits (0 on lanes beyond values*P).  The
// poll is bounded: on expiry it raises *watchdog and returns what it has.
__device__ __forceinline__ uint32_t split_poll(const SplitGroup& g, int stage, int values) {
  const int lane = threadIdx.x & (kWave - 1);
  const int n = g.members * values;
  const uint64_t* base = g.slots + static_cast<size_t>(stage % g.ring) * g.k_values * g.members;
  const uint32_t tag = plan::stage_tag(g.epoch, stage);
  uint64_t word = 0;
  uint32_t spins = 0;
  for (;;) {
    bool ok = true;
    if (lane < n) {
      word = __hip_atomic_load(base + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = static_cast<uint32_t>(word >> 32) == tag;
    }
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
    if (++spins > g.spin_limit) {
      if (lane == 0) {
        __hip_atomic_store(g.watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Also in host memory, so the next split call on this device reports
        // it without synchronising (api.hip, acquire_split_workspace).
        if (g.host_flag != nullptr)
          __hip_atomic_store(g.host_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return lane < n ? static_cast<uint32_t>(word) : 0u;
}

// Row tickets of a queued group pipeline travel as raw 32-bit words in
// member 0's value-k slot of the row step they name (a ticket does not fit a
// float).  One thread publishes; every member's communication wave reads the
// word back with split_poll_word.
__device__ __forceinline__ void split_publish_word(const SplitGroup& g, int stage, int k,
                                                   uint32_t bits) {
  const uint64_t word = (static_cast<uint64_t>(plan::stage_tag(g.epoch, stage)) << 32) | bits;
  uint64_t* slot = g.slots + (static_cast<size_t>(stage % g.ring) * g.k_values + k) * g.members;
  __hip_atomic_store(slot, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One whole wave: wait until member 0's value-k slot of `stage` carries the
// stage's tag and return its payload (the same in every lane).  Bounded like
// split_poll: on expiry it raises the watchdog and returns what it read.
__device__ __forceinline__ uint32_t split_poll_word(const SplitGroup& g, int stage, int k) {
  const uint64_t* slot =
      g.slots + (static_cast<size_t>(stage % g.ring) * g.k_values + k) * g.members;
  const uint32_t tag = plan::stage_tag(g.epoch, stage);
  uint32_t spins = 0;
  for (;;) {
    const uint64_t word = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(word >> 32));
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(word));
    if (hi == tag) return lo;
    if (++spins > g.spin_limit) {
      if ((threadIdx.x & (kWave - 1)) == 0) {
        __hip_atomic_store(g.watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (g.host_flag != nullptr)
          __hip_atomic_store(g.host_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      return lo;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// ---- Row-ticket queue of the group pipelines ----
// Row step i < L of group g takes the fixed row g + i G; step i >= L takes
// row first + t (first = L G), t a ticket drawn from a launch-wide counter.
// Member 0's ticket wave (queue_ticket_wave) draws step k + L's ticket once
// the communication wave has released stage k - 1 and publishes it in
// member 0's value-vk slot of stage k + L; every member's communication
// wave takes it at stage k (queue_take_row, for step k + L - 2) and hands
// the row id to its data waves through LDS before releasing the stage.  The
// first ticket naming no row ends the group's steps.  One ticket is drawn
// per row step processed, so a launch draws exactly `rows` tickets and the
// wave that draws value rows - 1 (its group's last draw) returns the counter
// to zero for the next launch.

// One whole wave (member 0's ticket wave).  n_fixed: the group's fixed
// steps (fewer than L: it has no other).  *ready: the communication wave's
// released-stage count.  Bounded like the exchange polls.
__device__ __forceinline__ void queue_ticket_wave(const SplitGroup& g, uint32_t* queue,
                                                  const uint32_t* ready, int n_fixed, int L,
                                                  int64_t first, int rows, int vk) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const buffer_rsrc_t qrs = make_rsrc(queue, 4u);  // lane 0 alone addresses it
  const uint32_t qoff = lane * 4u;
  int n = n_fixed < L ? n_fixed : INT32_MAX;  // the group's steps, once known
  for (int k = 0; k < n; ++k) {
    uint32_t spins = 0;
    while (__hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           static_cast<uint32_t>(k)) {
      if (++spins > g.spin_limit) {
        if (lane == 0) {
          __hip_atomic_store(g.watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (g.host_flag != nullptr)
            __hip_atomic_store(g.host_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    const uint32_t t = __builtin_amdgcn_readfirstlane(queue_add(qrs, qoff, 1u));
    if (first + t >= rows && n == INT32_MAX) n = k + L;
    if (lane == 0) split_publish_word(g, k + L, vk, t);
    queue_add(qrs, t == static_cast<uint32_t>(rows - 1) ? qoff : 4u,
              0u - static_cast<uint32_t>(rows));
  }
}

// One whole wave (a communication wave at stage k): the row of step
// k + L - 2, or rows when that step has none, or -1 when it is a fixed step
// (k < 2).  *n: the group's step count, INT32_MAX while open; set here at
// the first ticket that names no row.
__device__ __forceinline__ int queue_take_row(const SplitGroup& g, int k, int L, int64_t first,
                                              int rows, int vk, int* n) {
  const int j = k + L - 2;
  if (j < L) return -1;
  if (*n != INT32_MAX) return rows;
  const int64_t r = first + split_poll_word(g, j, vk);
  if (r < rows) return static_cast<int>(r);
  *n = j;
  return rows;
}

// One whole wave, after split_poll: sum of partial k over the members in
// member order (fp64), the same value in every lane.
__device__ __forceinline__ double split_wave_sum(uint32_t bits, int members, int k) {
  double s = 0.0;
  for (int m = 0; m < members; ++m)
    s += static_cast<double>(
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, k * members + m)));
  return s;
}

// LDS copy of the current stage's partials, double-buffered by stage parity
// (each exchange ends with a barrier, so no wave is two exchanges behind).
__device__ __forceinline__ float* split_lds(int stage) {
  __shared__ float xch[2][kMaxExchange];
  return xch[stage & 1];
}

// Every thread: wait for all members' partials of the current stage and
// make them readable through split_get / split_sum; advances the stage.
// `values` (default: the group's k_values) is how many partials per member
// this stage publishes: values 0..values-1.  Contains one __syncthreads.
__device__ __forceinline__ void split_exchange(SplitGroup& g, int values = 0) {
  float* xch = split_lds(g.stage);
  if (threadIdx.x < kWave) {
    const int v = values > 0 ? values : g.k_values;
    const uint32_t bits = split_poll(g, g.stage, v);
    if (static_cast<int>(threadIdx.x) < g.members * v) xch[threadIdx.x] = __builtin_bit_cast(float, bits);
  }
  __syncthreads();
  g.stage += 1;
}

// After split_exchange: member m's k-th partial of the stage just completed.
__device__ __forceinline__ double split_get(const SplitGroup& g, int k, int m) {
  return static_cast<double>(split_lds(g.stage - 1)[k * g.members + m]);
}

// Sum of the completed stage's k-th partials in member order.
__device__ __forceinline__ double split_sum(const SplitGroup& g, int k) {
  double s = 0.0;
  for (int m = 0; m < g.members; ++m) s += split_get(g, k, m);
  return s;
}

// e^x through the hardware base-2 exponential (v_exp_f32).  The product
// x*log2(e) is formed as t + e with an FMA-recovered residual (Dekker's exact
// product) plus the fp32 rounding of log2(e) itself, and the residual is
// applied as the first-order factor (1 + e*ln 2).  The relative error stays
// within a few ulp over the softmax argument range x in [-88, 0].  For
// x = +-inf the residual is not finite and exp2(t) is already exact
// (+inf, 0); NaN stays NaN.
__device__ __forceinline__ float exp_accurate(float x) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;
  constexpr float kLog2eLo = 1.925963033500011079013347625732421875e-8f;
  constexpr float kLn2 = 0.693147180559945309417232f;
  const float t = x * kLog2eHi;
  const float e = __builtin_fmaf(x, kLog2eHi, -t) + x * kLog2eLo;
  const float p = __builtin_amdgcn_exp2f(t);
  const float r = __builtin_fmaf(p * e, kLn2, p);
  return __builtin_isinf(t) ? p : r;
}

}  // namespace credit
