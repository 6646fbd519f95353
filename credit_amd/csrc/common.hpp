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

// --------------------------------------------------- memory access helpers
// Native clang vectors: the nontemporal builtins (global_load/store with the
// nt bit) accept these, not HIP's struct-wrapped float4/uint4.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 load_nt(const f32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ u32x4 load_nt(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void store_nt(f32x4* p, f32x4 v) {
  __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_nt(u32x4* p, u32x4 v) {
  __builtin_nontemporal_store(v, p);
}

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

// --------------------------------------------- split-row group barrier ----
// P workgroups ("members") that share a row form a group.  A persistent
// cooperative grid gives every group a sequence of rows; for the k-th row a
// member publishes its partial, arrives on the group's counter of parity
// k & 1, and later waits until all P members have arrived.
//
//  - Within a launch each parity counter only grows, by P per use, so the
//    k-th use of a parity completes at count == P * (uses + 1): a member can
//    only arrive at row k+2 after waiting for row k, so arrivals of
//    different rows never mix on one counter.
//  - The arrival is a returning atomic whose result is not needed until the
//    wait, so its latency overlaps whatever the member does in between.
//  - After a member's last wait, member 0 returns both counters to zero; a
//    waiter that reads a value at or below its own arrival index knows the
//    reset happened, which only follows completion.  A zero-filled counter
//    area therefore stays valid across launches of any shape.
//  - Partial slots are indexed by k % 4: a member cannot publish row k+4
//    before every member has arrived at row k+2, which each does only after
//    it has finished reading row k's slots.
//  - The two counters of a group sit in different 128-byte lines and
//    waiters poll with s_sleep backoff, so polling does not queue behind the
//    arrivals.
// Co-residency of the P members is guaranteed by the cooperative launch the
// host uses for every kernel that waits here.  The spin is still bounded: on
// expiry it raises `*watchdog` and returns, so a broken launch produces a
// reported error instead of a hung GPU.
constexpr int kGroupCounterStride = 64;  // uint32 slots per group (2 x 128 B)
constexpr int kMaxGroups = 16384 / kGroupCounterStride;
constexpr uint32_t kSpinLimit = 1u << 21;  // several seconds of s_sleep spins

struct GroupSync {
  uint32_t* count0;  // parity-0 counter
  uint32_t* count1;  // parity-1 counter (different cache line)
  uint32_t members;
  uint32_t uses[2];
  uint32_t old[2];
};

__device__ __forceinline__ GroupSync group_sync_init(uint32_t* counter_area, int group,
                                                     int members) {
  GroupSync s;
  s.count0 = counter_area + group * kGroupCounterStride;
  s.count1 = s.count0 + kGroupCounterStride / 2;
  s.members = static_cast<uint32_t>(members);
  s.uses[0] = s.uses[1] = 0;
  s.old[0] = s.old[1] = 0;
  return s;
}

// Called by every thread after this member's partial stores; only thread 0
// touches the counter.
__device__ __forceinline__ void group_arrive(GroupSync& s, int k) {
  publish_wait();
  __syncthreads();
  if (threadIdx.x == 0) s.old[k & 1] = arrive((k & 1) ? s.count1 : s.count0);
}

__device__ __forceinline__ void group_wait(GroupSync& s, int k, uint32_t* watchdog) {
  const int p = k & 1;
  if (threadIdx.x == 0) {
    const uint32_t target = s.members * (s.uses[p] + 1);
    const uint32_t mine = s.old[p];
    const uint32_t* c = p ? s.count1 : s.count0;
    uint32_t spins = 0;
    for (;;) {
      const uint32_t v = counter_read(c);
      if (v >= target || v <= mine) break;
      __builtin_amdgcn_s_sleep(2);
      if (++spins > kSpinLimit) {
        __hip_atomic_store(watchdog, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  s.uses[p] += 1;
  __syncthreads();
}

// After the member's last wait: member 0 returns the counters to zero.
__device__ __forceinline__ void group_finish(GroupSync& s, int member) {
  if (member == 0 && threadIdx.x == 0) {
    counter_reset(s.count0);
    counter_reset(s.count1);
  }
}

// Block -> (group, member) for a persistent split grid of groups x members
// workgroups.  Workgroups are dispatched to the 8 XCDs round-robin, so
// ids congruent mod 8 share an XCD: member m of group g is workgroup
// (g / 8) * 8 * members + m * 8 + g % 8 whenever the group count is a
// multiple of 8, and the group's exchange then stays on one XCD.
__device__ __forceinline__ void split_coords(int members, int groups, int* group, int* member) {
  const int b = blockIdx.x;
  if ((groups & 7) == 0) {
    const int tile = b / (8 * members);
    const int within = b - tile * 8 * members;
    *group = tile * 8 + (within & 7);
    *member = within >> 3;
  } else {
    *group = b / members;
    *member = b - *group * members;
  }
}

// e^x through the hardware base-2 exponential (v_exp_f32).  The product
// x*log2(e) is formed as t + e with an FMA-recovered residual (Dekker's exact
// product) plus the fp32 rounding of log2(e) itself, and the residual is
// applied as the first-order factor (1 + e*ln 2).  The relative error stays
// within a few ulp over the softmax argument range x in [-88, 0].
__device__ __forceinline__ float exp_accurate(float x) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;
  constexpr float kLog2eLo = 1.925963033500011079013347625732421875e-8f;
  constexpr float kLn2 = 0.693147180559945309417232f;
  const float t = x * kLog2eHi;
  const float e = __builtin_fmaf(x, kLog2eHi, -t) + x * kLog2eLo;
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p * e, kLn2, p);
}

}  // namespace credit
