// C5: norm-fused FFN on MFMA, bf16 with fp32 accumulation.
//
//   rstd = 1/sqrt(mean_j x^2 + eps)                          (unit RMSNorm weight)
//   h    = bf16(GELU_tanh(rstd * (x @ W1^T)))   256-tile kernel (the C5 path)
//   h    = bf16(GELU_tanh(bf16(x * rstd) @ W1^T))   128-tile kernel
//   out  = bf16(x + h @ W2^T)
//
// The 256-tile kernel multiplies the fp32 accumulator of x @ W1^T by the
// row's rstd in its epilogue (the row scale commutes with the GEMM), so the
// normalised input is never rounded; the 128-tile kernel scales and rounds
// the A tile to bf16 as it stages it.  Both are the same function up to that
// rounding (the oracle's round_a switch selects either).
//
// No FFN exists in the reference; this is the consumer of the row-norm
// kernels the BASELINE names.  Weights come in the nn.Linear layout
// ([out_features, in_features], K contiguous): W1 [f, d], W2 [d, f], so
// both GEMMs are "A row-major x B K-contiguous" and every MFMA operand
// fragment (8 consecutive k per lane) is one 16-byte LDS read.
// credit_transpose_bf16 converts a [d, f] weight once.
//
// Kernels:
//  1. ffn_rstd_kernel: rstd per row of x (one read of x, 64 MiB at C5).
//  2. GEMM1 with epilogue kEpiGelu: h = bf16(GELU_tanh(acc * rstd[m])); the
//     RMSNorm commutes with the GEMM and is applied as a row scale.
//  3. GEMM2 with epilogue kEpiResidual: out = bf16(acc + x).
// Each GEMM runs on ffn_gemm256_kernel (256 x 256 x 64 tiles, four waves,
// LDS-direct operand loads; the C5 path) when the shape allows, else on
// ffn_gemm_kernel (128 x 128 x 64 tiles, operands prefetched through
// registers one K-step ahead, the A tile scaled by rstd and rounded to bf16
// while it is staged into LDS).  The backward (credit_ffn_rmsnorm_gelu_bwd_bf16)
// runs five GEMMs on the same two kernels with its own epilogues.
#include <atomic>
#include <initializer_list>
#include <type_traits>
#include <utility>

#include "api_internal.hpp"
#include "common.hpp"

namespace credit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kLdsStride = kBK + 8;  // bf16 per LDS row: 16-byte pad against bank conflicts

// GEMM epilogues.  Forward: kEpiGelu (h = GELU(acc * rstd[m])),
// kEpiResidual (out = acc + x); the training forward's kEpiGeluSave (h =
// GELU(u) to C and u = acc * rstd[m] to C2, both row-major).  Backward
// (credit_ffn_rmsnorm_gelu_bwd_bf16): kEpiUH (u = acc * rstd[m] to C, h =
// GELU(u) transposed to C2), kEpiGeluBwd (du = acc * GELU'(u[m, n]) to C
// and, transposed, to C2), kEpiStore (bf16(acc)), kEpiStoreF32 (acc as fp32
// to Cf).
constexpr int kEpiGelu = 0;
constexpr int kEpiResidual = 1;
constexpr int kEpiUH = 2;
constexpr int kEpiGeluBwd = 3;
constexpr int kEpiStore = 4;
constexpr int kEpiStoreF32 = 5;
constexpr int kEpiGeluSave = 6;
constexpr int kEpiStoreT = 7;  // C^T [N, M] = bf16(acc): the output stored transposed

// GELU with the tanh approximation, z = sqrt(2/pi) (v + 0.044715 v^3):
// 0.5 (1 + tanh z) = sigmoid(2z), so GELU(v) = v / (1 + e') with
// e' = e^(-2z) = 2^(v t), t = -2 sqrt(2/pi) log2(e) (1 + 0.044715 v^2): one
// hardware exp2 and one hardware reciprocal (about 1 ulp each), no
// cancellation on either side.  On the negative tail e' is large and 1/(1 +
// e') keeps its relative accuracy until e' overflows (v below about -10.5,
// GELU below 4e-38 in magnitude), where rcp(inf) = 0 gives -0; on the
// positive side e' -> 0 and GELU -> v, +inf giving +inf.
constexpr float kGeluC = 0.7978845608028654f;   // sqrt(2/pi)
constexpr float kGeluC2 = 2.302208198144325f;   // 2 sqrt(2/pi) log2(e)
constexpr float kGeluA = 0.044715f;

__device__ __forceinline__ float gelu_tanh(float v) {
  const float t = __builtin_fmaf(-kGeluC2 * kGeluA, v * v, -kGeluC2);
  return v * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(v * t) + 1.0f);
}

// GELU' needs both s = sigmoid(2z) and r = 1 - s = sigmoid(-2z): with e =
// e^(2z) = 2^(arg), r = 1 / (e + 1) and s = e r, neither cancelling.  The
// exponent is capped at 64 (v above about 6.6), so e stays finite, s rounds
// to 1 and r to 2^-64.
struct GeluParts {
  float r;  // 1 / (e + 1) = 1 - s
  float s;  // sigmoid(2z) = 0.5 (1 + tanh z)
};

__device__ __forceinline__ GeluParts gelu_parts(float v, float v2) {
  const float arg = kGeluC2 * v * __builtin_fmaf(kGeluA, v2, 1.0f);
  const float e = __builtin_amdgcn_exp2f(arg < 64.0f ? arg : 64.0f);
  GeluParts g;
  g.r = __builtin_amdgcn_rcpf(e + 1.0f);
  g.s = e * g.r;
  return g;
}

// d/dv GELU = s + 2 v r s dz/dv, dz/dv = sqrt(2/pi) (1 + 3 * 0.044715 v^2).
__device__ __forceinline__ float gelu_tanh_grad(float v) {
  const float v2 = v * v;
  const GeluParts g = gelu_parts(v, v2);
  return __builtin_fmaf(2.0f * kGeluC * v * g.r * g.s, __builtin_fmaf(3.0f * kGeluA, v2, 1.0f),
                        g.s);
}

// One output element of every epilogue.  s is the row scale still to apply
// (rstd[m] for the 256-tile kernel, 1 where the A tile was scaled on load);
// rv is R[m, n] widened to fp32 for kEpiResidual and kEpiGeluBwd (unused
// otherwise).
template <int EPI>
__device__ __forceinline__ void epilogue(float acc, float s, float rv, int m, int n, int M, int N,
                                         uint16_t* __restrict__ C, uint16_t* __restrict__ C2,
                                         float* __restrict__ Cf) {
  const size_t idx = static_cast<size_t>(m) * N + n;
  const size_t tdx = static_cast<size_t>(n) * M + m;
  if (EPI == kEpiGelu) {
    C[idx] = f32_to_bf16(gelu_tanh(acc * s));
  } else if (EPI == kEpiGeluSave) {
    // The same h as kEpiGelu, and the u the backward's kEpiUH recomputes.
    const float u = acc * s;
    C[idx] = f32_to_bf16(gelu_tanh(u));
    C2[idx] = f32_to_bf16(u);
  } else if (EPI == kEpiResidual) {
    C[idx] = f32_to_bf16(acc + rv);
  } else if (EPI == kEpiUH) {
    const float u = acc * s;
    C[idx] = f32_to_bf16(u);
    C2[tdx] = f32_to_bf16(gelu_tanh(u));
  } else if (EPI == kEpiGeluBwd) {
    const uint16_t v = f32_to_bf16(acc * gelu_tanh_grad(rv));
    C[idx] = v;
    if (C2 != nullptr) C2[tdx] = v;
  } else if (EPI == kEpiStoreT) {
    C[tdx] = f32_to_bf16(acc);
  } else if (EPI == kEpiStore) {
    C[idx] = f32_to_bf16(acc);
  } else {
    Cf[idx] = acc;
  }
}

// Epilogues that read a second [M, N] operand.
template <int EPI>
constexpr bool kEpiReadsR = EPI == kEpiResidual || EPI == kEpiGeluBwd;

__device__ __forceinline__ u32x4 scale_bf16x8(u32x4 v, float s) {
  return u32x4{pack_bf16x2(bf16_lo(v.x) * s, bf16_hi(v.x) * s),
               pack_bf16x2(bf16_lo(v.y) * s, bf16_hi(v.y) * s),
               pack_bf16x2(bf16_lo(v.z) * s, bf16_hi(v.z) * s),
               pack_bf16x2(bf16_lo(v.w) * s, bf16_hi(v.w) * s)};
}

// rstd[m] = 1/sqrt(mean(x[m]^2) + eps); cols % 8 == 0, rows 16-byte aligned.
__global__ __launch_bounds__(256) void ffn_rstd_kernel(const uint16_t* __restrict__ x,
                                                       float* __restrict__ rstd, int cols,
                                                       float eps) {
  __shared__ double red[4];
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + static_cast<size_t>(blockIdx.x) * cols);
  const int nvec = cols >> 3;
  float s = 0.0f;
  for (int i = threadIdx.x; i < nvec; i += 256) {
    const u32x4 v = xr[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = bf16_lo(v[e]), hi = bf16_hi(v[e]);
      s += lo * lo + hi * hi;
    }
  }
  const double t = block_reduce_sum_f64<4>(static_cast<double>(s), red);
  if (threadIdx.x == 0) rstd[blockIdx.x] = static_cast<float>(1.0 / __builtin_sqrt(t / cols + eps));
}

// C[m, n] = epi(sum_k A[m, k] * B[n, k]).  A [M, K] and B [N, K] row-major
// bf16 (KN: B [K, N], element (n, k) at B[k * N + n]); M % 128 == 0,
// N % 128 == 0, K % 64 == 0 (checked on the host).
//  kEpiGelu:     A rows scaled by a_scale[m] on load; C = bf16(gelu(acc)).
//  kEpiGeluSave: likewise, and C2 = bf16(acc) (u).
//  kEpiResidual: C = bf16(acc + R[m, n]).
// KN: thread t stages 16-byte chunk t % 16 (8 columns) of K-rows t / 16 +
// 16 i of the 64 x 128 B tile and scatters its 8 values into the [n][k]
// LDS tile (2-byte stores; this kernel only serves shapes the 256-tile
// kernel does not take).
template <int EPI, bool KN>
__global__ __launch_bounds__(kThreads) void ffn_gemm_kernel(
    const uint16_t* __restrict__ A, const float* __restrict__ a_scale,
    const uint16_t* __restrict__ B, const uint16_t* __restrict__ R, uint16_t* __restrict__ C,
    uint16_t* __restrict__ C2, float* __restrict__ Cf, int M, int N, int K) {
  constexpr bool kScaleA = EPI == kEpiGelu || EPI == kEpiUH || EPI == kEpiGeluSave;
  __shared__ __attribute__((aligned(16))) uint16_t As[kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN * kLdsStride];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // Tile order: consecutive workgroups walk down M for a fixed N strip, so
  // the B strip (the weight tile) is reused from L2 by neighbours.
  const int tiles_m = M / kBM;
  const int tm = blockIdx.x % tiles_m;
  const int tn = blockIdx.x / tiles_m;
  const int m0 = tm * kBM, n0 = tn * kBN;

  // Global -> register staging: thread t moves rows t/8 + 32*i, 16-byte
  // chunk t%8 of the 128-byte K-row, for i = 0..3 (A and B alike).
  const int ld_row = tid >> 3;
  const int ld_chunk = tid & 7;
  const u32x4* a_src[4];
  const u32x4* b_src[4];
  float scale[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = ld_row + 32 * i;
    a_src[i] = reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m0 + r) * K) + ld_chunk;
    b_src[i] = KN ? reinterpret_cast<const u32x4*>(B + static_cast<size_t>((tid >> 4) + 16 * i) * N +
                                                   n0) + (tid & 15)
                  : reinterpret_cast<const u32x4*>(B + static_cast<size_t>(n0 + r) * K) + ld_chunk;
    scale[i] = kScaleA ? a_scale[m0 + r] : 1.0f;
  }
  const size_t b_step = KN ? static_cast<size_t>(kBK) * N / 8 : kBK / 8;  // u32x4 per K-step
  u32x4 ra[4], rb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ra[i] = a_src[i][0];
    rb[i] = b_src[i][0];
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ksteps = K / kBK;
  for (int ks = 0; ks < ksteps; ++ks) {
    __syncthreads();  // previous step's fragment reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = ld_row + 32 * i;
      const u32x4 av = kScaleA ? scale_bf16x8(ra[i], scale[i]) : ra[i];
      *reinterpret_cast<u32x4*>(&As[r * kLdsStride + ld_chunk * 8]) = av;
      if constexpr (KN) {
        const int kr = (tid >> 4) + 16 * i, n8 = (tid & 15) * 8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Bs[(n8 + 2 * e) * kLdsStride + kr] = static_cast<uint16_t>(rb[i][e] & 0xffffu);
          Bs[(n8 + 2 * e + 1) * kLdsStride + kr] = static_cast<uint16_t>(rb[i][e] >> 16);
        }
      } else {
        *reinterpret_cast<u32x4*>(&Bs[r * kLdsStride + ld_chunk * 8]) = rb[i];
      }
    }
    __syncthreads();
    if (ks + 1 < ksteps) {  // prefetch the next K-step into registers
      const int off = (ks + 1) * (kBK / 8);
      const size_t boff = (ks + 1) * b_step;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ra[i] = a_src[i][off];
        rb[i] = b_src[i][boff];
      }
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int kcol = kk * 16 + (lane >> 5) * 8;
      bf16x8_t af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const bf16x8_t*>(&As[r * kLdsStride + kcol]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = wn * 64 + j * 32 + (lane & 31);
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[c * kLdsStride + kcol]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue.  Accumulator register r of lane l holds row
  // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of the 32 x 32 tile.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        const float rv = kEpiReadsR<EPI> ? bf16_to_f32(R[static_cast<size_t>(m) * N + n]) : 0.0f;
        epilogue<EPI>(acc[i][j][r], 1.0f, rv, m, n, M, N, C, C2, Cf);
      }
}

// ----------------------------------------------------- 256 x 256 tiles ---
// The main GEMM: C[m, n] = epi(sum_k A[m, k] * B[n, k]) with 256 x 256 x 64
// tiles per 256-lane workgroup: four waves, one per SIMD.  Wave (wm, wn) of
// the 2 x 2 wave grid owns a 128 x 128 block as 4 x 4
// v_mfma_f32_32x32x16_bf16 tiles (256 fp32 accumulators per lane, held in
// AGPRs).  Measured on the C5 shapes against the eight-wave 256 x 256 x 32
// form with global_load_lds it replaces: +13-17% (1.07 -> 1.23-1.27
// PFLOP/s on GEMM1, bit-identical results); the gain is the K depth of 64
// (every 8 lanes of a load read one whole 128-byte line) and the buffer form
// of the LDS-direct load.
//  - Operand tiles go from global memory straight to LDS with
//    buffer_load_dwordx4 ... lds: a wave instruction writes 1 KiB of LDS
//    (lane l at M0 + 16 l), i.e. 8 rows of 128 bytes.  An operand tile
//    (256 rows x 64 K) is 32 KiB; A has two stages and B three, 160 KiB.
//  - The loads are issued from inline assembly.  The compiler's waitcnt
//    pass cannot tell an LDS-direct load's destination from the fragment
//    reads of the other stage and would wait for every load before every
//    read; here the only waits on the loads are the explicit ones below,
//    which count them (no other vector-memory instruction is in flight in
//    the K loop).
//  - K-step k (64 wide) reads A stage k & 1 and B stage k % 3.  Iteration
//    it runs four sub-steps of 16 MFMAs (k = 16 each), reading the next
//    sub-step's 8 fragments while the current MFMAs issue (interleaving
//    pinned with sched_group_barrier / sched_barrier).  The barrier sits
//    before the last sub-step: own loads of step it+1 landed, then
//    s_barrier publishes step it+1's stages to every wave and proves every
//    wave has read its last fragments of step it.  The last sub-step then
//    reads the first fragments of step it+1.
//  - Loads of step it+2: B (8 per lane) in sub-steps 0-2 of iteration it,
//    3 + 3 + 2 -- its stage (it+2) % 3 was last read in step it-1, before
//    the previous barrier; A (8) in sub-step 3, after the barrier, into A
//    stage it & 1.  Every load thus has at least three sub-steps to land
//    before the wait for it, vmcnt(8) (step it+2's B loads stay in flight).
//    Against two 64 KiB stages, where the last loads of a step had one
//    sub-step: +5.6% on the C5 forward (1291 -> 1363 TFLOP/s, bit-identical
//    outputs).  B's loads spread 2/3/3: the same; 4/4/0 -1%, 0/4/4 -1%,
//    all 8 in sub-step 0: -5%.  Tail steps re-load the last K-step into
//    stages nobody reads again, so the loop body has fixed wait counts.
//  - The barrier is a bare s_barrier after s_waitcnt lgkmcnt(0): a
//    workgroup-scope release fence would also drain the loads in flight.
//  - LDS rows are 128 bytes (64 bf16 of K); 16-byte chunk c of row r sits
//    at position c ^ ((r >> 1) & 7): the 16 lanes of one fragment read
//    (rows r..r+15, one chunk) and of one load's LDS write (rows r, r+1,
//    eight chunks each) hit 16 distinct 4-bank groups.  A load lane picks
//    its global chunk so that it lands at its fixed LDS position.
//   kEpiGelu:     C = bf16(GELU(acc * scale[m]))   (RMSNorm folded in: the
//                 row scale commutes with the GEMM)
//   kEpiResidual: C = bf16(acc + R[m, n])
constexpr int kBig = 256;
constexpr int kBigK = 64;
constexpr int kBigTile = kBig * kBigK * 2;   // one operand tile of a stage, bytes (32 KiB)
constexpr int kBigBRing = 3;                 // B stages (A has two)
constexpr int kBigBBase = 2 * kBigTile;      // B ring after the two A stages
constexpr int kBigLds = (2 + kBigBRing) * kBigTile;  // 160 KiB
// Tile blocks within an XCD: 8 M-tiles x 4 N-tiles run concurrently and
// share their A rows and B columns through that XCD's L2.
constexpr int kGroupM = 8;
constexpr int kBigThreads = 256;

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in
// bits 15:14; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt(((N >> 4) << 14) | (0xF << 8) | (0x7 << 4) | (N & 15));
}

// Workgroup barrier for LDS only: this wave's LDS operations complete
// (lgkmcnt(0)), then s_barrier; signal fences keep the compiler from moving
// memory operations across it.  Vector-memory loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// One LDS-direct load: 16 bytes per lane from rsrc at voff + soff into LDS
// at M0 = m0base + QOFF + 16 * lane.  s_nop covers the M0 write -> LDS-DMA
// hazard.  M0 is a reserved register to the compiler, which warns that it
// does not restore a clobbered M0; nothing else in these kernels reads M0
// (no LDS-direct builtins, GWS, s_sendmsg or indexed register moves), so a
// value left by one load is only ever overwritten by the next.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <uint32_t QOFF>
__device__ __forceinline__ void load_to_lds(buffer_rsrc_t rsrc, uint32_t voff, uint32_t m0base,
                                            uint32_t soff) {
  asm volatile(
      "s_add_u32 m0, %2, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, %4 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(m0base), "i"(QOFF), "s"(soff)
      : "memory", "m0", "scc");
}
#pragma clang diagnostic pop

// sched_group_barrier masks.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// ds_read_b64_tr_b16 at the LDS location of p (a pointer into smem).
__device__ __forceinline__ bf16x4_t ds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      reinterpret_cast<lds_bf16x4_t*>((lds_ptr_t)(const_cast<char*>(p))));
}

// Loads per thread per K-step: 16 (8 of A, 8 of B).  Load q of wave w fills
// rows 8 b .. 8 b + 7 of operand q >> 3, b = (q & 7) * 4 + w.
//
// KN: B is stored [K, N] (N contiguous: the [in, out] weight layout, W1
// [d, f] and W2 [f, d]) instead of [N, K].  Its stage is then 64 K-rows of
// 512 bytes (256 columns); load q >= 8 of wave w fills K-rows 8 (q & 7) + 2 w
// and + 1 (one 1 KiB wave instruction), lane l writing 16-byte chunk l % 32
// of row 2 w + l / 32.  Chunk c of K-row r sits at position c ^ 4 (r & 3).
// A B fragment (8 consecutive k of one column per lane) is then gathered by
// two ds_read_b64_tr_b16: within each 16-lane group, result lane 4 a + b
// takes 16-bit word b of the 8-byte pieces addressed by group lanes a,
// a + 4, a + 8, a + 12.  Group lane j addresses K-row k0 + j / 4 and
// columns c0 + 4 (j % 4) .. + 3, so lane j receives column c0 + j at
// K-rows k0 .. k0 + 3 -- the MFMA B operand's layout.  The 32 lanes of one
// half-wave read 4 K-rows x 64 bytes, which the swizzle spreads over all
// 64 banks.

// Clock probe (credit_set_clock_probe): with a non-null `probe`, thread 0 of
// every workgroup adds the shader cycles (s_memtime) and the 100 MHz
// constant-clock ticks (s_memrealtime) between the workgroup's start and its
// end to probe[0] and probe[1] (the start stamps subtracted as it starts, so
// nothing stays live across the kernel); their ratio is the mean shader clock
// the tiles ran at.
__device__ __forceinline__ void clock_probe_add(uint64_t* probe, bool start) {
  if (probe == nullptr || threadIdx.x != 0) return;
  const uint64_t c = __builtin_amdgcn_s_memtime();
  const uint64_t r = __builtin_amdgcn_s_memrealtime();
  __hip_atomic_fetch_add(probe, start ? 0 - c : c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(probe + 1, start ? 0 - r : r, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}

template <int EPI, bool KN>
__global__ __launch_bounds__(kBigThreads) void ffn_gemm256_kernel(
    const uint16_t* __restrict__ A, const float* __restrict__ scale,
    const uint16_t* __restrict__ B, const uint16_t* __restrict__ R, uint16_t* __restrict__ C,
    uint16_t* __restrict__ C2, float* __restrict__ Cf, int M, int N, int K,
    uint64_t* __restrict__ probe) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  clock_probe_add(probe, true);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // 2 x 2 waves, 128 x 128 each

  // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin,
  // so XCD x runs ids x, x + 8, ...; give each XCD a contiguous run of the
  // tile sequence, and walk that run in blocks of kGroupM M-tiles (8 M-tiles
  // x 4 N-tiles run at once per XCD and share A rows and B columns in its L2).
  const int tiles_m = M / kBig, tiles_n = N / kBig;
  const int total = tiles_m * tiles_n;
  const int per_xcd = total / 8;  // host guarantees total % 8 == 0
  const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  const int group = t / (kGroupM * tiles_n);
  const int gm = tiles_m - group * kGroupM < kGroupM ? tiles_m - group * kGroupM : kGroupM;
  const int within = t - group * kGroupM * tiles_n;
  const int tm = group * kGroupM + within % gm;
  const int tn = within / gm;
  const int m0 = tm * kBig, n0 = tn * kBig;
  const int iters = K / kBigK;  // host guarantees an even count >= 2

  // Load addressing.  Lane l of load q reads row 8 b + l / 8 (b as above)
  // and writes LDS chunk l % 8 of it, so it loads logical chunk
  // (l % 8) ^ ((row >> 1) & 7) = (l % 8) ^ ((w & 1) * 4 + l / 16).  The
  // lane-dependent part of the byte offset is one VGPR; row block (q & 7)
  // * 32 rows and the K step go into the scalar offset.
  const buffer_rsrc_t rsrc_a = make_rsrc(A + static_cast<size_t>(m0) * K, 256u * K * 2u);
  // KN: columns n0 .. n0 + 255 of K rows of pitch N (the host keeps K N 2
  // within 32 bits).
  const buffer_rsrc_t rsrc_b =
      KN ? make_rsrc(B + n0, static_cast<uint32_t>((static_cast<size_t>(K - 1) * N + 256) * 2))
         : make_rsrc(B + static_cast<size_t>(n0) * K, 256u * K * 2u);
  const int chunk = (lane & 7) ^ (((wave & 1) << 2) + (lane >> 4));
  const uint32_t voff = static_cast<uint32_t>(((wave * 8 + (lane >> 3)) * K + chunk * 8) * 2);
  const int kn_row = 2 * wave + (lane >> 5);  // K-row of the stage mod 8 (KN loads)
  const uint32_t voff_kn = static_cast<uint32_t>(
      (kn_row * N + (((lane & 31) ^ ((kn_row & 3) << 2)) * 8)) * 2);
  // LDS byte address of smem (an address-space cast; C++ casts do not express it).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
  const uint32_t m0_wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
      static_cast<int>(lds0 + wave * 1024)));
  auto load = [&](int k, auto qc) {
    constexpr int q = decltype(qc)::value;
    constexpr uint32_t qoff = static_cast<uint32_t>((q & 7) * 4096);
    const int kc = k < iters ? k : iters - 1;  // tail: a harmless re-load
    const int stage_off = q < 8 ? (k & 1) * kBigTile : kBigBBase + (k % kBigBRing) * kBigTile;
    const uint32_t base = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(m0_wave + stage_off)));
    const uint32_t soff_nk = static_cast<uint32_t>(kc * kBigK * 2 + (q & 7) * 64 * K);
    const uint32_t soff_kn =
        (static_cast<uint32_t>(kc * kBigK + (q & 7) * 8) * static_cast<uint32_t>(N)) * 2u;
    const uint32_t soff = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>(KN && q >= 8 ? soff_kn : soff_nk)));
    if constexpr (q < 8)
      load_to_lds<qoff>(rsrc_a, voff, base, soff);
    else
      load_to_lds<qoff>(rsrc_b, KN ? voff_kn : voff, base, soff);
  };

  // Fragment reads: A rows wm*128 + i*32 + (l & 31), B rows wn*128 + j*32 +
  // (l & 31); K sub-step kk covers logical chunks 2 kk and 2 kk + 1 (lanes
  // 0-31 and 32-63).
  const int fsw = ((lane & 31) >> 1) & 7;
  const int a_frag = (wm * 128 + (lane & 31)) * 128;
  const int b_frag = (wn * 128 + (lane & 31)) * 128;
  // KN fragment j of sub-step kk: group lane j' = l % 16 of group g = (l / 16)
  // % 4 addresses K-row 16 kk + 8 (g / 2) + s (s = j' / 4; + 4 for the
  // second read) and logical chunk 16 wn + 4 j + 2 (g & 1) + (j' / 2) % 2,
  // byte 8 (j' % 2) of it, which sits at position 16 wn + 4 (j ^ s) + ...
  const int kn_g = (lane >> 4) & 3, kn_s = (lane & 15) >> 2;
  const int kn_lane = (8 * (kn_g >> 1) + kn_s) * 512 +
                      (wn * 16 + 2 * (kn_g & 1) + ((lane >> 1) & 1)) * 16 + 8 * (lane & 1);
  struct Frags { bf16x8_t a[4], b[4]; };
  // step: the K-step whose stages are read (A stage step & 1, B stage step % 3).
  auto frag = [&](int step, int kk, int idx) {
    const int c = ((2 * kk + (lane >> 5)) ^ fsw) << 4;
    const char* abase = smem + (step & 1) * kBigTile;
    const char* bbase = smem + kBigBBase + __builtin_amdgcn_readfirstlane(step % kBigBRing) * kBigTile;
    if (KN && idx >= 4) {
      const char* p = bbase + kn_lane + (((idx - 4) ^ kn_s) << 6) + kk * 8192;
      return __builtin_shufflevector(ds_read_tr16(p), ds_read_tr16(p + 2048), 0, 1, 2, 3, 4, 5,
                                     6, 7);
    }
    return idx < 4 ? *reinterpret_cast<const bf16x8_t*>(abase + a_frag + idx * 4096 + c)
                   : *reinterpret_cast<const bf16x8_t*>(bbase + b_frag + (idx - 4) * 4096 + c);
  };
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // MFMA Mi of a sub-step: fragment read Mi of the next sub-step first (Mi < 8).
  auto mfma = [&]<int Mi>(const Frags& cur, Frags& nxt, int ns, int nkk) {
    if constexpr (Mi < 8) {
      const bf16x8_t v = frag(ns, nkk, Mi);
      if constexpr (Mi < 4)
        nxt.a[Mi] = v;
      else
        nxt.b[Mi - 4] = v;
    }
    acc[Mi >> 2][Mi & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        cur.a[Mi >> 2], cur.b[Mi & 3], acc[Mi >> 2][Mi & 3], 0, 0, 0);
  };
  // A sub-step is four quarters of four MFMAs; load Q0 + j (of step lk)
  // follows quarter j.  Each quarter is a scheduling region of its own (the
  // MFMAs would otherwise drift past the inline-assembly loads and leave
  // them in bursts), with its fragment reads pinned one per MFMA.
  auto sub_step = [&]<int Q0>(const Frags& cur, Frags& nxt, int ns, int nkk, int lk) {
    [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
      (
          [&] {
            constexpr int Qi = Qs;
            [&]<int... Js>(std::integer_sequence<int, Js...>) {
              (mfma.template operator()<4 * Qi + Js>(cur, nxt, ns, nkk), ...);
            }(std::make_integer_sequence<int, 4>{});
            load(lk, std::integral_constant<int, Q0 + Qi>{});
            [&]<int... Js>(std::integer_sequence<int, Js...>) {
              (
                  [&] {
                    constexpr int Mi = 4 * Qi + Js;
                    if constexpr (Mi < 8)  // a KN B fragment is two reads
                      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, KN && Mi >= 4 ? 2 : 1, 0);
                    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                  }(),
                  ...);
            }(std::make_integer_sequence<int, 4>{});
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, 4>{});
  };

  // Prologue: step 0 whole, then B of step 1 and the first half of its A.
  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (load(0, std::integral_constant<int, Qs>{}), ...);
  }(std::make_integer_sequence<int, 16>{});
  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (load(1, std::integral_constant<int, 8 + Qs>{}), ...);
  }(std::make_integer_sequence<int, 8>{});
  [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
    (load(1, std::integral_constant<int, Qs>{}), ...);
  }(std::make_integer_sequence<int, 4>{});
  wait_vmcnt<12>();  // own loads of step 0 landed
  lds_barrier();
  Frags f0, f1;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const bf16x8_t v = frag(0, 0, m);
    if (m < 4)
      f0.a[m] = v;
    else
      f0.b[m - 4] = v;
  }
  // Iteration it computes step it, four loads per sub-step.  Sub-step 0
  // issues the second half of A of step it+1 (its stage (it+1) & 1 was last
  // read in step it-1, before the previous barrier), sub-steps 1-2 B of step
  // it+2 (stage (it+2) % 3, last read in step it-1), and after this
  // iteration's barrier sub-step 3 the first half of A of step it+2 into A
  // stage it & 1, whose reads all precede the barrier.  The wait before the
  // barrier leaves B of step it+2 (8 loads) in flight.
  auto iteration = [&](int it) {
    sub_step.template operator()<4>(f0, f1, it, 1, it + 1);
    sub_step.template operator()<8>(f1, f0, it, 2, it + 2);
    sub_step.template operator()<12>(f0, f1, it, 3, it + 2);
    wait_vmcnt<8>();  // own loads of step it+1 landed
    lds_barrier();
    sub_step.template operator()<0>(f1, f0, it + 1, 0, it + 2);
  };
  for (int it = 0; it < iters; ++it) iteration(it);
  wait_vmcnt<0>();  // the tail re-loads

  // R tile (256 x 256 bf16 = 128 KiB, the whole LDS) for the epilogues that
  // read it: LDS-direct loads, 2 rows of 512 bytes per wave instruction
  // (wave w fills rows 64 w .. 64 w + 63), so the epilogue's per-element
  // reads come from LDS instead of 256 scattered 2-byte global loads per
  // lane.
  const uint16_t* r_tile = reinterpret_cast<const uint16_t*>(smem);
  if constexpr (kEpiReadsR<EPI>) {
    lds_barrier();  // every wave has read its last fragments
    const buffer_rsrc_t rsrc_r = make_rsrc(R + static_cast<size_t>(m0) * N + n0,
                                           static_cast<uint32_t>((255u * N + 256u) * 2u));
    const uint32_t voff_r = static_cast<uint32_t>(((lane >> 5) * N + (lane & 31) * 8) * 2);
    const uint32_t m0_r = static_cast<uint32_t>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(lds0 + wave * 32768)));
    [&]<int... Is>(std::integer_sequence<int, Is...>) {
      (load_to_lds<static_cast<uint32_t>(Is * 1024)>(
           rsrc_r, voff_r, m0_r,
           static_cast<uint32_t>(__builtin_amdgcn_readfirstlane((64 * wave + 2 * Is) * N * 2))),
       ...);
    }(std::make_integer_sequence<int, 32>{});
    wait_vmcnt<0>();
    lds_barrier();
  }
  // R at rows mb .. mb + 3 (mb = the row of accumulator register 4q of tile
  // (i, j)) and the lane's column, by one ds_read_b64_tr_b16: group lane k
  // of each 16-lane group addresses tile row mb + k / 4, columns c0 + 4 (k %
  // 4) .. + 3, so result lane k receives column c0 + k of the four rows --
  // the layout of accumulator registers 4q .. 4q + 3.
  auto r_quad = [&](int i, int j, int q) {
    const int g = lane >> 4, k = lane & 15;
    const int row = wm * 128 + i * 32 + 8 * q + 4 * (g >> 1) + (k >> 2);
    const int col = wn * 128 + j * 32 + 16 * (g & 1) + 4 * (k & 3);
    return ds_read_tr16(reinterpret_cast<const char*>(r_tile) + row * (kBig * 2) + col * 2);
  };

  // Epilogue.  Accumulator register r of lane l holds row
  // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of its 32 x 32 tile.
  if constexpr (EPI == kEpiUH || EPI == kEpiGeluBwd || EPI == kEpiStoreT) {
    // Also (kEpiStoreT: only) stored transposed: registers 4q..4q+3 are four
    // consecutive rows of one column, so each lane writes them as one 8-byte
    // run of C2 (kEpiStoreT: of C).  kEpiGeluBwd with C2 == nullptr skips
    // the transposed copy.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int mb = m0 + wm * 128 + i * 32 + 8 * q + 4 * (lane >> 5);
          const int n = n0 + wn * 128 + j * 32 + (lane & 31);
          uint32_t t[2];
          bf16x4_t rq;
          if constexpr (EPI == kEpiGeluBwd) rq = r_quad(i, j, q);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = mb + e;
            const size_t idx = static_cast<size_t>(m) * N + n;
            float c, ct;
            if (EPI == kEpiUH) {
              c = acc[i][j][4 * q + e] * scale[m];
              ct = gelu_tanh(c);
            } else if (EPI == kEpiGeluBwd) {
              c = ct = acc[i][j][4 * q + e] * gelu_tanh_grad(static_cast<float>(rq[e]));
            } else {
              c = ct = acc[i][j][4 * q + e];
            }
            if (EPI != kEpiStoreT) C[idx] = f32_to_bf16(c);
            const uint32_t b = f32_to_bf16(ct);
            if (e & 1)
              t[e >> 1] |= b << 16;
            else
              t[e >> 1] = b;
          }
          uint16_t* dst = EPI == kEpiStoreT ? C : C2;
          if (EPI != kEpiGeluBwd || C2 != nullptr)
            *reinterpret_cast<uint2*>(dst + static_cast<size_t>(n) * M + mb) = uint2{t[0], t[1]};
        }
    clock_probe_add(probe, false);
    return;
  } else {
  // Registers r and r + 1 (r even) are rows m and m + 1 of one column: both
  // are converted by one packed bf16 conversion and stored as its two halves.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x4_t rq[4][4];  // [j][q]: R of registers 4q .. 4q + 3 of tile (i, j)
    if constexpr (EPI == kEpiResidual) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) rq[j][q] = r_quad(i, j, q);
    }
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const int m = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      constexpr bool kScaled = EPI == kEpiGelu || EPI == kEpiGeluSave;
      const float sc0 = kScaled ? scale[m] : 1.0f;
      const float sc1 = kScaled ? scale[m + 1] : 1.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 128 + j * 32 + (lane & 31);
        const float a0 = acc[i][j][r], a1 = acc[i][j][r + 1];
        const size_t idx = static_cast<size_t>(m) * N + n;
        if constexpr (EPI == kEpiStoreF32) {
          Cf[idx] = a0;
          Cf[idx + N] = a1;
        } else {
          uint32_t p, p2 = 0;
          if constexpr (EPI == kEpiGelu) {
            p = pack_bf16x2(gelu_tanh(a0 * sc0), gelu_tanh(a1 * sc1));
          } else if constexpr (EPI == kEpiGeluSave) {
            // The same h as kEpiGelu, and the u the backward's kEpiUH recomputes.
            const float u0 = a0 * sc0, u1 = a1 * sc1;
            p = pack_bf16x2(gelu_tanh(u0), gelu_tanh(u1));
            p2 = pack_bf16x2(u0, u1);
          } else if constexpr (EPI == kEpiResidual) {
            p = pack_bf16x2(a0 + static_cast<float>(rq[j][r >> 2][r & 3]),
                            a1 + static_cast<float>(rq[j][r >> 2][(r & 3) + 1]));
          } else {
            static_assert(EPI == kEpiStore, "row-major epilogues only");
            p = pack_bf16x2(a0, a1);
          }
          C[idx] = static_cast<uint16_t>(p);
          C[idx + N] = static_cast<uint16_t>(p >> 16);
          if constexpr (EPI == kEpiGeluSave) {
            C2[idx] = static_cast<uint16_t>(p2);
            C2[idx + N] = static_cast<uint16_t>(p2 >> 16);
          }
        }
      }
    }
  }
  }
  clock_probe_add(probe, false);
}

// dst[c, r] = bf16(src[r, c] * scale[r]) (scale == nullptr: a plain copy
// of the bits) for a rows x cols bf16 matrix, through a 64 x 64 LDS tile.
// Full tiles (rows and cols multiples of 64, 16-byte aligned rows) move 16
// bytes per lane on both sides; any other shape takes the element path.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ src,
                                                             uint16_t* __restrict__ dst,
                                                             int rows, int cols,
                                                             const float* __restrict__ scale,
                                                             int vec) {
  __shared__ uint16_t tile[64][66];  // row stride 132 bytes: column reads spread over banks
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  if (vec) {
    // Load: lane t reads 8 consecutive columns of rows t/8 and t/8 + 32.
    const int lr = threadIdx.x >> 3, lc = (threadIdx.x & 7) * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = lr + 32 * h;
      const u32x4 v = *reinterpret_cast<const u32x4*>(src + static_cast<size_t>(r0 + r) * cols + c0 + lc);
      const float sc = scale ? scale[r0 + r] : 1.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t w = v[e];
        if (scale) w = pack_bf16x2(bf16_lo(w) * sc, bf16_hi(w) * sc);
        tile[r][lc + 2 * e] = static_cast<uint16_t>(w & 0xffffu);
        tile[r][lc + 2 * e + 1] = static_cast<uint16_t>(w >> 16);
      }
    }
    __syncthreads();
    // Store: lane t writes 8 consecutive rows of source columns t/8, t/8+32.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = lr + 32 * h;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = static_cast<uint32_t>(tile[lc + 2 * e][c]) |
               (static_cast<uint32_t>(tile[lc + 2 * e + 1][c]) << 16);
      *reinterpret_cast<u32x4*>(dst + static_cast<size_t>(c0 + c) * rows + r0 + lc) = o;
    }
    return;
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols) {
      uint16_t v = src[static_cast<size_t>(r) * cols + c];
      if (scale) v = f32_to_bf16(bf16_to_f32(v) * scale[r]);
      tile[i][tx] = v;
    }
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols) dst[static_cast<size_t>(c) * rows + r] = tile[tx][i];
  }
}

// dx = dout + rstd * (da - ahat * mean(da * ahat)), ahat = x * rstd: the
// unit-weight RMSNorm backward of the FFN input plus the residual branch.
// One workgroup per row; x, da and dout are read twice (L2-resident rows).
__global__ __launch_bounds__(256) void ffn_dx_kernel(const uint16_t* __restrict__ x,
                                                     const float* __restrict__ rstd,
                                                     const float* __restrict__ da,
                                                     const uint16_t* __restrict__ dout,
                                                     uint16_t* __restrict__ dx, int cols) {
  __shared__ double red[1][4];
  const size_t off = static_cast<size_t>(blockIdx.x) * cols;
  const float rs = rstd[blockIdx.x];
  const int nvec = cols >> 3;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x + off);
  const f32x4* dav = reinterpret_cast<const f32x4*>(da + off);
  float acc = 0.0f;
  for (int i = threadIdx.x; i < nvec; i += 256) {
    const u32x4 v = xv[i];
    const f32x4 d0 = dav[2 * i], d1 = dav[2 * i + 1];
    acc += (bf16_lo(v.x) * d0.x + bf16_hi(v.x) * d0.y) + (bf16_lo(v.y) * d0.z + bf16_hi(v.y) * d0.w) +
           (bf16_lo(v.z) * d1.x + bf16_hi(v.z) * d1.y) + (bf16_lo(v.w) * d1.z + bf16_hi(v.w) * d1.w);
  }
  double dot[1] = {acc};
  block_reduce_sum_f64_multi<4, 1>(dot, red);
  // mean(da * ahat) = rstd * sum(da * x) / cols
  const float c = static_cast<float>(dot[0] * rs / cols);
  const u32x4* gv = reinterpret_cast<const u32x4*>(dout + off);
  u32x4* ov = reinterpret_cast<u32x4*>(dx + off);
  for (int i = threadIdx.x; i < nvec; i += 256) {
    const u32x4 v = xv[i], g = gv[i];
    const f32x4 d0 = dav[2 * i], d1 = dav[2 * i + 1];
    const float dd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = bf16_lo(g[e]) + rs * (dd[2 * e] - bf16_lo(v[e]) * rs * c);
      const float hi = bf16_hi(g[e]) + rs * (dd[2 * e + 1] - bf16_hi(v[e]) * rs * c);
      o[e] = pack_bf16x2(lo, hi);
    }
    ov[i] = o;
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Sums the 256-tile GEMMs add their clock stamps to (credit_set_clock_probe).
std::atomic<uint64_t*> g_clock_probe{nullptr};

// The 256-tile kernels take 160 KiB of dynamic LDS; allow it once per
// process (the attribute belongs to the kernel, not to a device).
template <int EPI, bool KN>
hipError_t allow_big_lds() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(ffn_gemm256_kernel<EPI, KN>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, kBigLds);
}
template <bool KN>
int enable_big_lds() {
  static int status = [] {
    for (const hipError_t e :
         {allow_big_lds<kEpiGelu, KN>(), allow_big_lds<kEpiGeluSave, KN>(),
          allow_big_lds<kEpiResidual, KN>(),
          allow_big_lds<kEpiUH, KN>(), allow_big_lds<kEpiGeluBwd, KN>(),
          allow_big_lds<kEpiStore, KN>(), allow_big_lds<kEpiStoreF32, KN>(),
          allow_big_lds<kEpiStoreT, KN>()})
      if (e != hipSuccess) return hip_failure(e, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    return static_cast<int>(CREDIT_OK);
  }();
  return status;
}

// C[M, N] = epi(A[M, K] B^T) with B [N, K] (KN false) or [K, N] (KN true):
// the 256-tile kernel when M and N are multiples of 256, K a multiple of
// 128 (an even number of 64-wide K-steps), the tile count a multiple of the
// 8 XCDs and a B tile (256 * K * 2 bytes, KN: (K - 1) * N * 2 + 512), an A
// tile and the epilogue's R tile ((255 * N + 256) * 2 bytes) fit a buffer
// resource; otherwise the 128-tile kernel (M, N multiples of 128, K of 64).
template <int EPI, bool KN = false>
int launch_gemm(const uint16_t* A, const float* scale, const uint16_t* B, const uint16_t* R,
                uint16_t* C, uint16_t* C2, float* Cf, int M, int N, int K, hipStream_t stream,
                const char* name) {
  const bool big = M % kBig == 0 && N % kBig == 0 && K % (2 * kBigK) == 0 &&
                   ((M / kBig) * (N / kBig)) % 8 == 0 && K <= (1 << 22) && N <= (1 << 22) &&
                   (!KN || static_cast<uint64_t>(K) * N * 2 < (uint64_t{1} << 32));
  if (big) {
    CREDIT_TRY(enable_big_lds<KN>());
    ffn_gemm256_kernel<EPI, KN><<<dim3(static_cast<unsigned>((M / kBig) * (N / kBig))),
                                  dim3(kBigThreads), kBigLds, stream>>>(
        A, scale, B, R, C, C2, Cf, M, N, K, g_clock_probe.load(std::memory_order_relaxed));
  } else {
    ffn_gemm_kernel<EPI, KN><<<dim3(static_cast<unsigned>((M / kBM) * (N / kBN))),
                               dim3(kThreads), 0, stream>>>(A, scale, B, R, C, C2, Cf, M, N, K);
  }
  return check_launch(name);
}

int launch_transpose(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t cols,
                     const float* scale, hipStream_t stream) {
  const int vec = rows % 64 == 0 && cols % 64 == 0 && aligned16(src) && aligned16(dst);
  const dim3 grid(static_cast<unsigned>((cols + 63) / 64), static_cast<unsigned>((rows + 63) / 64));
  transpose_bf16_kernel<<<grid, 256, 0, stream>>>(src, dst, static_cast<int>(rows),
                                                  static_cast<int>(cols), scale, vec);
  return check_launch("transpose_bf16_kernel");
}

// Backward workspace, in order (each region 256-byte aligned): rstd [M]
// fp32; u, du [M, f] and h^T, du^T [f, M] bf16; dout^T, a^T [d, M] bf16;
// da [M, d] fp32.
struct BwdLayout {
  size_t rstd, u, du, ht, dut, doutt, at, da, total;
};
BwdLayout bwd_layout(int64_t M, int64_t d, int64_t f) {
  BwdLayout l;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(bytes, 256);
    return at;
  };
  l.rstd = take(M * sizeof(float));
  l.u = take(M * f * 2);
  l.du = take(M * f * 2);
  l.ht = take(M * f * 2);
  l.dut = take(M * f * 2);
  l.doutt = take(M * d * 2);
  l.at = take(M * d * 2);
  l.da = take(M * d * sizeof(float));
  l.total = o;
  return l;
}

int check_ffn_shape(int64_t rows, int64_t d, int64_t f) {
  if (rows < 0 || d < 1 || f < 1)
    return set_error(CREDIT_ERR_BAD_SHAPE, "ffn: need rows >= 0, d >= 1, f >= 1");
  if (rows % kBM != 0 || d % kBN != 0 || f % kBN != 0 || d % kBK != 0 || f % kBK != 0)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "ffn: rows, d and f must be multiples of 128 (got %lld, %lld, %lld)",
                     static_cast<long long>(rows), static_cast<long long>(d),
                     static_cast<long long>(f));
  if (rows > (int64_t{1} << 24) || d > (int64_t{1} << 20) || f > (int64_t{1} << 20) ||
      rows * f >= (int64_t{1} << 31) || d * f >= (int64_t{1} << 31) ||
      rows * d >= (int64_t{1} << 31))
    return set_error(CREDIT_ERR_BAD_SHAPE, "ffn: shape too large");
  return CREDIT_OK;
}

}  // namespace

size_t ffn_workspace(int64_t rows, int64_t ffn_dim) {
  return align_up(static_cast<size_t>(rows) * sizeof(float), 256) +
         align_up(static_cast<size_t>(rows) * ffn_dim * sizeof(uint16_t), 256);
}

size_t ffn_bwd_workspace(int64_t rows, int64_t d, int64_t ffn_dim) {
  return bwd_layout(rows, d, ffn_dim).total;
}

}  // namespace credit

using namespace credit;

extern "C" int credit_set_clock_probe(uint64_t* sums) {
  if (sums != nullptr) CREDIT_TRY(check_aligned(sums, 8, "sums"));
  g_clock_probe.store(sums, std::memory_order_relaxed);
  return CREDIT_OK;
}

extern "C" int credit_transpose_bf16(const uint16_t* src, uint16_t* dst, int64_t rows,
                                     int64_t cols, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(src, "src", rows));
  CREDIT_TRY(check_row_ptr(dst, "dst", rows));
  CREDIT_TRY(check_shape(rows, cols, int64_t{1} << 30));
  CREDIT_TRY(check_cfg(cfg));
  if (rows == 0) return CREDIT_OK;
  if (rows > (int64_t{1} << 30))
    return set_error(CREDIT_ERR_BAD_SHAPE, "transpose supports at most 2^30 rows");
  return launch_transpose(src, dst, rows, cols, nullptr, cfg_stream(cfg));
}

namespace credit {
namespace {

// The forward for either weight layout: KN false takes w1 [f, d], w2 [d, f]
// (nn.Linear), KN true w1 [d, f], w2 [f, d] ([in, out]).
template <bool KN>
int ffn_forward(const uint16_t* x, const uint16_t* w1, const uint16_t* w2, uint16_t* out,
                int64_t rows, int64_t d, int64_t f, float eps, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w1, "w1"));
  CREDIT_TRY(check_ptr(w2, "w2"));
  CREDIT_TRY(check_row_ptr(out, "out", rows));
  CREDIT_TRY(check_cfg(cfg));
  CREDIT_TRY(check_ffn_shape(rows, d, f));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w2) || !aligned16(out))
    return set_error(CREDIT_ERR_ALIGNMENT, "ffn: x, w1, w2 and out must be 16-byte aligned");
  if (rows == 0) return CREDIT_OK;
  char* ws = nullptr;
  CREDIT_TRY(acquire_workspace(cfg, ffn_workspace(rows, f), &ws));
  float* rstd = reinterpret_cast<float*>(ws_scratch(ws));
  uint16_t* h = reinterpret_cast<uint16_t*>(
      ws_scratch(ws) + align_up(static_cast<size_t>(rows) * sizeof(float), 256));
  hipStream_t stream = cfg_stream(cfg);
  const int M = static_cast<int>(rows), D = static_cast<int>(d), F = static_cast<int>(f);
  ffn_rstd_kernel<<<dim3(M), dim3(256), 0, stream>>>(x, rstd, D, eps);
  CREDIT_TRY(check_launch("ffn_rstd_kernel"));
  CREDIT_TRY((launch_gemm<kEpiGelu, KN>(x, rstd, w1, nullptr, h, nullptr, nullptr, M, F, D,
                                       stream, "ffn gemm1 (gelu)")));
  return launch_gemm<kEpiResidual, KN>(h, nullptr, w2, x, out, nullptr, nullptr, M, D, F, stream,
                                       "ffn gemm2 (residual)");
}

}  // namespace
}  // namespace credit

extern "C" int credit_ffn_rmsnorm_gelu_bf16(const uint16_t* x, const uint16_t* w1,
                                            const uint16_t* w2, uint16_t* out, int64_t rows,
                                            int64_t d, int64_t f, float eps,
                                            const credit_cfg* cfg) {
  return ffn_forward<false>(x, w1, w2, out, rows, d, f, eps, cfg);
}

namespace credit {
namespace {

template <bool KN>
int ffn_train_forward(const uint16_t* x, const uint16_t* w1, const uint16_t* w2, uint16_t* out,
                      float* rstd, uint16_t* u, uint16_t* h, int64_t rows, int64_t d, int64_t f,
                      float eps, const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w1, "w1"));
  CREDIT_TRY(check_ptr(w2, "w2"));
  CREDIT_TRY(check_row_ptr(out, "out", rows));
  CREDIT_TRY(check_row_ptr(rstd, "rstd", rows));
  CREDIT_TRY(check_row_ptr(u, "u", rows));
  CREDIT_TRY(check_row_ptr(h, "h", rows));
  CREDIT_TRY(check_cfg(cfg));
  CREDIT_TRY(check_ffn_shape(rows, d, f));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(w1),
                        static_cast<const void*>(w2), static_cast<const void*>(out),
                        static_cast<const void*>(u), static_cast<const void*>(h)})
    if (p && !aligned16(p))
      return set_error(CREDIT_ERR_ALIGNMENT,
                       "ffn training forward: x, w1, w2, out, u and h must be 16-byte aligned");
  if (rows == 0) return CREDIT_OK;
  hipStream_t stream = cfg_stream(cfg);
  const int M = static_cast<int>(rows), D = static_cast<int>(d), F = static_cast<int>(f);
  ffn_rstd_kernel<<<dim3(M), dim3(256), 0, stream>>>(x, rstd, D, eps);
  CREDIT_TRY(check_launch("ffn_rstd_kernel"));
  CREDIT_TRY((launch_gemm<kEpiGeluSave, KN>(x, rstd, w1, nullptr, h, u, nullptr, M, F, D, stream,
                                            "ffn gemm1 (gelu, saving u and h)")));
  return launch_gemm<kEpiResidual, KN>(h, nullptr, w2, x, out, nullptr, nullptr, M, D, F, stream,
                                       "ffn gemm2 (residual)");
}

}  // namespace
}  // namespace credit

extern "C" int credit_ffn_rmsnorm_gelu_fwd_train_bf16(const uint16_t* x, const uint16_t* w1,
                                                      const uint16_t* w2, uint16_t* out,
                                                      float* rstd, uint16_t* u, uint16_t* h,
                                                      int64_t rows, int64_t d, int64_t f,
                                                      float eps, const credit_cfg* cfg) {
  return ffn_train_forward<false>(x, w1, w2, out, rstd, u, h, rows, d, f, eps, cfg);
}

extern "C" int credit_ffn_rmsnorm_gelu_fwd_train_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                                         const uint16_t* w2, uint16_t* out,
                                                         float* rstd, uint16_t* u, uint16_t* h,
                                                         int64_t rows, int64_t d, int64_t f,
                                                         float eps, const credit_cfg* cfg) {
  return ffn_train_forward<true>(x, w1, w2, out, rstd, u, h, rows, d, f, eps, cfg);
}

extern "C" int credit_ffn_rmsnorm_gelu_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                               const uint16_t* w2, uint16_t* out, int64_t rows,
                                               int64_t d, int64_t f, float eps,
                                               const credit_cfg* cfg) {
  return ffn_forward<true>(x, w1, w2, out, rows, d, f, eps, cfg);
}

namespace credit {
namespace {

// The backward.  With saved == nullptr it recomputes rstd, u and h^T from x
// (one extra GEMM); with the training forward's rstd, u and h it skips that
// GEMM.  Both give the same bits: the saved u and h are the recomputed ones.
// KN false takes the nn.Linear weights (w1 [f, d], w2 [d, f]) and returns
// dW1 [f, d], dW2 [d, f]; KN true the [in, out] weights (w1 [d, f], w2
// [f, d]) and returns dW1 [d, f], dW2 [f, d].  Every GEMM reads the weights,
// dout and the activations in place, as A (K contiguous) or as B in either
// layout; the [in, out] form swaps the operands of the weight-gradient GEMMs
// instead, so it needs neither dout^T nor du^T (only the saved form's dW2,
// whose h^T no GEMM produced, takes dout^T and a transposed store).
struct FfnSaved {
  const float* rstd;
  const uint16_t* u;
  const uint16_t* h;
};

template <bool KN>
int ffn_backward(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                 const uint16_t* dout, const FfnSaved* saved, uint16_t* dx, uint16_t* dw1,
                 uint16_t* dw2, int64_t rows, int64_t d, int64_t f, float eps,
                 const credit_cfg* cfg) {
  CREDIT_TRY(check_row_ptr(x, "x", rows));
  CREDIT_TRY(check_ptr(w1, "w1"));
  CREDIT_TRY(check_ptr(w2, "w2"));
  CREDIT_TRY(check_row_ptr(dout, "dout", rows));
  CREDIT_TRY(check_row_ptr(dx, "dx", rows));
  CREDIT_TRY(check_ptr(dw1, "dw1"));
  CREDIT_TRY(check_ptr(dw2, "dw2"));
  CREDIT_TRY(check_cfg(cfg));
  CREDIT_TRY(check_ffn_shape(rows, d, f));
  if (!(eps >= 0.0f)) return set_error(CREDIT_ERR_BAD_CONFIG, "eps must be >= 0");
  if (saved != nullptr) {
    CREDIT_TRY(check_row_ptr(saved->rstd, "rstd", rows));
    CREDIT_TRY(check_row_ptr(saved->u, "u", rows));
    CREDIT_TRY(check_row_ptr(saved->h, "h", rows));
  }
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(w1),
                        static_cast<const void*>(w2), static_cast<const void*>(dout),
                        static_cast<const void*>(dx), static_cast<const void*>(dw1),
                        static_cast<const void*>(dw2),
                        static_cast<const void*>(saved ? saved->u : nullptr),
                        static_cast<const void*>(saved ? saved->h : nullptr)})
    if (p && !aligned16(p))
      return set_error(CREDIT_ERR_ALIGNMENT, "ffn backward: every buffer must be 16-byte aligned");
  hipStream_t stream = cfg_stream(cfg);
  if (rows == 0) {
    // No rows: the weight gradients are sums over nothing (zero bits; a
    // fill kernel rather than a memset, so the call can be graph-captured).
    const int64_t words = d * f / 2;  // two bf16 per fp32 word (d, f even)
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    fill_f32_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(reinterpret_cast<float*>(dw1), 0.0f,
                                                             words);
    CREDIT_TRY(check_launch("fill_f32_kernel"));
    fill_f32_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(reinterpret_cast<float*>(dw2), 0.0f,
                                                             words);
    return check_launch("fill_f32_kernel");
  }
  const BwdLayout L = bwd_layout(rows, d, f);
  char* ws = nullptr;
  CREDIT_TRY(acquire_workspace(cfg, L.total, &ws));
  char* b = ws_scratch(ws);
  const float* rstd = saved ? saved->rstd : reinterpret_cast<float*>(b + L.rstd);
  const uint16_t* u = saved ? saved->u : reinterpret_cast<uint16_t*>(b + L.u);
  uint16_t* du = reinterpret_cast<uint16_t*>(b + L.du);
  uint16_t* ht = reinterpret_cast<uint16_t*>(b + L.ht);
  uint16_t* dut = reinterpret_cast<uint16_t*>(b + L.dut);
  uint16_t* doutt = reinterpret_cast<uint16_t*>(b + L.doutt);
  uint16_t* at = reinterpret_cast<uint16_t*>(b + L.at);
  float* da = reinterpret_cast<float*>(b + L.da);
  const int M = static_cast<int>(rows), D = static_cast<int>(d), F = static_cast<int>(f);
  if (saved == nullptr) {
    ffn_rstd_kernel<<<dim3(M), dim3(256), 0, stream>>>(x, reinterpret_cast<float*>(b + L.rstd), D,
                                                       eps);
    CREDIT_TRY(check_launch("ffn_rstd_kernel"));
  }
  // The A operands of the weight gradients in the K-contiguous layout A
  // takes: a^T = bf16(x rstd)^T always, dout^T where no other form reads it.
  if (!KN || saved != nullptr) CREDIT_TRY(launch_transpose(dout, doutt, M, D, nullptr, stream));
  CREDIT_TRY(launch_transpose(x, at, M, D, rstd, stream));
  // u = (x W1^T) rstd (x W1 for [in, out]), h^T = GELU(u)^T, unless saved.
  if (saved == nullptr)
    CREDIT_TRY((launch_gemm<kEpiUH, KN>(x, rstd, w1, nullptr, reinterpret_cast<uint16_t*>(b + L.u),
                                        ht, nullptr, M, F, D, stream, "ffn bwd gemm u")));
  // du = (dout W2) * GELU'(u) (dout W2^T for [in, out]), with du^T for the
  // nn.Linear dW1 GEMM.
  CREDIT_TRY((launch_gemm<kEpiGeluBwd, !KN>(dout, nullptr, w2, u, du, KN ? nullptr : dut,
                                            nullptr, M, F, D, stream, "ffn bwd gemm du")));
  if constexpr (!KN) {
    // dW2 [d, f] = dout^T h: h^T [f, M] as the B operand, or the saved h
    // [M, f] read as [K, N].
    if (saved == nullptr)
      CREDIT_TRY(launch_gemm<kEpiStore>(doutt, nullptr, ht, nullptr, dw2, nullptr, nullptr, D, F,
                                        M, stream, "ffn bwd gemm dw2"));
    else
      CREDIT_TRY((launch_gemm<kEpiStore, true>(doutt, nullptr, saved->h, nullptr, dw2, nullptr,
                                               nullptr, D, F, M, stream, "ffn bwd gemm dw2")));
    // dW1 [f, d] = du^T a.
    CREDIT_TRY(launch_gemm<kEpiStore>(dut, nullptr, at, nullptr, dw1, nullptr, nullptr, F, D, M,
                                      stream, "ffn bwd gemm dw1"));
  } else {
    // dW2 [f, d] = h^T dout: h^T as A and dout [M, d] read as [K, N]; from
    // the saved h, (dout^T h)^T with h read as [K, N] and the output stored
    // transposed.
    if (saved == nullptr)
      CREDIT_TRY((launch_gemm<kEpiStore, true>(ht, nullptr, dout, nullptr, dw2, nullptr, nullptr,
                                               F, D, M, stream, "ffn bwd gemm dw2")));
    else
      CREDIT_TRY((launch_gemm<kEpiStoreT, true>(doutt, nullptr, saved->h, nullptr, dw2, nullptr,
                                                nullptr, D, F, M, stream, "ffn bwd gemm dw2")));
    // dW1 [d, f] = a^T du: du [M, f] read as [K, N].
    CREDIT_TRY((launch_gemm<kEpiStore, true>(at, nullptr, du, nullptr, dw1, nullptr, nullptr, D, F,
                                             M, stream, "ffn bwd gemm dw1")));
  }
  // da [M, d] = du W1 (du W1^T for [in, out]), fp32, then dx = dout +
  // RMSNorm backward of da.
  CREDIT_TRY((launch_gemm<kEpiStoreF32, !KN>(du, nullptr, w1, nullptr, nullptr, nullptr, da, M, D,
                                             F, stream, "ffn bwd gemm da")));
  ffn_dx_kernel<<<dim3(M), dim3(256), 0, stream>>>(x, rstd, da, dout, dx, D);
  return check_launch("ffn_dx_kernel");
}

}  // namespace
}  // namespace credit

extern "C" int credit_ffn_rmsnorm_gelu_bwd_bf16(const uint16_t* x, const uint16_t* w1,
                                                const uint16_t* w2, const uint16_t* dout,
                                                uint16_t* dx, uint16_t* dw1, uint16_t* dw2,
                                                int64_t rows, int64_t d, int64_t f, float eps,
                                                const credit_cfg* cfg) {
  return ffn_backward<false>(x, w1, w2, dout, nullptr, dx, dw1, dw2, rows, d, f, eps, cfg);
}

extern "C" int credit_ffn_rmsnorm_gelu_bwd_saved_bf16(
    const uint16_t* x, const uint16_t* w1, const uint16_t* w2, const uint16_t* dout,
    const float* rstd, const uint16_t* u, const uint16_t* h, uint16_t* dx, uint16_t* dw1,
    uint16_t* dw2, int64_t rows, int64_t d, int64_t f, const credit_cfg* cfg) {
  const FfnSaved saved{rstd, u, h};
  return ffn_backward<false>(x, w1, w2, dout, &saved, dx, dw1, dw2, rows, d, f, 0.0f, cfg);
}

extern "C" int credit_ffn_rmsnorm_gelu_bwd_kn_bf16(const uint16_t* x, const uint16_t* w1,
                                                   const uint16_t* w2, const uint16_t* dout,
                                                   uint16_t* dx, uint16_t* dw1, uint16_t* dw2,
                                                   int64_t rows, int64_t d, int64_t f, float eps,
                                                   const credit_cfg* cfg) {
  return ffn_backward<true>(x, w1, w2, dout, nullptr, dx, dw1, dw2, rows, d, f, eps, cfg);
}

extern "C" int credit_ffn_rmsnorm_gelu_bwd_saved_kn_bf16(
    const uint16_t* x, const uint16_t* w1, const uint16_t* w2, const uint16_t* dout,
    const float* rstd, const uint16_t* u, const uint16_t* h, uint16_t* dx, uint16_t* dw1,
    uint16_t* dw2, int64_t rows, int64_t d, int64_t f, const credit_cfg* cfg) {
  const FfnSaved saved{rstd, u, h};
  return ffn_backward<true>(x, w1, w2, dout, &saved, dx, dw1, dw2, rows, d, f, 0.0f, cfg);
}
