// Host plumbing of libcredit_hip.so: errors, argument checks, device
// properties, the workspace cache and the watchdog query.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "api_internal.hpp"
#include "common.hpp"
#include "workspace_cache.hpp"

namespace credit {

namespace {
thread_local char g_last_error[512] = "";

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// A new buffer for the cache: hipMalloc, then its header, counter and slot
// areas zeroed by a fill kernel queued on the stream that will use it (a
// kernel, not a memset node, so it stays correct inside a captured graph;
// the allocation itself cannot be captured).
struct DeviceAlloc {
  int operator()(int device, void* stream, size_t bytes, char** out) const {
    (void)device;
    void* p = nullptr;
    CREDIT_HIP(hipMalloc(&p, bytes));
    const int64_t words = static_cast<int64_t>(kScratchOffset / 4);
    fill_u32_kernel<<<dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0,
                      static_cast<hipStream_t>(stream)>>>(static_cast<uint32_t*>(p), 0u, words);
    CREDIT_TRY(check_launch("fill_u32_kernel"));
    *out = static_cast<char*>(p);
    return CREDIT_OK;
  }
};
WorkspaceCache<DeviceAlloc>& workspace_cache() {
  static WorkspaceCache<DeviceAlloc>* cache = new WorkspaceCache<DeviceAlloc>();  // never freed
  return *cache;
}

std::mutex g_props_mutex;
std::vector<DeviceProps> g_props;
}  // namespace

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_failure(hipError_t err, const char* what) {
  return set_error(CREDIT_ERR_HIP, "%s failed: %s (%d)", what,
                   hipGetErrorString(err), static_cast<int>(err));
}

int check_ptr(const void* p, const char* name) {
  if (p == nullptr) return set_error(CREDIT_ERR_NULL_POINTER, "%s is NULL", name);
  return CREDIT_OK;
}

int check_aligned(const void* p, size_t align, const char* name) {
  if (reinterpret_cast<uintptr_t>(p) % align != 0)
    return set_error(CREDIT_ERR_ALIGNMENT, "%s is not %zu-byte aligned", name,
                     align);
  return CREDIT_OK;
}

int check_shape(int64_t rows, int64_t cols, int64_t max_cols) {
  if (rows < 0 || cols < 1)
    return set_error(CREDIT_ERR_BAD_SHAPE,
                     "shape (%lld, %lld): need rows >= 0 and cols >= 1",
                     static_cast<long long>(rows), static_cast<long long>(cols));
  if (cols > max_cols)
    return set_error(CREDIT_ERR_BAD_SHAPE, "cols %lld exceeds the maximum %lld",
                     static_cast<long long>(cols),
                     static_cast<long long>(max_cols));
  if (rows > (int64_t{1} << 31) - 1)
    return set_error(CREDIT_ERR_BAD_SHAPE, "rows %lld exceeds 2^31-1",
                     static_cast<long long>(rows));
  return CREDIT_OK;
}

int check_cfg(const credit_cfg* cfg) {
  if (cfg == nullptr) return CREDIT_OK;
  if (cfg->variant < CREDIT_VARIANT_AUTO || cfg->variant > CREDIT_VARIANT_SPLIT)
    return set_error(CREDIT_ERR_BAD_CONFIG, "unknown variant %d", cfg->variant);
  if (cfg->split < 0 || cfg->split > 64)
    return set_error(CREDIT_ERR_BAD_CONFIG, "split %d outside [0, 64]",
                     cfg->split);
  if (cfg->workspace != nullptr &&
      reinterpret_cast<uintptr_t>(cfg->workspace) % 256 != 0)
    return set_error(CREDIT_ERR_WORKSPACE, "workspace is not 256-byte aligned");
  return CREDIT_OK;
}

// XCDs (XCCs) of a device as the runtime reports them; gfx950 carries 32
// CUs per XCD, the fallback when the attribute is unavailable.
int xcd_count_of(int device, int cu_count) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, device) == hipSuccess && n > 0)
    return n;
  (void)hipGetLastError();
  return cu_count >= 32 ? cu_count / 32 : 1;
}

int current_device_props(const DeviceProps** out) {
  int dev = 0;
  CREDIT_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_props_mutex);
  if (static_cast<int>(g_props.size()) <= dev) g_props.resize(dev + 1);
  DeviceProps& p = g_props[dev];
  if (p.device != dev) {
    hipDeviceProp_t prop;
    CREDIT_HIP(hipGetDeviceProperties(&prop, dev));
    p.cu_count = prop.multiProcessorCount;
    p.max_lds_per_block = static_cast<int>(prop.sharedMemPerBlock);
    p.lds_per_cu = static_cast<int>(prop.maxSharedMemoryPerMultiProcessor);
    p.clock_khz = prop.clockRate;
    p.cooperative = prop.cooperativeLaunch;
    p.l2_bytes = prop.l2CacheSize;
    // The XCD count is what the blockIdx -> XCD round-robin mapping needs.
    p.xcd_count = xcd_count_of(dev, p.cu_count);
    p.device = dev;
  }
  *out = &p;
  return CREDIT_OK;
}

int acquire_workspace(const credit_cfg* cfg, size_t bytes, char** base) {
  const size_t need = kScratchOffset + bytes;
  if (cfg != nullptr && cfg->workspace != nullptr) {
    if (cfg->workspace_bytes < need)
      return set_error(CREDIT_ERR_WORKSPACE,
                       "workspace of %zu bytes is smaller than the %zu needed",
                       cfg->workspace_bytes, need);
    *base = static_cast<char*>(cfg->workspace);
    return CREDIT_OK;
  }
  int dev = 0;
  CREDIT_HIP(hipGetDevice(&dev));
  return workspace_cache().get(dev, cfg_stream(cfg), need, base);
}

__global__ void fill_f32_kernel(float* __restrict__ p, float v, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

std::atomic<uint32_t> g_spin_limit{kSpinLimit};

uint32_t split_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

// One host-mapped word per device, raised by a split launch whose bounded
// wait expired (common.hpp, split_poll), read by the host without a sync.
struct HostFlag {
  int device;
  volatile uint32_t* host;
  uint32_t* dev;
};
std::mutex g_host_flag_mu;
std::vector<HostFlag> g_host_flags;
thread_local bool g_in_noalloc = false;

// The device's flag; with allow_alloc false and none allocated yet, a flag
// with null words (the caller then goes without it).
int host_watchdog_flag(int device, HostFlag* out, bool allow_alloc = true) {
  std::lock_guard<std::mutex> lock(g_host_flag_mu);
  for (const HostFlag& f : g_host_flags)
    if (f.device == device) {
      *out = f;
      return CREDIT_OK;
    }
  if (!allow_alloc) {
    *out = HostFlag{device, nullptr, nullptr};
    return CREDIT_OK;
  }
  void* p = nullptr;
  CREDIT_HIP(hipHostMalloc(&p, 64, hipHostMallocMapped));
  *static_cast<volatile uint32_t*>(p) = 0;
  void* d = nullptr;
  CREDIT_HIP(hipHostGetDevicePointer(&d, p, 0));
  g_host_flags.push_back(HostFlag{device, static_cast<volatile uint32_t*>(p),
                                  static_cast<uint32_t*>(d)});
  *out = g_host_flags.back();
  return CREDIT_OK;
}

NoAllocScope::NoAllocScope() : prev_(g_in_noalloc) { g_in_noalloc = true; }
NoAllocScope::~NoAllocScope() { g_in_noalloc = prev_; }
bool in_noalloc_call() { return g_in_noalloc; }

int acquire_split_workspace(const credit_cfg* cfg, int64_t groups, int members,
                            int k_values, int ring, size_t extra_bytes, SplitWorkspace* out) {
  int device = 0;
  CREDIT_HIP(hipGetDevice(&device));
  HostFlag flag;
  CREDIT_TRY(host_watchdog_flag(device, &flag, !g_in_noalloc));
  if (flag.host != nullptr && *flag.host != 0)
    return set_error(CREDIT_ERR_WATCHDOG,
                     "an earlier split launch on device %d gave up waiting for its group (its "
                     "outputs are wrong); credit_check_watchdog() reports and clears this",
                     device);
  if (members * k_values > kMaxExchangeValues)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "split of %d members exchanges %d partials per stage (at most %d)", members,
                     members * k_values, kMaxExchangeValues);
  const size_t slot_bytes = split_slot_bytes(groups, members, k_values, ring);
  if (slot_bytes > kSlotAreaBytes)
    return set_error(CREDIT_ERR_UNSUPPORTED,
                     "split launch of %lld groups x %d members x %d values x ring %d needs %zu "
                     "bytes of exchange slots (at most %zu)", static_cast<long long>(groups),
                     members, k_values, ring, slot_bytes, kSlotAreaBytes);
  char* base = nullptr;
  CREDIT_TRY(acquire_workspace(cfg, extra_bytes, &base));
  out->counters = ws_counters(base);
  out->watchdog = ws_watchdog(base);
  out->slots = ws_slots(base);
  out->extra = ws_scratch(base);
  out->host_flag = flag.dev;
  return CREDIT_OK;
}

// Shape of the last co-resident split launch this thread planned
// (credit_last_split_shape).
struct SplitShape {
  int threads = 0;
  int lds_bytes = 0;
  int per_cu = 0;
  int dispensers = 0;
  int64_t groups = 0;
};
thread_local SplitShape g_last_split;

int coresident_groups(const void* kernel, int threads, size_t dynamic_lds, int members,
                      int64_t* groups, int* dispensers) {
  struct Entry {
    int device;
    const void* kernel;
    int threads;
    size_t lds;
    int per_cu;
    size_t static_lds;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  CREDIT_HIP(hipGetDevice(&dev));
  int per_cu = -1;
  size_t static_lds = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.device == dev && e.kernel == kernel && e.threads == threads && e.lds == dynamic_lds) {
        per_cu = e.per_cu;
        static_lds = e.static_lds;
      }
  }
  if (per_cu < 0) {
    CREDIT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads,
                                                            dynamic_lds));
    hipFuncAttributes attr;
    CREDIT_HIP(hipFuncGetAttributes(&attr, kernel));
    static_lds = attr.sharedSizeBytes;
    std::lock_guard<std::mutex> lock(mu);
    cache.push_back(Entry{dev, kernel, threads, dynamic_lds, per_cu, static_lds});
  }
  const DeviceProps* props = nullptr;
  CREDIT_TRY(current_device_props(&props));
  const int64_t resident = static_cast<int64_t>(per_cu) * props->cu_count;
  *groups = plan::coresident_group_count(resident, members);
  const int d = plan::dispensers_for(resident, members);
  if (dispensers != nullptr) *dispensers = d;
  g_last_split = SplitShape{threads, static_cast<int>(static_lds + dynamic_lds), per_cu, d,
                            *groups};
  return CREDIT_OK;
}

int split_dispensers(int per_cu, int cu_count, int members) {
  return plan::dispensers_for(static_cast<int64_t>(per_cu) * cu_count, members);
}

int cu_count_or_default() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    (void)hipGetLastError();
    return 256;
  }
  const DeviceProps* p = nullptr;
  if (current_device_props(&p) != CREDIT_OK) return 256;
  return p->cu_count;
}

int check_launch(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_failure(err, kernel);
  return CREDIT_OK;
}

}  // namespace credit

using namespace credit;

extern "C" {

const char* credit_version(void) { return "credit-hip 0.1.0 gfx950"; }

const char* credit_last_error(void) { return g_last_error; }

const char* credit_status_string(int status) {
  switch (status) {
    case CREDIT_OK: return "CREDIT_OK";
    case CREDIT_ERR_NULL_POINTER: return "CREDIT_ERR_NULL_POINTER";
    case CREDIT_ERR_BAD_SHAPE: return "CREDIT_ERR_BAD_SHAPE";
    case CREDIT_ERR_ALIGNMENT: return "CREDIT_ERR_ALIGNMENT";
    case CREDIT_ERR_UNSUPPORTED: return "CREDIT_ERR_UNSUPPORTED";
    case CREDIT_ERR_WORKSPACE: return "CREDIT_ERR_WORKSPACE";
    case CREDIT_ERR_HIP: return "CREDIT_ERR_HIP";
    case CREDIT_ERR_WATCHDOG: return "CREDIT_ERR_WATCHDOG";
    case CREDIT_ERR_BAD_CONFIG: return "CREDIT_ERR_BAD_CONFIG";
    default: return "CREDIT_ERR_UNKNOWN";
  }
}

int credit_query_device(int32_t device, credit_device_info* info) {
  CREDIT_TRY(check_ptr(info, "info"));
  if (device < 0) return set_error(CREDIT_ERR_BAD_CONFIG, "device %d < 0", device);
  int count = 0;
  CREDIT_HIP(hipGetDeviceCount(&count));
  if (device >= count)
    return set_error(CREDIT_ERR_BAD_CONFIG, "device %d of %d", device, count);
  hipDeviceProp_t prop;
  CREDIT_HIP(hipGetDeviceProperties(&prop, device));
  memset(info, 0, sizeof(*info));
  snprintf(info->name, sizeof(info->name), "%s", prop.name);
  snprintf(info->arch, sizeof(info->arch), "%s", prop.gcnArchName);
  info->device = device;
  info->cu_count = prop.multiProcessorCount;
  info->xcd_count = xcd_count_of(device, prop.multiProcessorCount);
  info->wave_size = prop.warpSize;
  info->max_threads_per_block = prop.maxThreadsPerBlock;
  info->cooperative_launch = prop.cooperativeLaunch;
  info->lds_bytes_per_block = static_cast<int64_t>(prop.sharedMemPerBlock);
  info->lds_bytes_per_cu =
      static_cast<int64_t>(prop.maxSharedMemoryPerMultiProcessor);
  info->l2_bytes = prop.l2CacheSize;
  info->hbm_bytes = static_cast<int64_t>(prop.totalGlobalMem);
  info->clock_khz = prop.clockRate;
  info->mem_clock_khz = prop.memoryClockRate;
  info->mem_bus_width_bits = prop.memoryBusWidth;
  return CREDIT_OK;
}

size_t credit_workspace_bytes(int32_t op, int64_t rows, int64_t cols,
                              int32_t variant, int32_t split) {
  if (rows <= 0 || cols <= 0) return 0;
  const int cus = cu_count_or_default();
  size_t body = 0;
  switch (op) {
    case CREDIT_OP_ROW_SUM_MAX:
      body = row_sum_max_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_RMSNORM_FWD:
      body = rmsnorm_fwd_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_LAYERNORM_FWD:
      body = layernorm_fwd_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_RMSNORM_BWD:
      body = rmsnorm_bwd_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_RMSNORM_FWD_BWD:
      body = rmsnorm_fused_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_LAYERNORM_BWD:
      body = layernorm_bwd_workspace(rows, cols, variant, split, 4, cus);
      break;
    case CREDIT_OP_LAYERNORM_BWD_BF16:
      body = layernorm_bwd_workspace(rows, cols, variant, split, 2, cus);
      break;
    case CREDIT_OP_FFN:  // cols = the FFN hidden width f
      body = ffn_workspace(rows, cols);
      break;
    case CREDIT_OP_SOFTMAX_FWD:
    case CREDIT_OP_SOFTMAX_BWD:
    case CREDIT_OP_SOFTMAX_LOGITS_BWD:
      body = softmax_workspace(op, rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_ROWWISE_QUANT:
      body = rowwise_quant_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_LARS_MOMENTUM:
      body = lars_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_WEIGHTED_VAR_BWD:
      body = wvar_bwd_workspace(rows, cols, variant, split, cus);
      break;
    case CREDIT_OP_PEARSON_BWD:
      body = pearson_bwd_workspace(rows, cols, variant, split, cus);
      break;
    default:
      body = 0;
  }
  return body == 0 ? 0 : kScratchOffset + body;
}

size_t credit_ffn_bwd_workspace_bytes(int64_t rows, int64_t d, int64_t f) {
  if (rows <= 0 || d <= 0 || f <= 0) return 0;
  return kScratchOffset + ffn_bwd_workspace(rows, d, f);
}

int credit_check_watchdog(const credit_cfg* cfg) {
  CREDIT_TRY(check_cfg(cfg));
  // The allocation-free entry points' fixed array has a watchdog word of its
  // own (they go without the host-mapped one when none exists yet).
  bool noalloc_flag = false;
  {
    int dev = 0;
    CREDIT_HIP(hipGetDevice(&dev));
    if (char* na = noalloc_scratch_base(dev)) {
      uint32_t w = 0;
      CREDIT_HIP(hipDeviceSynchronize());
      CREDIT_HIP(hipMemcpy(&w, na, sizeof(w), hipMemcpyDeviceToHost));
      if (w != 0) {
        CREDIT_HIP(hipMemset(na, 0, kScratchOffset));
        CREDIT_HIP(hipDeviceSynchronize());
        noalloc_flag = true;
      }
    }
  }
  char* base = nullptr;
  if (cfg != nullptr && cfg->workspace != nullptr) {
    CREDIT_TRY(acquire_workspace(cfg, 0, &base));
  } else {
    int dev = 0;
    CREDIT_HIP(hipGetDevice(&dev));
    base = workspace_cache().peek(dev, cfg_stream(cfg));
    if (base == nullptr) {  // no call on this stream used a workspace
      CREDIT_HIP(hipDeviceSynchronize());
      HostFlag hf;
      CREDIT_TRY(host_watchdog_flag(dev, &hf));
      if (*hf.host == 0 && !noalloc_flag) return CREDIT_OK;
      *hf.host = 0;
      return set_error(CREDIT_ERR_WATCHDOG, "a split-row barrier exceeded its spin limit");
    }
  }
  uint32_t flag = 0;
  CREDIT_HIP(hipStreamSynchronize(cfg_stream(cfg)));
  CREDIT_HIP(hipMemcpy(&flag, base, sizeof(flag), hipMemcpyDeviceToHost));
  // The device-wide host word: cleared here, so split calls run again.
  int device = 0;
  CREDIT_HIP(hipGetDevice(&device));
  HostFlag hf;
  CREDIT_TRY(host_watchdog_flag(device, &hf));
  const bool device_flag = *hf.host != 0;
  *hf.host = 0;
  if (flag != 0) {
    // A barrier that gave up leaves its counters mid-protocol: return the
    // whole header and counter area to the zero state.
    CREDIT_HIP(hipMemset(base, 0, kScratchOffset));
    CREDIT_HIP(hipDeviceSynchronize());
  }
  if (flag != 0 || device_flag || noalloc_flag)
    return set_error(CREDIT_ERR_WATCHDOG,
                     "a split-row barrier exceeded its spin limit");
  return CREDIT_OK;
}

int credit_host_watchdog_words(int32_t* count) {
  CREDIT_TRY(check_ptr(count, "count"));
  std::lock_guard<std::mutex> lock(g_host_flag_mu);
  *count = static_cast<int32_t>(g_host_flags.size());
  return CREDIT_OK;
}

int credit_last_split_shape(int32_t* threads, int32_t* lds_bytes, int32_t* per_cu,
                            int32_t* dispensers) {
  CREDIT_TRY(check_ptr(threads, "threads"));
  CREDIT_TRY(check_ptr(lds_bytes, "lds_bytes"));
  CREDIT_TRY(check_ptr(per_cu, "per_cu"));
  CREDIT_TRY(check_ptr(dispensers, "dispensers"));
  if (g_last_split.threads == 0)
    return set_error(CREDIT_ERR_UNSUPPORTED, "no co-resident split launch on this thread yet");
  *threads = g_last_split.threads;
  *lds_bytes = g_last_split.lds_bytes;
  *per_cu = g_last_split.per_cu;
  *dispensers = g_last_split.dispensers;
  return CREDIT_OK;
}

int credit_set_spin_limit(uint32_t polls, uint32_t* previous) {
  const uint32_t old = g_spin_limit.exchange(polls, std::memory_order_relaxed);
  if (previous != nullptr) *previous = old;
  return CREDIT_OK;
}

}  // extern "C"
