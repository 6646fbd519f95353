// Host-side plumbing shared by every C-ABI entry point: status codes and the
// thread-local error text, argument checks that run before anything touches
// the GPU, the per-device workspace cache and device-property cache.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/credit.h"
#include "split_plan.hpp"

namespace credit {

int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_failure(hipError_t err, const char* what);

#define CREDIT_HIP(expr)                                       \
  do {                                                         \
    hipError_t credit_err__ = (expr);                          \
    if (credit_err__ != hipSuccess)                            \
      return ::credit::hip_failure(credit_err__, #expr);       \
  } while (0)

#define CREDIT_TRY(expr)                 \
  do {                                   \
    int credit_status__ = (expr);        \
    if (credit_status__ != CREDIT_OK)    \
      return credit_status__;            \
  } while (0)

struct DeviceProps {
  int device = -1;
  int cu_count = 0;
  int xcd_count = 0;
  int max_lds_per_block = 0;
  int lds_per_cu = 0;
  int clock_khz = 0;
  int cooperative = 0;
  long long l2_bytes = 0;
};

// Cached hipGetDeviceProperties for the current device.
int current_device_props(const DeviceProps** out);

// Argument checks.  Every one returns CREDIT_OK or a negative status after
// recording a message; none of them calls into HIP.
int check_ptr(const void* p, const char* name);
// A buffer indexed by row: NULL is accepted when there are no rows (torch
// hands out NULL data pointers for empty tensors).
inline int check_row_ptr(const void* p, const char* name, int64_t rows) {
  return rows == 0 ? CREDIT_OK : check_ptr(p, name);
}
int check_aligned(const void* p, size_t align, const char* name);
int check_shape(int64_t rows, int64_t cols, int64_t max_cols);
int check_cfg(const credit_cfg* cfg);

inline hipStream_t cfg_stream(const credit_cfg* cfg) {
  return cfg ? static_cast<hipStream_t>(cfg->stream) : nullptr;
}
inline int cfg_variant(const credit_cfg* cfg) {
  return cfg ? cfg->variant : CREDIT_VARIANT_AUTO;
}
inline int cfg_split(const credit_cfg* cfg) { return cfg ? cfg->split : 0; }

// Workspace layout, identical for every operation:
//   [0, 256)                 header, one 64-byte line per word: the watchdog
//                            word the split-row barrier raises (byte 0), the
//                            exchange-tag sequence of split launches (byte
//                            64, split_plan.hpp) and the count of dispenser
//                            subsets whose workgroups have all exited (byte
//                            128)
//   [256, 256 + 1 MiB)       counter area: 262144 uint32 slots.  The first
//                            kDispensers lines are the ticket dispensers of
//                            split launches (word 0: the next ticket, word 1:
//                            the subset's exited workgroups); group arrival
//                            counters follow from slot kGroupCounterBase,
//                            one 64-byte line each.  Every protocol returns
//                            its counters to zero, so the area stays zero
//                            between calls whatever shapes the calls have.
//   [kSlotOffset, +4 MiB)    exchange slots of the tagged-slot split
//                            protocol.  Only split launches write here, and
//                            every slot carries the tag of the launch stage
//                            that wrote it; tags come from the sequence word,
//                            which every split launch advances on the device,
//                            so a later launch (or a graph replay) never
//                            takes an old value for its own.
//   [kScratchOffset, ...)    op-specific scratch (dweight partials, FFN h,
//                            row-sum partials): written before it is read
//                            within one call, so its contents between calls
//                            do not matter.
// The first kScratchOffset bytes must read zero before the workspace's
// first use; calls keep them that way (counters return to zero, the
// sequence and slot tags only grow, and the launch that takes the sequence
// past its limit returns the slot area to zero itself).  Uses the caller's
// buffer when cfg->workspace is set, else the library's buffer for (device,
// stream) (workspace_cache.hpp).
constexpr size_t kWorkspaceHeader = 256;
constexpr int kHeaderSeqWord = 16;   // uint32 index of the sequence word
constexpr int kHeaderExitWord = 32;  // uint32 index of the exited-subset count
constexpr int kCounterSlots = 262144;
constexpr size_t kSlotOffset = kWorkspaceHeader + size_t{4} * kCounterSlots;
// Tagged slots of one split launch: at most (resident workgroups) x ring x
// values per member; 512 KiB at 256 CUs for the largest (softmax group
// kernel, ring 16, two values), 4 MiB leaves room for larger devices.
constexpr size_t kSlotAreaBytes = size_t{4} << 20;
constexpr size_t kScratchOffset = kSlotOffset + kSlotAreaBytes;
constexpr int kDispensers = plan::kMaxDispensers;  // ticket dispensers at most (blockIdx % 8)
constexpr int kDispenserStride = 16;     // one 64-byte line each
constexpr int kGroupCounterBase = kDispensers * kDispenserStride;  // first group counter
constexpr int kGroupCounterStride = 16;  // one 64-byte line per group counter
// The counter area's last line holds the row-ticket counter of the queued
// group pipelines (returned to zero by the launch that draws its last ticket).
constexpr int kQueueWord = kCounterSlots - 16;
constexpr int kMaxGroupsPerLaunch =
    (kQueueWord - kGroupCounterBase) / kGroupCounterStride / kDispensers * kDispensers;
// Groups of a split launch are padded to a multiple of kDispensers (the
// padding groups exit at once).
inline int64_t padded_groups(int64_t groups) {
  return (groups + kDispensers - 1) / kDispensers * kDispensers;
}
// Partials one exchange stage carries (members * values): one wave polls
// them, one lane per slot.
constexpr int kMaxExchangeValues = 64;
// Bytes of exchange slots a split launch needs: one 64-bit slot per
// (group, slot row, value, member); `ring` slot rows per group.
inline size_t split_slot_bytes(int64_t groups, int members, int k_values, int ring) {
  return static_cast<size_t>(groups) * ring * k_values * members * sizeof(uint64_t);
}
int acquire_workspace(const credit_cfg* cfg, size_t bytes, char** base);

// Workspace of a ticketed split launch: the counter area, the partial slots
// of `groups` groups (in the slot area), then `extra_bytes` of scratch for
// the operation's own use.
struct SplitWorkspace {
  uint32_t* counters = nullptr;
  uint32_t* watchdog = nullptr;
  uint64_t* slots = nullptr;
  char* extra = nullptr;
  uint32_t* host_flag = nullptr;  // device address of the device's host-mapped watchdog word
};
// Polls a split wait makes before it gives up (credit_set_spin_limit).
uint32_t split_spin_limit();
// Scratch bytes (after kScratchOffset) of a split launch, never 0 so that
// credit_workspace_bytes reports that the launch needs a workspace.
inline size_t split_workspace_bytes(int64_t groups, int members, int k_values, int ring,
                                    size_t extra_bytes) {
  (void)groups, (void)members, (void)k_values, (void)ring;
  return (extra_bytes + 255) / 256 * 256 + 256;
}
int acquire_split_workspace(const credit_cfg* cfg, int64_t groups, int members,
                            int k_values, int ring, size_t extra_bytes, SplitWorkspace* out);

// Marks the calls this thread makes inside an allocation-free entry point
// (credit_*_noalloc): the split workspace then uses the device's host-mapped
// watchdog word only if an earlier call already allocated it, and allocates
// none (the expiry still raises the workspace's own watchdog word, which
// credit_check_watchdog reads).
class NoAllocScope {
 public:
  NoAllocScope();
  ~NoAllocScope();
  NoAllocScope(const NoAllocScope&) = delete;
  NoAllocScope& operator=(const NoAllocScope&) = delete;

 private:
  bool prev_;
};
bool in_noalloc_call();
// The allocation-free scratch array of `device` once an allocation-free
// call has looked its address up on that device (nullptr before).
char* noalloc_scratch_base(int device);

// Split launches wait inside a group for all of its members, and the
// dispatcher does not reliably start a pending workgroup on a CU that a
// finished group freed while resident workgroups spin (measured on MI355X:
// pending members started seconds late when launches were queued back to
// back).  So a split launch is one resident wave: G groups of P members,
// G a multiple of kDispensers, G*P no more than the workgroups of the kernel
// resident at once on the device, and each group loops over its rows.
// *groups = G (0: not even kDispensers groups fit).  *dispensers: the ticket
// subsets of the launch (plan::dispensers_for), chosen so that every subset's
// slots hold at least two groups: no group spans every slot of its subset.
int coresident_groups(const void* kernel, int threads, size_t dynamic_lds, int members,
                      int64_t* groups, int* dispensers = nullptr);
// Dispenser subsets of a launch of `groups` x `members` of a kernel with
// `per_cu` workgroups resident per CU (plan::dispensers_for).
int split_dispensers(int per_cu, int cu_count, int members);
// Upper bound of G for workspace sizing without a device query.
inline int64_t coresident_groups_bound(int members, int cu_count) {
  const int64_t resident = static_cast<int64_t>(cu_count) * 32;  // >= blocks per CU
  return (resident / members + kDispensers - 1) / kDispensers * kDispensers;
}
// Slot rows per group of the barrier-synchronised split kernels: every
// exchange ends with a workgroup barrier, so no member publishes stage s+2
// before every member has polled stage s.  Four rows leave margin.
constexpr int kSplitRing = 4;
inline uint32_t* ws_watchdog(char* base) { return reinterpret_cast<uint32_t*>(base); }
inline uint32_t* ws_counters(char* base) {
  return reinterpret_cast<uint32_t*>(base + kWorkspaceHeader);
}
inline uint64_t* ws_slots(char* base) { return reinterpret_cast<uint64_t*>(base + kSlotOffset); }
inline char* ws_scratch(char* base) { return base + kScratchOffset; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Launch helpers that turn a launch failure into a status.
int check_launch(const char* kernel);

// Workspace sizes of the individual operations (bytes after the header).
size_t row_sum_max_workspace(int64_t rows, int64_t cols, int variant, int split,
                             int cu_count);
size_t ffn_workspace(int64_t rows, int64_t ffn_dim);
size_t ffn_bwd_workspace(int64_t rows, int64_t d, int64_t ffn_dim);
size_t layernorm_bwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int elem_bytes, int cu_count);
size_t softmax_workspace(int op, int64_t rows, int64_t cols, int variant, int split,
                         int cu_count);
size_t rmsnorm_fwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t layernorm_fwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t rowwise_quant_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t lars_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t wvar_bwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t pearson_bwd_workspace(int64_t rows, int64_t cols, int variant, int split, int cu_count);
size_t rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int variant, int split,
                             int cu_count);
size_t rmsnorm_fused_workspace(int64_t rows, int64_t cols, int variant, int split,
                               int cu_count);

// CU count of the current device, or 256 (MI355X) when none is visible.
int cu_count_or_default();

}  // namespace credit
