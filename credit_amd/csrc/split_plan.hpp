// Integer rules of the split-row protocol, shared by the device code
// (common.hpp), the host sizing (api.hip) and the host-threaded model of the
// protocol that the CPU tests build with g++ (tests/cpp/split_protocol_model.cpp).
// Nothing here touches memory: tickets to (group, member), the number of
// dispenser subsets of a launch, and the exchange-tag sequence.
#pragma once

#include <stdint.h>

#ifndef CREDIT_HD
#define CREDIT_HD __host__ __device__
#endif

namespace credit {
namespace plan {

// Ticket dispensers of a split launch: at most 8 (one per XCD: workgroup b
// runs on XCD b % 8), each on its own 64-byte line.
constexpr int kMaxDispensers = 8;

// Dispenser subsets of a launch whose kernel holds `resident` workgroups at
// once on the device, for groups of `members`: the most subsets (8, 4, 2, 1)
// whose resident slots each hold at least two groups.  A group then never
// occupies every slot of its subset, so one slot that is not available to the
// launch (held by other work, or a workgroup the dispatcher starts late)
// delays a group until another group of its subset exits instead of
// stranding it.  0 when even one subset holds fewer than two groups.
CREDIT_HD inline int dispensers_for(int64_t resident, int members) {
  if (members <= 0) return 0;
  for (int d = kMaxDispensers; d >= 1; d /= 2)
    if (resident / d >= 2 * static_cast<int64_t>(members)) return d;
  return 0;
}

// Groups of a co-resident launch: as many as the resident slots hold, a
// multiple of kMaxDispensers (so also of any dispenser count above).
CREDIT_HD inline int64_t coresident_group_count(int64_t resident, int members) {
  if (members <= 0) return 0;
  return resident / (static_cast<int64_t>(kMaxDispensers) * members) * kMaxDispensers;
}

// Ticket `ticket` of the subset of workgroup `block` makes it member
// ticket % P of group subset * (subset size / P) + ticket / P.  `grid` is a
// multiple of dispensers * members.
struct Seat {
  int group;
  int member;
};
CREDIT_HD inline Seat seat_of(uint32_t block, uint32_t ticket, uint32_t grid, uint32_t dispensers,
                              uint32_t members) {
  const uint32_t subset = block % dispensers;
  const uint32_t per_subset = grid / dispensers;
  return Seat{static_cast<int>(subset * (per_subset / members) + ticket / members),
              static_cast<int>(ticket % members)};
}

// Exchange tags.  The workspace header holds a sequence word `seq`; a launch
// reads it as it starts and tags exchange stage s with seq + 1 + s (never 0,
// the zero-filled state of a fresh workspace).  The last workgroup of the
// launch to exit advances seq by the launch's stage count, so the next launch
// on the workspace -- a later call, or a replay of a captured graph with the
// same arguments -- tags its stages with values no slot holds yet.
constexpr uint32_t kMaxLaunchStages = 1u << 30;
// seq never exceeds this after a launch, so the next launch's tags (at most
// kMaxLaunchStages of them) stay below 2^32.
constexpr uint32_t kSeqLimit = 0xFFFFFFFFu - kMaxLaunchStages;

CREDIT_HD inline uint32_t launch_epoch(uint32_t seq) { return seq + 1u; }
CREDIT_HD inline uint32_t stage_tag(uint32_t epoch, int stage) {
  return epoch + static_cast<uint32_t>(stage);
}
// seq after a launch of `stages` tags.  *clear: the tags restart at 1, so the
// slot area must return to zero before the next launch (an old slot could
// otherwise carry a tag a later stage polls for).
CREDIT_HD inline uint32_t advance_seq(uint32_t seq, uint32_t stages, bool* clear) {
  const uint64_t next = static_cast<uint64_t>(seq) + stages;
  *clear = next > kSeqLimit;
  return *clear ? 0u : static_cast<uint32_t>(next);
}

}  // namespace plan
}  // namespace credit
