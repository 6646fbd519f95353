// Host-threaded model of the split-row protocol (credit_amd/csrc/common.hpp):
// one std::thread per workgroup, std::atomic words for the ticket
// dispensers, the tagged exchange slots, the exit counts and the workspace's
// tag sequence.  The integer rules -- tickets to (group, member), the number
// of dispenser subsets, tag and sequence arithmetic -- are the library's own
// (credit_amd/csrc/split_plan.hpp, included here); the rest restates the
// device code step by step:
//   split_join   seq read, ticket draw, seat_of, last ticket resets the dispenser
//   rows         group g takes rows g, g + G, ... (the group kernels' deal)
//   publish      one 64-bit store: tag << 32 | value, slot [group][stage % ring][member]
//   poll         until every member's slot carries the stage's tag; bounded, and
//                on expiry the watchdog is raised and the wait gives up
//   split_leave  subset exit count, launch exit count, the last advances seq
//                (clearing the slot area when it wraps)
// A workgroup runs on XCD (b + start) % xcds and starts only when its XCD has
// a free slot, in blockIdx order per XCD (the dispatcher); a slot can be
// withheld from the launch for a while or for the whole launch, and pending
// workgroups can be started late.  Every wait in the model is bounded, so
// every scenario ends.
//
// Scenarios (argv[1]); each prints "<name>: watchdog=W wrong=R" and exits 0:
//   withheld_old   one slot of XCD 0 withheld for the whole launch; the old
//                  sizing: 8 subsets, one group spanning every slot of each
//                  (C4 backward AUTO: 32 members, one workgroup per CU)
//   withheld_new   the same launch and withheld slot under plan::dispensers_for
//   late_new       workgroups ask to start in random order, a slot is
//                  withheld and the workgroup left pending starts late
//   ring_ok        members publish DEPTH stages ahead; ring = 2 DEPTH
//   ring_short     the same with ring = 2 DEPTH - 1: a slot is overwritten
//                  before a slow member polled it (member 1 of group 0 polls
//                  every stage late)
//   replay_host    a captured launch replayed with new inputs, tags fixed on
//                  the host at capture (the protocol before the sequence word)
//   replay_device  the same with the device-side sequence word
//   wrap           the sequence at its limit: the wrapping launch clears the
//                  slot area, so planted stale tags are never taken
//   wrap_noclear   the same with the clear left out (a planted mistake)
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

#define CREDIT_HD
#include "../../credit_amd/csrc/split_plan.hpp"

namespace plan = credit::plan;
using Clock = std::chrono::steady_clock;

// ------------------------------------------------------------ the device --
struct Dispatcher {
  int xcds;
  int start;                       // XCD of workgroup 0
  std::vector<int> free_slots;     // per XCD
  std::vector<uint32_t> next;      // next blockIdx position to start, per XCD
  std::mutex mu;
  std::condition_variable cv;
  int late_us = 0;                 // random delay (0 .. late_us) before a workgroup asks to start
  int pending_late_ms = 0;         // a workgroup that had to wait for a slot starts this late

  Dispatcher(int x, int slots, int s) : xcds(x), start(s), free_slots(x, slots), next(x, 0) {}
  int xcd_of(uint32_t b) const { return static_cast<int>((b + start) % xcds); }
  // Blocks until workgroup b may start: its turn on its XCD and a free slot.
  // Bounded: gives up (returns false) after `limit`.
  bool acquire(uint32_t b, std::chrono::milliseconds limit) {
    const int x = xcd_of(b);
    const uint32_t pos = b / xcds;
    std::unique_lock<std::mutex> lk(mu);
    auto ready = [&] { return next[x] == pos && free_slots[x] > 0; };
    const bool pending = !ready();
    if (!cv.wait_for(lk, limit, ready)) return false;
    --free_slots[x];
    ++next[x];
    cv.notify_all();
    if (pending && pending_late_ms) {
      lk.unlock();
      std::this_thread::sleep_for(std::chrono::milliseconds(pending_late_ms));
    }
    return true;
  }
  void release(uint32_t b) {
    std::lock_guard<std::mutex> lk(mu);
    ++free_slots[xcd_of(b)];
    cv.notify_all();
  }
  // A new launch: its workgroups start from position 0 on every XCD.
  void new_launch() {
    std::lock_guard<std::mutex> lk(mu);
    std::fill(next.begin(), next.end(), 0u);
  }
  void withhold(int x, int n) {
    std::lock_guard<std::mutex> lk(mu);
    free_slots[x] -= n;
  }
  void give_back(int x, int n) {
    std::lock_guard<std::mutex> lk(mu);
    free_slots[x] += n;
    cv.notify_all();
  }
};

// ---------------------------------------------------------- the workspace --
constexpr int kDispenserStride = 16;
constexpr size_t kSlotWords = 1 << 16;
struct Workspace {
  std::atomic<uint32_t> watchdog{0};
  std::atomic<uint32_t> seq{0};
  std::atomic<uint32_t> launch_out{0};
  std::atomic<uint32_t> counters[plan::kMaxDispensers * kDispenserStride];
  std::unique_ptr<std::atomic<uint64_t>[]> slots{new std::atomic<uint64_t>[kSlotWords]};
  Workspace() {
    for (auto& c : counters) c.store(0);
    for (size_t i = 0; i < kSlotWords; ++i) slots[i].store(0);
  }
};

struct Launch {
  uint32_t grid;
  int members;
  int dispensers;
  int ring;
  int rows;
  int depth = 1;               // stages a member publishes ahead of its poll
  bool host_epoch = false;     // tags fixed by the caller (the old protocol)
  uint32_t epoch = 0;          // the caller's epoch when host_epoch
  uint64_t input = 1;          // input generation: partials depend on it
  int slow_publish_us = 0;     // member 1 of group 0 publishes this late
  int slow_poll_us = 0;        // member 1 of group 0 polls this late
  bool clear_on_wrap = true;   // false: the wrapping launch leaves the slots
  std::chrono::milliseconds spin_limit{1500};
};

struct Outcome {
  std::atomic<int> wrong{0};
  std::atomic<int> expired{0};
};

// Member m's partial of row r for input generation `in` (small integers, so
// sums are exact in any order).
uint32_t partial(int row, int member, uint64_t in) {
  return static_cast<uint32_t>((row * 131 + member * 7 + in * 1009) % 1000);
}

void workgroup(uint32_t b, const Launch& L, Workspace& ws, Dispatcher& dev, Outcome& out) {
  if (dev.late_us) {
    std::mt19937 rng(b);
    std::this_thread::sleep_for(std::chrono::microseconds(rng() % (dev.late_us + 1)));
  }
  if (!dev.acquire(b, L.spin_limit * 4)) {  // never started: the launch is stuck
    out.expired++;
    return;
  }
  // split_join
  const uint32_t seq = ws.seq.load();
  const uint32_t subset = b % static_cast<uint32_t>(L.dispensers);
  const uint32_t per_subset = L.grid / static_cast<uint32_t>(L.dispensers);
  std::atomic<uint32_t>& dispenser = ws.counters[subset * kDispenserStride];
  const uint32_t t = dispenser.fetch_add(1);
  if (t == per_subset - 1) dispenser.store(0);
  const plan::Seat seat = plan::seat_of(b, t, L.grid, static_cast<uint32_t>(L.dispensers),
                                        static_cast<uint32_t>(L.members));
  const uint32_t epoch = L.host_epoch ? L.epoch : plan::launch_epoch(seq);
  const int G = static_cast<int>(L.grid) / L.members;
  const size_t group_base = static_cast<size_t>(seat.group) * L.ring * L.members;

  // The group's rows, dealt round-robin; stage i is the group's i-th row.
  std::vector<int> rows;
  for (int r = seat.group; r < L.rows; r += G) rows.push_back(r);
  const int n = static_cast<int>(rows.size());
  auto publish = [&](int stage) {
    if (seat.group == 0 && seat.member == 1 && L.slow_publish_us)
      std::this_thread::sleep_for(std::chrono::microseconds(L.slow_publish_us));
    const uint64_t word = (static_cast<uint64_t>(plan::stage_tag(epoch, stage)) << 32) |
                          partial(rows[stage], seat.member, L.input);
    ws.slots[group_base + static_cast<size_t>(stage % L.ring) * L.members + seat.member].store(
        word);
  };
  bool gave_up = false;
  for (int s = 0; s < std::min(L.depth, n); ++s) publish(s);
  for (int s = 0; s < n && !gave_up; ++s) {
    if (seat.group == 0 && seat.member == 1 && L.slow_poll_us)
      std::this_thread::sleep_for(std::chrono::microseconds(L.slow_poll_us));
    const uint32_t tag = plan::stage_tag(epoch, s);
    const auto t0 = Clock::now();
    uint64_t sum = 0;
    for (;;) {
      bool all = true;
      sum = 0;
      for (int m = 0; m < L.members; ++m) {
        const uint64_t w =
            ws.slots[group_base + static_cast<size_t>(s % L.ring) * L.members + m].load();
        if (static_cast<uint32_t>(w >> 32) != tag) {
          all = false;
          break;
        }
        sum += static_cast<uint32_t>(w);
      }
      if (all) break;
      if (Clock::now() - t0 > L.spin_limit) {
        ws.watchdog.store(1);
        out.expired++;
        gave_up = true;
        break;
      }
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
    if (gave_up) break;
    uint64_t expect = 0;
    for (int m = 0; m < L.members; ++m) expect += partial(rows[s], m, L.input);
    if (sum != expect) out.wrong++;
    if (s + L.depth < n) publish(s + L.depth);
  }
  // split_leave
  bool clear = false;
  const uint32_t next = plan::advance_seq(seq, static_cast<uint32_t>(
                                                   (L.rows + G - 1) / G), &clear);
  std::atomic<uint32_t>& sub_out = ws.counters[subset * kDispenserStride + 1];
  if (sub_out.fetch_add(1) == per_subset - 1) {
    sub_out.store(0);
    if (ws.launch_out.fetch_add(1) == static_cast<uint32_t>(L.dispensers) - 1) {
      ws.launch_out.store(0);
      if (clear && L.clear_on_wrap)
        for (size_t i = 0; i < kSlotWords; ++i) ws.slots[i].store(0);
      if (!L.host_epoch) ws.seq.store(next);
    }
  }
  dev.release(b);
}

void run(const Launch& L, Workspace& ws, Dispatcher& dev, Outcome& out) {
  dev.new_launch();
  std::vector<std::thread> th;
  th.reserve(L.grid);
  for (uint32_t b = 0; b < L.grid; ++b)
    th.emplace_back(workgroup, b, std::cref(L), std::ref(ws), std::ref(dev), std::ref(out));
  for (auto& t : th) t.join();
}

void report(const char* name, const Outcome& o, const Workspace& ws) {
  printf("%s: watchdog=%u wrong=%d expired=%d seq=%u\n", name, ws.watchdog.load(),
         o.wrong.load(), o.expired.load(), ws.seq.load());
}

// A launch sized the way the library sizes it for `members` on a device of
// xcds x slots resident workgroups (api.hip coresident_groups), or with the
// old rule (8 subsets whatever the members) when `old_rule`.
Launch sized(int xcds, int slots, int members, int rows, bool old_rule) {
  const int64_t resident = static_cast<int64_t>(xcds) * slots;
  Launch L{};
  L.members = members;
  const int64_t groups = plan::coresident_group_count(resident, members);
  L.grid = static_cast<uint32_t>(groups * members);
  L.dispensers = old_rule ? plan::kMaxDispensers : plan::dispensers_for(resident, members);
  L.ring = 16;
  L.rows = rows;
  return L;
}

int main(int argc, char** argv) {
  const std::string sc = argc > 1 ? argv[1] : "";
  Workspace ws;
  Outcome out;
  if (sc == "withheld_old" || sc == "withheld_new") {
    // MI355X at one workgroup per CU: 8 XCDs x 32 slots, 32 members.
    Dispatcher dev(8, 32, 0);
    Launch L = sized(8, 32, 32, 64, sc == "withheld_old");
    L.spin_limit = std::chrono::milliseconds(sc == "withheld_old" ? 300 : 3000);
    dev.withhold(0, 1);  // held by other work for the whole launch
    run(L, ws, dev, out);
    printf("dispensers=%d groups=%u\n", L.dispensers, L.grid / L.members);
  } else if (sc == "late_new") {
    // Workgroups ask to start in random order over 2 ms, a slot of XCD 5 is
    // withheld, and the workgroup left pending starts 100 ms after its slot
    // frees; dispatch starts on XCD 3.
    Dispatcher dev(8, 32, 3);
    dev.late_us = 2000;
    dev.pending_late_ms = 100;
    dev.withhold(5, 1);
    Launch L = sized(8, 32, 32, 64, false);
    run(L, ws, dev, out);
  } else if (sc == "ring_ok" || sc == "ring_short") {
    Dispatcher dev(8, 8, 0);
    Launch L = sized(8, 8, 4, 160, false);
    L.depth = 3;
    L.ring = sc == "ring_ok" ? 2 * L.depth : 2 * L.depth - 1;
    L.slow_poll_us = 3000;  // member 1 of group 0 polls every stage late
    L.spin_limit = std::chrono::milliseconds(500);
    run(L, ws, dev, out);
  } else if (sc == "replay_host" || sc == "replay_device") {
    // The same launch replayed three times with new inputs; member 1 of
    // group 0 publishes late, so its group-mates poll before it has written.
    Dispatcher dev(8, 4, 0);
    Launch L = sized(8, 4, 2, 32, false);
    L.host_epoch = sc == "replay_host";
    L.epoch = 1;
    L.slow_publish_us = 2000;
    for (int replay = 0; replay < 3; ++replay) {
      L.input = 1 + static_cast<uint64_t>(replay);
      run(L, ws, dev, out);
    }
  } else if (sc == "wrap" || sc == "wrap_noclear") {
    Dispatcher dev(8, 4, 0);
    Launch L = sized(8, 4, 2, 32, false);
    // Plant, for every group and member, the tags the launch after the wrap
    // polls (stage s: tag 1 + s) with wrong values.
    for (size_t i = 0; i < kSlotWords; ++i) {
      const uint64_t tag = 1 + (i / static_cast<size_t>(L.members)) % L.ring;
      ws.slots[i].store((tag << 32) | 999999u);
    }
    ws.seq.store(plan::kSeqLimit);
    L.clear_on_wrap = sc == "wrap";
    Launch first = L;
    first.rows = 1;  // one group takes a row; the others leave untouched slots
    run(first, ws, dev, out);
    const uint32_t after_first = ws.seq.load();
    run(L, ws, dev, out);
    printf("seq after the wrapping launch=%u\n", after_first);
  } else {
    fprintf(stderr, "unknown scenario %s\n", sc.c_str());
    return 2;
  }
  report(sc.c_str(), out, ws);
  return 0;
}
