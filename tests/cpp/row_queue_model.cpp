// Host-threaded model of the row-ticket queue of the group pipelines
// (credit_amd/csrc/common.hpp: queue_ticket_wave, queue_take_row; the
// RMSNorm forward group body in credit_amd/csrc/rmsnorm.hip).  One
// std::thread per row group, a std::atomic word for the launch-wide ticket
// counter, random delays so that groups run at different rates.  Restated
// from the device code:
//   fixed steps   step i < L of group g takes row g + i G (those below rows:
//                 n_fixed of them; fewer than L means the group has no other)
//   draws         at stage k < n the group draws the ticket of step k + L
//                 (one fetch_add of 1); the first ticket t with L G + t >=
//                 rows sets n = k + L
//   rows          step i >= L takes row L G + t_i; the group's steps end at
//                 the first step without a row
//   reset         the draw that returns rows - 1 adds -rows to the counter
// A launch is correct when every row is processed exactly once and the
// counter reads zero afterwards; several launches run back to back on the
// same counter, as calls on one stream do.
//
// Scenarios (argv[1]); each prints "<name>: launches=N wrong=W dup=D
// counter=C" (W rows never processed, D rows processed twice, C the counter
// after the last launch) and exits 0:
//   queue          the library's rules, rows from 1 to 3000 over 8-32 groups
//   no_reset       the same with the reset left out (a planted mistake)
//   extra_draw     the same with one more draw after a group's last stage
//                  (a planted mistake)
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <random>
#include <thread>
#include <vector>

namespace {

constexpr int L = 8;  // the RMSNorm forward pipeline: DEPTH 4 + AHEAD 1 + 3

struct Result {
  int64_t wrong = 0;
  int64_t dup = 0;
};

enum class Mode { kLibrary, kNoReset, kExtraDraw };

void run_group(int g, int G, int rows, Mode mode, std::atomic<uint32_t>* counter,
               std::vector<std::atomic<int>>* seen, uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::uniform_int_distribution<int> pause(0, 40);
  const int r1 = (rows - g + G - 1) / G;
  const int n_fixed = r1 < L ? r1 : L;
  const int64_t first = static_cast<int64_t>(L) * G;
  int n = n_fixed < L ? n_fixed : INT32_MAX;
  std::vector<int> rowid;  // row of step i >= L
  auto row_of = [&](int i) -> int {
    if (i < L) return i < n_fixed ? g + i * G : rows;
    return rowid[i - L];
  };
  const int limit = mode == Mode::kExtraDraw ? 1 : 0;
  for (int k = 0; k < n + limit; ++k) {
    // The ticket wave: the draw for step k + L, and the reset after the
    // launch's last draw.
    const uint32_t t = counter->fetch_add(1u);
    const int64_t r = first + t;
    if (k < n) {
      rowid.push_back(r < rows ? static_cast<int>(r) : rows);
      if (r >= rows && n == INT32_MAX) n = k + L;
    }
    if (mode != Mode::kNoReset && t == static_cast<uint32_t>(rows - 1))
      counter->fetch_sub(static_cast<uint32_t>(rows));
    // The data waves finish step k (it has a row: k < n).
    if (k < n) {
      const int row = row_of(k);
      if (row < 0 || row >= rows) {
        fprintf(stderr, "group %d step %d: row %d out of range\n", g, k, row);
        return;
      }
      (*seen)[row].fetch_add(1);
    }
    std::this_thread::sleep_for(std::chrono::microseconds(pause(rng)));
  }
}

Result launch(int rows, int G, Mode mode, std::atomic<uint32_t>* counter, uint64_t seed) {
  std::vector<std::atomic<int>> seen(rows);
  for (auto& s : seen) s.store(0);
  std::vector<std::thread> threads;
  // Groups beyond the rows (padding) draw nothing.
  const int active = G < rows ? G : rows;
  for (int g = 0; g < active; ++g)
    threads.emplace_back(run_group, g, G, rows, mode, counter, &seen, seed * 1000003u + g);
  for (auto& t : threads) t.join();
  Result res;
  for (auto& s : seen) {
    const int v = s.load();
    if (v == 0) ++res.wrong;
    if (v > 1) ++res.dup;
  }
  return res;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s queue|no_reset|extra_draw\n", argv[0]);
    return 2;
  }
  const char* name = argv[1];
  Mode mode;
  if (!strcmp(name, "queue")) mode = Mode::kLibrary;
  else if (!strcmp(name, "no_reset")) mode = Mode::kNoReset;
  else if (!strcmp(name, "extra_draw")) mode = Mode::kExtraDraw;
  else {
    fprintf(stderr, "unknown scenario %s\n", name);
    return 2;
  }
  std::atomic<uint32_t> counter{0};
  const int shapes[][2] = {{1, 32},  {7, 32},    {255, 32},  {256, 32}, {257, 32},
                           {300, 8}, {1024, 32}, {1500, 16}, {64, 8},   {3000, 32}};
  Result total;
  int launches = 0;
  for (int rep = 0; rep < 3; ++rep) {
    for (const auto& s : shapes) {
      const Result r = launch(s[0], s[1], mode, &counter, 17u * rep + launches);
      total.wrong += r.wrong;
      total.dup += r.dup;
      ++launches;
    }
  }
  printf("%s: launches=%d wrong=%lld dup=%lld counter=%u\n", name, launches,
         static_cast<long long>(total.wrong), static_cast<long long>(total.dup),
         counter.load());
  return 0;
}
