// Host-only check of the library's per-(device, stream) workspace cache
// (credit_amd/csrc/workspace_cache.hpp) with a recording allocator: keying,
// growth, retirement (never freeing a pointer a caller may hold) and a
// failing allocation.  Built with g++ by tests/test_workspace_cache.py.
#include <stdio.h>
#include <stdlib.h>

#include <thread>
#include <vector>

#include "../../credit_amd/csrc/workspace_cache.hpp"

struct FakeAlloc {
  std::vector<size_t>* sizes;
  bool* fail;
  int operator()(int, void*, size_t bytes, char** out) const {
    if (*fail) return -6;
    sizes->push_back(bytes);
    *out = static_cast<char*>(malloc(bytes));
    return 0;
  }
};

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      fprintf(stderr, "FAILED line %d: %s\n", __LINE__, #c);       \
      return 1;                                                    \
    }                                                              \
  } while (0)

int main() {
  std::vector<size_t> sizes;
  bool fail = false;
  credit::WorkspaceCache<FakeAlloc> cache(FakeAlloc{&sizes, &fail});
  void* s1 = reinterpret_cast<void*>(0x1000);
  void* s2 = reinterpret_cast<void*>(0x2000);
  char *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;
  // Distinct (device, stream) keys get distinct buffers; the same key the same one.
  CHECK(cache.get(0, s1, 100, &a) == 0);
  CHECK(cache.get(0, s2, 100, &b) == 0);
  CHECK(cache.get(1, s1, 100, &c) == 0);
  CHECK(a != b && a != c && b != c);
  CHECK(cache.get(0, s1, 5000, &d) == 0 && d == a);  // fits the 1 MiB minimum
  CHECK(sizes.size() == 3 && sizes[0] == (size_t{1} << 20));
  CHECK(cache.peek(0, s2) == b && cache.peek(0, nullptr) == nullptr);
  // Growth: at least double, rounded to 1 MiB; the old buffer is retired, not freed.
  char* e = nullptr;
  CHECK(cache.get(0, s1, (size_t{1} << 20) + 1, &e) == 0);
  CHECK(e != a && sizes.back() == (size_t{2} << 20));
  CHECK(cache.retired_count() == 1);
  CHECK(cache.get(0, s1, (size_t{5} << 20) + 3, &e) == 0 && sizes.back() == (size_t{6} << 20));
  CHECK(cache.retired_count() == 2);
  a[0] = 1;  // still owned: a retired buffer stays valid for its holders
  // A failing allocation reports its status and keeps the old buffer.
  fail = true;
  char* f = nullptr;
  CHECK(cache.get(0, s1, size_t{64} << 20, &f) == -6 && f == nullptr);
  CHECK(cache.peek(0, s1) == e);
  fail = false;
  // Concurrent first use of one key from several threads yields one buffer.
  void* s3 = reinterpret_cast<void*>(0x3000);
  std::vector<char*> got(8, nullptr);
  std::vector<std::thread> ts;
  for (int i = 0; i < 8; ++i)
    ts.emplace_back([&, i] { cache.get(2, s3, 4096, &got[i]); });
  for (auto& t : ts) t.join();
  for (int i = 1; i < 8; ++i) CHECK(got[i] == got[0] && got[0] != nullptr);
  CHECK(cache.live().size() == 4);
  printf("workspace cache: ok\n");
  return 0;
}
