// The library's own workspaces for calls that pass no cfg->workspace.
//
// One buffer per (device, stream).  Work on one stream runs in issue order,
// so two calls sharing a buffer never overlap on the GPU; calls on different
// streams get different buffers and cannot race on partials, tickets or the
// FFN's hidden activation.  When a call needs more than its stream's buffer
// holds, a larger one (at least twice the old size) replaces it and the old
// one is retired, not freed: work queued earlier on that stream, or a call
// on another host thread that already took the old pointer, may still use
// it.  Retired buffers are released only when the process ends (doubling
// bounds them by the live size).  The allocation policy is a template
// parameter so the bookkeeping is testable without a GPU.
#pragma once

#include <stddef.h>

#include <mutex>
#include <vector>

namespace credit {

struct WsBuffer {
  char* ptr = nullptr;
  size_t bytes = 0;
};

// Alloc provides  int operator()(int device, void* stream, size_t bytes,
// char** out)  returning 0 on success (and a fresh buffer whose first
// `zeroed prefix` bytes read zero once work on `stream` that follows it
// runs), or a negative status.
template <class Alloc>
class WorkspaceCache {
 public:
  explicit WorkspaceCache(Alloc alloc = Alloc()) : alloc_(alloc) {}

  // The buffer of (device, stream), grown to at least `need` bytes.
  int get(int device, void* stream, size_t need, char** out) {
    std::lock_guard<std::mutex> lock(mu_);
    Entry* e = find(device, stream);
    if (e == nullptr) {
      entries_.push_back(Entry{device, stream, WsBuffer{}});
      e = &entries_.back();
    }
    if (e->buf.bytes < need) {
      size_t grow = round_up(need);
      if (grow < 2 * e->buf.bytes) grow = 2 * e->buf.bytes;
      char* p = nullptr;
      const int status = alloc_(device, stream, grow, &p);
      if (status != 0) return status;
      if (e->buf.ptr != nullptr) retired_.push_back(e->buf);
      e->buf = WsBuffer{p, grow};
    }
    *out = e->buf.ptr;
    return 0;
  }

  // The buffer of (device, stream) if one exists (no allocation).
  char* peek(int device, void* stream) {
    std::lock_guard<std::mutex> lock(mu_);
    Entry* e = find(device, stream);
    return e == nullptr ? nullptr : e->buf.ptr;
  }

  // Every live buffer (for maintenance that must reach all of them).
  std::vector<WsBuffer> live() {
    std::lock_guard<std::mutex> lock(mu_);
    std::vector<WsBuffer> out;
    for (const Entry& e : entries_) out.push_back(e.buf);
    return out;
  }

  size_t retired_count() {
    std::lock_guard<std::mutex> lock(mu_);
    return retired_.size();
  }

 private:
  struct Entry {
    int device;
    void* stream;
    WsBuffer buf;
  };
  static size_t round_up(size_t v) {
    constexpr size_t kMiB = size_t{1} << 20;
    return (v < kMiB ? kMiB : v + kMiB - 1) / kMiB * kMiB;
  }
  Entry* find(int device, void* stream) {
    for (Entry& e : entries_)
      if (e.device == device && e.stream == stream) return &e;
    return nullptr;
  }

  std::mutex mu_;
  std::vector<Entry> entries_;
  std::vector<WsBuffer> retired_;
  Alloc alloc_;
};

}  // namespace credit
