// arena.h -- the caching arena's bookkeeping, independent of the device API so
// that its reuse rules are unit-tested on the CPU (tests/cpp/test_arena.cpp).
//
// Blocks come from the device allocator in rounded sizes (512 B granularity up
// to 1 MiB, 2 MiB above) and go back to exact-size free lists. A freed block
// remembers the stream its last user queued work on:
//   * reuse on that same stream is immediate: stream order runs the new work
//     after the old;
//   * reuse on another stream first makes the new stream wait (on the device,
//     the host does not block) for an event that marks the old stream's work:
//     recorded at the free for caller streams (which may be destroyed later),
//     or at the reuse for the persistent stream (the runtime's own, alive until
//     shutdown), which then also covers work queued after the free -- a later
//     point, so still safe.
// Among the blocks of one size, one last used on the requesting stream is
// preferred, then the most recently freed.
//
// Dev supplies: using Stream (a pointer-like handle) and Event; int
// dev_malloc(void**, size_t) and int dev_free(void*) (0 = ok); Event
// record(Stream) (a null Event on failure); int stream_wait(Stream, Event);
// void release(Event); bool persistent(Stream).
#pragma once
#include <algorithm>
#include <cstddef>
#include <map>
#include <unordered_map>
#include <vector>

template <class Dev>
struct ArenaCore {
  using Stream = typename Dev::Stream;
  using Event = typename Dev::Event;
  struct Block {
    void* p;
    Stream last;  // stream of the last user's work
    Event ev;     // marks that work (null: record lazily, `last` is persistent)
  };

  Dev dev;
  std::map<size_t, std::vector<Block>> free_lists;
  std::unordered_map<void*, size_t> live;
  size_t live_bytes = 0, cached_bytes = 0, peak_bytes = 0, dev_bytes = 0;

  static size_t rounded(size_t b) {
    if (b == 0) b = 1;
    if (b <= (size_t(1) << 20)) return (b + 511) & ~size_t(511);
    const size_t g = size_t(2) << 20;
    return (b + g - 1) / g * g;
  }

  // 0: ok; 1: a device call failed (the block, if any, stays cached);
  // 2: out of memory even after giving the cache back.
  int alloc(size_t bytes, Stream s, void** out) {
    const size_t r = rounded(bytes);
    void* p = nullptr;
    auto it = free_lists.find(r);
    if (it != free_lists.end() && !it->second.empty()) {
      std::vector<Block>& v = it->second;
      size_t pick = v.size() - 1;
      for (size_t i = v.size(); i-- > 0;)
        if (v[i].last == s) {
          pick = i;
          break;
        }
      Block b = v[pick];
      if (b.last != s) {
        Event ev = b.ev ? b.ev : dev.record(b.last);
        if (!ev) return 1;
        const int rc = dev.stream_wait(s, ev);
        if (ev != b.ev) dev.release(ev);
        if (rc != 0) return 1;
      }
      if (b.ev) dev.release(b.ev);
      v.erase(v.begin() + (std::ptrdiff_t)pick);
      cached_bytes -= r;
      p = b.p;
    } else {
      if (dev.dev_malloc(&p, r) != 0) {
        // Give the cache back to the device and retry once.
        if (release_all_cached() != 0) return 1;
        if (dev.dev_malloc(&p, r) != 0) return 2;
      }
      dev_bytes += r;
    }
    live.emplace(p, r);
    live_bytes += r;
    peak_bytes = std::max(peak_bytes, live_bytes);
    *out = p;
    return 0;
  }

  // 0: ok; -1: not a live block of this arena; 1: the event could not be recorded.
  int free(void* p, Stream s) {
    auto it = live.find(p);
    if (it == live.end()) return -1;
    Event ev{};
    if (!dev.persistent(s)) {
      ev = dev.record(s);
      if (!ev) return 1;
    }
    const size_t r = it->second;
    live.erase(it);
    live_bytes -= r;
    free_lists[r].push_back(Block{p, s, ev});
    cached_bytes += r;
    return 0;
  }

  // Hands every cached block back to the device allocator (which, on HIP,
  // waits for the device first). 0 ok, 1 a device call failed.
  int release_all_cached() {
    for (auto& kv : free_lists) {
      std::vector<Block>& v = kv.second;
      while (!v.empty()) {
        const Block b = v.back();
        if (dev.dev_free(b.p) != 0) return 1;
        if (b.ev) dev.release(b.ev);
        v.pop_back();
        dev_bytes -= kv.first;
        cached_bytes -= kv.first;
      }
    }
    free_lists.clear();
    return 0;
  }
};
