// CPU unit test of the arena's free-list rules (vearo_amd/csrc/arena.h) with a
// fake device that logs every allocation, event record and stream wait.
// Built and run by tests/test_arena_cpu.py; exits non-zero on the first failure.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "arena.h"

namespace {
int g_fail = 0;
#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);     \
      ++g_fail;                                                    \
    }                                                              \
  } while (0)

struct FakeEvent {
  int stream;  // stream it was recorded on
  int seq;     // record order
};

struct FakeDev {
  using Stream = const void*;
  using Event = FakeEvent*;
  std::vector<std::string> log;
  int next = 0x1000, records = 0, mallocs = 0, frees = 0;
  bool fail_malloc = false;
  std::vector<Event> released;
  std::vector<FakeEvent> store = std::vector<FakeEvent>(64);  // owns the events (no reallocation)

  static int id(Stream s) { return (int)(reinterpret_cast<uintptr_t>(s) & 0xff); }
  int dev_malloc(void** p, size_t r) {
    if (fail_malloc) return 1;
    *p = reinterpret_cast<void*>((uintptr_t)next);
    next += (int)r;
    ++mallocs;
    log.push_back("malloc " + std::to_string(r));
    return 0;
  }
  int dev_free(void*) {
    ++frees;
    log.push_back("free");
    return 0;
  }
  Event record(Stream s) {
    ++records;
    log.push_back("record " + std::to_string(id(s)));
    store[(size_t)records] = FakeEvent{id(s), records};
    return &store[(size_t)records];
  }
  int stream_wait(Stream s, Event e) {
    log.push_back("wait " + std::to_string(id(s)) + " on " + std::to_string(e->stream));
    return 0;
  }
  void release(Event e) { released.push_back(e); }
  bool persistent(Stream s) { return id(s) == 1; }
};

const void* S(int i) { return reinterpret_cast<const void*>((uintptr_t)i); }
// Stream 1 is the persistent (runtime) stream; 2 and 3 are caller streams.

void test_same_stream_reuse_is_immediate() {
  ArenaCore<FakeDev> a;
  void *p, *q;
  CHECK(a.alloc(1000, S(1), &p) == 0);
  CHECK(a.free(p, S(1)) == 0);
  CHECK(a.dev.records == 0);  // persistent stream: nothing recorded at the free
  CHECK(a.alloc(900, S(1), &q) == 0);  // same rounded size (1024)
  CHECK(q == p);
  CHECK(a.dev.records == 0 && a.dev.mallocs == 1);
  CHECK(a.dev.log.back() == "malloc 1024");
}

void test_runtime_block_to_other_stream_waits_lazily() {
  ArenaCore<FakeDev> a;
  void *p, *q;
  CHECK(a.alloc(4096, S(1), &p) == 0);
  CHECK(a.free(p, S(1)) == 0);
  CHECK(a.alloc(4096, S(2), &q) == 0);
  CHECK(q == p);
  // Recorded at the reuse on the runtime stream, waited on by stream 2.
  const size_t n = a.dev.log.size();
  CHECK(n >= 2 && a.dev.log[n - 2] == "record 1" && a.dev.log[n - 1] == "wait 2 on 1");
  CHECK(a.dev.released.size() == 1);
}

void test_caller_stream_event_recorded_at_free() {
  ArenaCore<FakeDev> a;
  void *p, *q, *r;
  CHECK(a.alloc(5000, S(2), &p) == 0);
  CHECK(a.free(p, S(2)) == 0);
  CHECK(a.dev.records == 1 && a.dev.log.back() == "record 2");
  // Same stream: no wait, the free's event goes back to the pool.
  CHECK(a.alloc(5000, S(2), &q) == 0 && q == p);
  CHECK(a.dev.log.back() == "record 2" && a.dev.released.size() == 1);
  CHECK(a.free(q, S(2)) == 0);
  // Another stream waits on the event recorded at the free (no new record).
  const int rec = a.dev.records;
  CHECK(a.alloc(5000, S(3), &r) == 0 && r == p);
  CHECK(a.dev.records == rec && a.dev.log.back() == "wait 3 on 2");
}

void test_prefers_block_of_the_requesting_stream() {
  ArenaCore<FakeDev> a;
  void *p2, *p3, *q;
  CHECK(a.alloc(2048, S(2), &p2) == 0);
  CHECK(a.alloc(2048, S(3), &p3) == 0);
  CHECK(p2 != p3);
  CHECK(a.free(p2, S(2)) == 0);
  CHECK(a.free(p3, S(3)) == 0);  // most recent
  CHECK(a.alloc(2048, S(2), &q) == 0);
  CHECK(q == p2);  // stream 2's own block, not the most recently freed
  CHECK(a.dev.log.back() == "record 3");  // no wait issued
  CHECK(a.alloc(2048, S(1), &q) == 0 && q == p3);
  CHECK(a.dev.log.back() == "wait 1 on 3");
}

void test_sizes_accounting_and_errors() {
  ArenaCore<FakeDev> a;
  CHECK(ArenaCore<FakeDev>::rounded(0) == 512 && ArenaCore<FakeDev>::rounded(513) == 1024);
  CHECK(ArenaCore<FakeDev>::rounded((1 << 20) + 1) == (size_t(2) << 20));
  void *p, *q;
  CHECK(a.alloc(100, S(1), &p) == 0 && a.alloc(3 << 20, S(1), &q) == 0);
  CHECK(a.live_bytes == 512 + (size_t(4) << 20) && a.peak_bytes == a.live_bytes);
  CHECK(a.free(q, S(1)) == 0);
  CHECK(a.cached_bytes == (size_t(4) << 20) && a.live_bytes == 512);
  CHECK(a.free(q, S(1)) == -1);  // double free
  int x;
  CHECK(a.free(&x, S(1)) == -1);  // not the arena's
  // Out of memory: the cache goes back to the device, then one retry fails.
  a.dev.fail_malloc = true;
  void* r;
  CHECK(a.alloc(64 << 20, S(1), &r) == 2);
  CHECK(a.cached_bytes == 0 && a.dev.frees == 1);
  CHECK(a.dev_bytes == 512);
  a.dev.fail_malloc = false;
  CHECK(a.release_all_cached() == 0);
}
}  // namespace

int main() {
  test_same_stream_reuse_is_immediate();
  test_runtime_block_to_other_stream_waits_lazily();
  test_caller_stream_event_recorded_at_free();
  test_prefers_block_of_the_requesting_stream();
  test_sizes_accounting_and_errors();
  if (g_fail) return 1;
  std::printf("arena tests ok\n");
  return 0;
}
