// runtime.cpp -- host side of libvearo_hip.so: device init, the gfx950 code
// object loaded with hipModuleLoadData, kernel lookup and launch through
// hipModuleLaunchKernel, the caching arena over hipMalloc, the device error
// record, and every C-ABI entry point declared in include/vearo_hip.h.
//
// Launch shapes are chosen here from the operand sizes, and every shape / size /
// alignment assumption a kernel makes is checked before it is launched.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vearo_hip.h"
#include "vh_kargs.h"
#include "arena.h"
#include "rt_internal.h"

extern "C" const unsigned char vh_code_object_start[];
extern "C" const unsigned char vh_code_object_end[];

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

#define VH_HIP(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(VH_ERR_HIP, std::string(#expr) + " failed: " + hipGetErrorString(e_)); \
  } while (0)

#define VH_TRY(expr)        \
  do {                      \
    int rc_ = (expr);       \
    if (rc_ != VH_OK) return rc_; \
  } while (0)

struct Runtime {
  bool ready = false;
  int device = -1;
  int cu_count = 0;
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  VhErrRecord* err = nullptr;  // device memory
  std::mutex fn_mu;
  std::unordered_map<std::string, hipFunction_t> fns;
};

Runtime g_rt;
std::mutex g_init_mu;

hipStream_t S(void* s) { return s ? static_cast<hipStream_t>(s) : g_rt.stream; }

int require_init() {
  if (!g_rt.ready) return fail(VH_ERR_NOT_INIT, "vh_init has not been called");
  return VH_OK;
}

int get_fn(const std::string& name, hipFunction_t* out) {
  std::lock_guard<std::mutex> lk(g_rt.fn_mu);
  auto it = g_rt.fns.find(name);
  if (it != g_rt.fns.end()) {
    *out = it->second;
    return VH_OK;
  }
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, g_rt.module, name.c_str());
  if (e != hipSuccess)
    return fail(VH_ERR_HIP, "kernel " + name + " not found in code object: " + hipGetErrorString(e));
  g_rt.fns.emplace(name, f);
  *out = f;
  return VH_OK;
}

// Grid sizes arrive as 64-bit counts so that none is narrowed on the way: a
// launch whose x dimension reaches 2^32 work-items (the dispatch packet's
// limit), or whose y / z exceed 32 bits, is refused rather than truncated.
template <typename A>
int launch(const std::string& name, int64_t gx, int64_t gy, unsigned block, unsigned shmem,
           hipStream_t s, A args, int64_t gz = 1) {
  if (gx <= 0 || gy <= 0 || gz <= 0) return VH_OK;
  if (gx * (int64_t)block > (int64_t)UINT32_MAX || gy > (int64_t)UINT32_MAX || gz > (int64_t)UINT32_MAX)
    return fail(VH_ERR_UNSUPPORTED, "kernel " + name + ": grid too large for one launch");
  hipFunction_t f;
  VH_TRY(get_fn(name, &f));
  void* params[] = {&args};
  VH_HIP(hipModuleLaunchKernel(f, (unsigned)gx, (unsigned)gy, (unsigned)gz, block, 1, 1, shmem, s, params, nullptr));
  return VH_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ arena --
// The caching arena: free-list bookkeeping and reuse rules in arena.h, device
// calls here. A freed block is reused at once on the stream its last user
// queued work on, and on any other stream only after that stream waits for an
// event marking the work (hipStreamWaitEvent: the device waits, the host does
// not). Events come from a small pool.
struct HipArenaDev {
  using Stream = hipStream_t;
  using Event = hipEvent_t;
  std::vector<hipEvent_t> pool;
  int dev_malloc(void** p, size_t r) {
    if (hipMalloc(p, r) == hipSuccess) return 0;
    (void)hipGetLastError();
    return 1;
  }
  int dev_free(void* p) { return hipFree(p) == hipSuccess ? 0 : 1; }
  Event record(Stream s) {
    hipEvent_t e = nullptr;
    if (!pool.empty()) {
      e = pool.back();
      pool.pop_back();
    } else if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      return nullptr;
    }
    if (hipEventRecord(e, s) != hipSuccess) {
      (void)hipEventDestroy(e);
      return nullptr;
    }
    return e;
  }
  int stream_wait(Stream s, Event e) { return hipStreamWaitEvent(s, e, 0) == hipSuccess ? 0 : 1; }
  void release(Event e) { pool.push_back(e); }
  bool persistent(Stream s) { return s == g_rt.stream; }
  void destroy_pool() {
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    pool.clear();
  }
};

struct Arena {
  std::mutex mu;
  ArenaCore<HipArenaDev> core;

  static size_t rounded(size_t b) { return ArenaCore<HipArenaDev>::rounded(b); }

  // A block of at least `bytes` for work queued on stream s.
  int alloc(size_t bytes, hipStream_t s, void** out) {
    std::lock_guard<std::mutex> lk(mu);
    const int rc = core.alloc(bytes, s, out);
    if (rc == 1) return fail(VH_ERR_HIP, "arena: a device call failed while allocating " + std::to_string(bytes) +
                                             " bytes");
    if (rc == 2)
      return fail(VH_ERR_OOM, "hipMalloc of " + std::to_string(rounded(bytes)) + " bytes failed");
    return VH_OK;
  }

  // Returns p, last used by work queued on stream s.
  int free(void* p, hipStream_t s) {
    std::lock_guard<std::mutex> lk(mu);
    const int rc = core.free(p, s);
    if (rc < 0) return fail(VH_ERR_INVALID, "vh_free: pointer not allocated by vh_alloc");
    if (rc > 0) return fail(VH_ERR_HIP, "arena: could not record the freeing stream's event");
    return VH_OK;
  }

  int release_all_cached() {  // caller holds mu
    if (core.release_all_cached() != 0) return fail(VH_ERR_HIP, "hipFree of a cached block failed");
    return VH_OK;
  }
};

Arena g_arena;

// Scratch buffer for one call: the caller's, or a block from the arena that is
// returned when the call's launches are queued (reused in stream order on the
// call's stream, after an event wait on any other).
struct Scratch {
  void* p = nullptr;
  hipStream_t s = nullptr;
  bool owned = false;
  ~Scratch() {
    if (owned && p) g_arena.free(p, s);
  }
  int get(hipStream_t stream, void* user, size_t user_bytes, size_t need) {
    s = stream;
    if (need == 0) return VH_OK;
    if (user) {
      if (user_bytes < need)
        return fail(VH_ERR_INVALID, "scratch buffer too small: need " + std::to_string(need) +
                                        " bytes, got " + std::to_string(user_bytes));
      if (!aligned16(user)) return fail(VH_ERR_INVALID, "scratch buffer must be 16-byte aligned");
      p = user;
      return VH_OK;
    }
    VH_TRY(g_arena.alloc(need, s, &p));
    owned = true;
    return VH_OK;
  }
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int fill(void* p, float value, int64_t n, hipStream_t s) {
  if (n <= 0) return VH_OK;
  FillArgs a{static_cast<float*>(p), n, value};
  const int64_t blocks = std::min<int64_t>(cdiv(cdiv(n, 4), 256), 8192);
  return launch("vh_fill", blocks, 1, 256, 0, s, a);
}

// --------------------------------------------------------- row engine cfg --
constexpr unsigned RW_TEAM_HOST = 1024;  // threads of the streaming wide-row kernels (kernels/rowwide.h)
struct RowCfg {
  int team, nv, vw;
  int rpw = 1;        // rows per team (forward kernels)
  int bs = 0;         // workgroup size (0: max(team, 256))
  bool full = false;  // a "_f" form: every unit of the row live, no bounds tests
};

// Rows per team for short rows (wave or sub-wave teams holding <= 4 units per
// lane): chosen from kernel timings on MI355X at the GPT-2 shapes.
constexpr int kLnFwdRpw = 4;
constexpr int kSmFwdRpw = 1;
constexpr int kSmBwdRpw = 1;

const int kNV[] = {1, 2, 3, 4, 6, 8, 12, 16};

int pick_nv(int64_t need, int cap) {
  for (int v : kNV)
    if (v >= need && v <= cap) return v;
  return -1;
}

// Units of VW floats per row: TEAM 16/32 for short rows, a wave64 up to 64*cap
// units, a 1024-thread workgroup up to 1024*cap units.
bool pick_row_cfg(int64_t C, bool vec_ok, int cap, RowCfg* out) {
  const int vw = (vec_ok && C % 4 == 0) ? 4 : 1;
  const int64_t U = C / vw;
  if (U <= 16) {
    *out = {16, 1, vw};
    return true;
  }
  if (U <= 32) {
    *out = {32, 1, vw};
    return true;
  }
  int nv = pick_nv(cdiv(U, 64), cap);
  if (nv > 0) {
    *out = {64, nv, vw};
    return true;
  }
  nv = pick_nv(cdiv(U, 1024), cap);
  if (nv > 0) {
    *out = {1024, nv, vw};
    return true;
  }
  return false;
}

int block_of(const RowCfg& c) { return c.bs ? c.bs : (c.team > 256 ? c.team : 256); }

std::string row_base(const char* base, const RowCfg& c) {
  return std::string(base) + "_t" + std::to_string(c.team) + "_n" + std::to_string(c.nv) + "_v" +
         std::to_string(c.vw);
}
// Forward kernels carry the rows-per-team suffix, backward LayerNorm the block size.
std::string fwd_kernel(const char* base, const RowCfg& c) {
  return row_base(base, c) + "_r" + std::to_string(c.rpw) + (c.full ? "_f" : "");
}
std::string bwd_kernel(const char* base, const RowCfg& c) {
  return row_base(base, c) + "_b" + std::to_string(block_of(c)) + (c.full ? "_f" : "");
}
// The LayerNorm kernels come in full-row forms for wave teams of 128-bit
// units with up to 4 units per lane when C fills them exactly.
void set_ln_full(RowCfg* c, int64_t C) {
  c->full = c->team == 64 && c->vw == 4 && c->nv <= 4 && C == (int64_t)c->team * c->nv * c->vw;
}

// Multi-row variants exist for teams <= 64 lanes holding <= 4 units per lane.
void set_rpw(RowCfg* c, int rpw) { c->rpw = (c->team <= 64 && c->nv <= 4) ? rpw : 1; }
// LayerNorm backward runs wave teams of short rows 8 to a 512-thread workgroup,
// one workgroup per CU: at [16384, 768] (cold caches, MI355X) 29.0 us against
// 30.7 us for 16 teams per CU and 33.3 us with the next row loaded during each
// row's arithmetic -- fewer rows in flight stream this pattern faster.
void set_ln_bwd_bs(RowCfg* c) { c->bs = (c->team == 64 && c->nv <= 4) ? 512 : 0; }

// LayerNorm backward workgroup count: fixed caps (independent of the device) so
// the scratch size and the reduction order depend on (rows, C) only.
int64_t ln_bwd_blocks(int64_t rows, const RowCfg& c) {
  const int groups = block_of(c) / c.team;
  const int64_t cap = block_of(c) >= 512 ? 256 : 1024;
  int64_t G = std::min<int64_t>(cdiv(rows, groups), cap);
  if (G < 1) G = 1;
  const int64_t rpb = cdiv(rows, G);
  return cdiv(rows, rpb);
}

int64_t gb_blocks(int64_t rows) { return std::max<int64_t>(1, std::min<int64_t>(rows, 1024)); }

// ----------------------------------------------------- device error record --
std::string fmt_f32(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  char buf[128];
  auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::fixed);
  return std::string(buf, r.ptr);
}

unsigned long long round_usize(float v) {
  const float r = std::round(v);
  if (!(r > 0.0f)) return 0;
  if ((double)r >= 18446744073709551616.0) return ~0ull;
  return (unsigned long long)r;
}

int check_error_record() {
  VhErrRecord h;
  VH_HIP(hipStreamSynchronize(g_rt.stream));
  VH_HIP(hipMemcpy(&h, g_rt.err, sizeof h, hipMemcpyDeviceToHost));
  if (h.token == VH_ERR_NONE && h.target == VH_ERR_NONE) return VH_OK;
  VhErrRecord clean{VH_ERR_NONE, VH_ERR_NONE, 0, 0};
  VH_HIP(hipMemcpy(g_rt.err, &clean, sizeof clean, hipMemcpyHostToDevice));
  auto value_of = [](unsigned long long packed) {
    uint32_t bits = (uint32_t)(packed & 0xFFFFFFFFu);
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
  };
  if (h.token != VH_ERR_NONE) {
    const float v = value_of(h.token);
    if (!(v >= 0.0f)) return fail(VH_ERR_DEVICE_PANIC, "Token ID cannot be negative: " + fmt_f32(v));
    return fail(VH_ERR_DEVICE_PANIC, "Token ID " + std::to_string(round_usize(v)) +
                                         " out of vocabulary bound " + std::to_string(h.token_bound));
  }
  const float v = value_of(h.target);
  if (!(v >= 0.0f)) return fail(VH_ERR_DEVICE_PANIC, "Target class cannot be negative: " + fmt_f32(v));
  return fail(VH_ERR_DEVICE_PANIC, "Target class " + std::to_string(round_usize(v)) +
                                       " out of vocab bounds " + std::to_string(h.target_bound));
}

StridedLayout to_kl(const vh_layout& l) {
  StridedLayout k{};
  k.rank = l.rank;
  for (int i = 0; i < l.rank; ++i) {
    k.dims[i] = l.dims[i];
    k.strides[i] = l.strides[i];
  }
  return k;
}

int check_layout(const vh_layout* l, const char* what) {
  if (!l) return fail(VH_ERR_INVALID, std::string(what) + ": null layout");
  if (l->rank < 0 || l->rank > VH_MAX_RANK)
    return fail(VH_ERR_INVALID, std::string(what) + ": rank must be in [0, 8]");
  for (int i = 0; i < l->rank; ++i)
    if (l->dims[i] < 0 || l->strides[i] < 0)
      return fail(VH_ERR_INVALID, std::string(what) + ": negative dim or stride");
  return VH_OK;
}

int64_t numel(const vh_layout* l) {
  int64_t n = 1;
  for (int i = 0; i < l->rank; ++i) n *= l->dims[i];
  return n;
}

bool is_contig(const vh_layout* l) {
  int64_t acc = 1;
  for (int i = l->rank - 1; i >= 0; --i) {
    if (l->dims[i] != 1 && l->strides[i] != acc) return false;
    acc *= l->dims[i];
  }
  return true;
}

}  // namespace

namespace vh_rt {
int fail(int code, const std::string& msg) { return ::fail(code, msg); }
int require_init() { return ::require_init(); }
hipStream_t stream_of(void* s) { return S(s); }
}  // namespace vh_rt

// ===================================================================== ABI ==
extern "C" {

int vh_init(int device) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_rt.ready) {
    if (device != g_rt.device)
      return fail(VH_ERR_INVALID, "vh_init: already initialised on device " + std::to_string(g_rt.device));
    return VH_OK;
  }
  int count = 0;
  VH_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(VH_ERR_INVALID, "vh_init: device " + std::to_string(device) + " not present (" +
                                    std::to_string(count) + " devices)");
  VH_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  VH_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(VH_ERR_UNSUPPORTED, std::string("vh_init: code object is built for gfx950, device is ") +
                                        prop.gcnArchName);
  VH_HIP(hipDeviceGetAttribute(&g_rt.cu_count, hipDeviceAttributeMultiprocessorCount, device));
  VH_HIP(hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking));
  VH_HIP(hipModuleLoadData(&g_rt.module, vh_code_object_start));
  void* e = nullptr;
  VH_HIP(hipMalloc(&e, sizeof(VhErrRecord)));
  g_rt.err = static_cast<VhErrRecord*>(e);
  VhErrRecord clean{VH_ERR_NONE, VH_ERR_NONE, 0, 0};
  VH_HIP(hipMemcpy(g_rt.err, &clean, sizeof clean, hipMemcpyHostToDevice));
  VH_TRY(vh_rt::noalloc_setup(device));
  g_rt.device = device;
  g_rt.ready = true;
  return VH_OK;
}

int vh_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (!g_rt.ready) return VH_OK;
  VH_HIP(hipStreamSynchronize(g_rt.stream));
  vh_rt::blaslt_shutdown();
  {
    std::lock_guard<std::mutex> al(g_arena.mu);
    VH_TRY(g_arena.release_all_cached());
    for (auto& kv : g_arena.core.live) (void)hipFree(kv.first);
    g_arena.core.live.clear();
    g_arena.core.live_bytes = 0;
    g_arena.core.dev_bytes = 0;
    g_arena.core.dev.destroy_pool();
  }
  VH_HIP(hipFree(g_rt.err));
  VH_HIP(hipModuleUnload(g_rt.module));
  VH_HIP(hipStreamDestroy(g_rt.stream));
  g_rt.fns.clear();
  g_rt.ready = false;
  g_rt.device = -1;
  return VH_OK;
}

const char* vh_last_error(void) { return g_last_error.c_str(); }

void* vh_stream(void) { return g_rt.stream; }

int vh_device_cu_count(void) { return g_rt.cu_count; }

int vh_sync(void) {
  VH_TRY(require_init());
  return check_error_record();
}

int vh_check_device_error(void) {
  VH_TRY(require_init());
  return check_error_record();
}

int vh_alloc(size_t bytes, int zero, void** out) {
  VH_TRY(require_init());
  if (!out) return fail(VH_ERR_INVALID, "vh_alloc: null out");
  // Blocks handed to callers belong to the runtime stream: vh_h2d / vh_d2h /
  // vh_fill_f32 and every entry given stream = NULL queue on it.
  VH_TRY(g_arena.alloc(bytes, g_rt.stream, out));
  if (zero) VH_TRY(fill(*out, 0.0f, (int64_t)(Arena::rounded(bytes) / 4), g_rt.stream));
  return VH_OK;
}

int vh_free(void* ptr) {
  if (!ptr) return VH_OK;
  VH_TRY(require_init());
  return g_arena.free(ptr, g_rt.stream);
}

int vh_h2d(void* dst, const void* src, size_t bytes) {
  VH_TRY(require_init());
  if (bytes == 0) return VH_OK;
  VH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_rt.stream));
  VH_HIP(hipStreamSynchronize(g_rt.stream));
  return VH_OK;
}

int vh_d2h(void* dst, const void* src, size_t bytes) {
  VH_TRY(require_init());
  if (bytes == 0) return VH_OK;
  VH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_rt.stream));
  VH_HIP(hipStreamSynchronize(g_rt.stream));
  return VH_OK;
}

int vh_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  VH_TRY(require_init());
  if (bytes == 0) return VH_OK;
  // 16-byte aligned copies: the library's streaming copy kernel for the whole
  // units, the runtime's copy for a tail of under 16 bytes.
  const size_t n4 = bytes / 16;
  if (aligned16(dst) && aligned16(src) && n4 > 0 && cdiv((int64_t)n4, 256) <= INT32_MAX) {
    StreamCopyArgs a{static_cast<const float*>(src), static_cast<float*>(dst), (int64_t)n4};
    VH_TRY(launch("vh_stream_copy", cdiv((int64_t)n4, 256), 1, 256, 0, S(stream), a));
    if (bytes == n4 * 16) return VH_OK;
    VH_HIP(hipMemcpyAsync(static_cast<char*>(dst) + n4 * 16, static_cast<const char*>(src) + n4 * 16,
                          bytes - n4 * 16, hipMemcpyDeviceToDevice, S(stream)));
    return VH_OK;
  }
  VH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(stream)));
  return VH_OK;
}

int vh_fill_f32(float* out, float value, int64_t n, void* stream) {
  VH_TRY(require_init());
  if (n < 0 || (n > 0 && !out)) return fail(VH_ERR_INVALID, "vh_fill_f32: bad arguments");
  return fill(out, value, n, S(stream));
}

int vh_math_probe(int32_t which, const float* x, float* y, int64_t n, void* stream) {
  VH_TRY(require_init());
  if (which < VH_MATH_EXP || which > VH_MATH_TANH) return fail(VH_ERR_INVALID, "vh_math_probe: unknown function");
  if (n < 0 || (n > 0 && (!x || !y))) return fail(VH_ERR_INVALID, "vh_math_probe: bad arguments");
  if (n == 0) return VH_OK;
  MathProbeArgs a{x, y, n, which};
  return launch("vh_math_probe", std::min<int64_t>(cdiv(n, 256), 8192), 1, 256, 0, S(stream), a);
}

int vh_mem_stats_get(vh_mem_stats* out) {
  if (!out) return fail(VH_ERR_INVALID, "vh_mem_stats_get: null out");
  std::lock_guard<std::mutex> lk(g_arena.mu);
  out->live_bytes = g_arena.core.live_bytes;
  out->cached_bytes = g_arena.core.cached_bytes;
  out->peak_bytes = g_arena.core.peak_bytes;
  out->hip_bytes = g_arena.core.dev_bytes;
  return VH_OK;
}

int vh_empty_cache(void) {
  VH_TRY(require_init());
  VH_HIP(hipStreamSynchronize(g_rt.stream));
  std::lock_guard<std::mutex> lk(g_arena.mu);
  return g_arena.release_all_cached();
}

// ------------------------------------------------------------- layernorm --

int vh_layernorm_fwd(const float* x, const float* w, const float* b, float* y, int64_t rows,
                     int64_t C, float eps, void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || C < 0) return fail(VH_ERR_INVALID, "vh_layernorm_fwd: negative size");
  if (rows == 0 || C == 0) return VH_OK;
  if (!x || !w || !b || !y) return fail(VH_ERR_INVALID, "vh_layernorm_fwd: null pointer");
  if (C > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_layernorm_fwd: C too large");
  RowCfg c;
  const bool vec = aligned16(x) && aligned16(w) && aligned16(b) && aligned16(y);
  if (!pick_row_cfg(C, vec, 16, &c)) {
    // Longer rows: one workgroup per row streams it (kernels/rowwide.h).
    if (rows > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_layernorm_fwd: too many rows");
    LnFwdArgs a{x, w, b, y, rows, (int32_t)C, eps};
    return launch(std::string("vh_ln_fwd_wide_v") + (vec && C % 4 == 0 ? "4" : "1"), rows, 1, RW_TEAM_HOST,
                  0, S(stream), a);
  }
  set_rpw(&c, kLnFwdRpw);
  set_ln_full(&c, C);
  if (c.full && c.rpw != 4) c.full = false;
  const int bs = block_of(c);
  const int64_t rpb = (int64_t)(bs / c.team) * c.rpw;
  LnFwdArgs a{x, w, b, y, rows, (int32_t)C, eps};
  return launch(fwd_kernel("vh_ln_fwd", c), cdiv(rows, rpb), 1, bs, 0, S(stream), a);
}

}  // extern "C"

namespace {
// The LayerNorm backward plan for (rows, C) and the operands' alignment: the
// row configuration, workgroup count and scratch bytes.
struct LnBwdPlan {
  RowCfg c;
  int64_t G;
  size_t need;
  // Rows too long for the register kernel (or whose register form spills:
  // 1024-thread teams holding more than 16 floats of x per lane): per-row
  // statistics, then G row blocks of rpb rows under column tiles.
  bool wide = false;
  int vw = 1;
  int64_t rpb = 0;
  size_t stats_bytes = 0;
};

int ln_bwd_plan(int64_t rows, int64_t C, bool vec, LnBwdPlan* p) {
  if (!pick_row_cfg(C, vec, 8, &p->c) || (p->c.team == 1024 && p->c.nv * p->c.vw > 16)) {
    if (rows > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_layernorm_bwd: too many rows");
    p->wide = true;
    p->vw = vec && C % 4 == 0 ? 4 : 1;
    const int64_t tiles = cdiv(C / p->vw, 256);
    // About 1024 workgroups (column tiles x row blocks), at most 64 row blocks:
    // the partials and the reduction order depend on (rows, C) only.
    const int64_t want = std::max<int64_t>(1, std::min<int64_t>(64, cdiv(1024, tiles)));
    p->rpb = cdiv(rows, std::min<int64_t>(rows, want));
    p->G = cdiv(rows, p->rpb);
    p->stats_bytes = align256((size_t)rows * 4 * sizeof(float));
    p->need = p->stats_bytes + align256((size_t)p->G * 2 * (size_t)C * sizeof(float));
    return VH_OK;
  }
  set_ln_bwd_bs(&p->c);
  set_ln_full(&p->c, C);
  if (p->c.full && block_of(p->c) != 512) p->c.full = false;
  p->G = ln_bwd_blocks(rows, p->c);
  p->need = align256((size_t)p->G * 2 * (size_t)C * sizeof(float));
  return VH_OK;
}

// Launches the backward with `part` as the partials buffer (at least p.need bytes).
int ln_bwd_launch(const LnBwdPlan& p, const float* x, const float* w, const float* dy, float* dx, float* dw,
                  float* db, int64_t rows, int64_t C, float eps, float* part, hipStream_t s) {
  if (p.wide) {
    float* stats = part;
    float* parts = reinterpret_cast<float*>(reinterpret_cast<char*>(part) + p.stats_bytes);
    LnWideArgs a{x, w, dy, dx, stats, parts, rows, p.rpb, (int32_t)C, eps};
    const std::string v = p.vw == 4 ? "4" : "1";
    VH_TRY(launch("vh_ln_stats_wide_v" + v, rows, 1, RW_TEAM_HOST, 0, s, a));
    VH_TRY(launch("vh_ln_tile_wide_v" + v, cdiv(C / p.vw, 256), p.G, 256, 0, s, a));
    ColReduceArgs r{parts, dw, db, (int32_t)p.G, (int32_t)C, 2};
    return launch("vh_col_reduce", cdiv(C, VH_COLR_COLS), 2, VH_COLR_COLS * 16, 0, s, r);
  }
  const int bs = block_of(p.c);
  const int groups = bs / p.c.team;
  // Full-row forms fold in static LDS; the others in a dynamic pairwise tree.
  const unsigned shmem = (!p.c.full && groups > 1) ? (unsigned)((groups / 2) * 2 * C * sizeof(float)) : 0;
  if (shmem > 64 * 1024) return fail(VH_ERR_UNSUPPORTED, "vh_layernorm_bwd: LDS budget exceeded");
  LnBwdArgs a{x, w, dy, dx, part, rows, (int32_t)C, eps};
  VH_TRY(launch(bwd_kernel("vh_ln_bwd", p.c), p.G, 1, bs, shmem, s, a));
  ColReduceArgs r{part, dw, db, (int32_t)p.G, (int32_t)C, 2};
  return launch("vh_col_reduce", cdiv(C, VH_COLR_COLS), 2, VH_COLR_COLS * 16, 0, s, r);
}

// Argument checks shared by both entries; *done is set when nothing is left
// to launch (C == 0, or rows == 0 after zero-filling dw and db).
int ln_bwd_check(const char* fn, const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                 int64_t rows, int64_t C, hipStream_t s, bool* done) {
  *done = true;
  if (rows < 0 || C < 0) return fail(VH_ERR_INVALID, std::string(fn) + ": negative size");
  if (C > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, std::string(fn) + ": C too large");
  if (C == 0) return VH_OK;
  if (!dw || !db) return fail(VH_ERR_INVALID, std::string(fn) + ": null pointer");
  if (rows == 0) {  // reference returns zero gradients (cpu:752-758)
    VH_TRY(fill(dw, 0.0f, C, s));
    return fill(db, 0.0f, C, s);
  }
  if (!x || !w || !dy || !dx) return fail(VH_ERR_INVALID, std::string(fn) + ": null pointer");
  *done = false;
  return VH_OK;
}
}  // namespace

extern "C" {

size_t vh_layernorm_bwd_scratch_bytes(int64_t rows, int64_t C) {
  // The largest need over the vector and scalar configurations (the one used
  // depends on operand alignment).
  if (rows <= 0 || C <= 0) return 0;
  size_t need = 0;
  for (bool vec : {true, false}) {
    LnBwdPlan p;
    if (ln_bwd_plan(rows, C, vec, &p) == VH_OK) need = std::max(need, p.need);
  }
  return need;
}

int vh_layernorm_bwd(const float* x, const float* w, const float* dy, float* dx, float* dw,
                     float* db, int64_t rows, int64_t C, float eps, void* scratch,
                     size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  hipStream_t s = S(stream);
  bool done;
  VH_TRY(ln_bwd_check("vh_layernorm_bwd", x, w, dy, dx, dw, db, rows, C, s, &done));
  if (done) return VH_OK;
  const bool vec = aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx);
  LnBwdPlan p;
  VH_TRY(ln_bwd_plan(rows, C, vec, &p));
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, p.need));
  return ln_bwd_launch(p, x, w, dy, dx, dw, db, rows, C, eps, static_cast<float*>(sc.p), s);
}

int vh_layernorm_bwd_noalloc(const float* x, const float* w, const float* dy, float* dx, float* dw,
                             float* db, int64_t rows, int64_t C, float eps, void* stream) {
  VH_TRY(require_init());
  hipStream_t s = S(stream);
  bool done;
  VH_TRY(ln_bwd_check("vh_layernorm_bwd_noalloc", x, w, dy, dx, dw, db, rows, C, s, &done));
  if (done) return VH_OK;
  const bool vec = aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx);
  LnBwdPlan p;
  VH_TRY(ln_bwd_plan(rows, C, vec, &p));
  if (p.need > VH_NOALLOC_SCRATCH_BYTES)
    return fail(VH_ERR_UNSUPPORTED, "vh_layernorm_bwd_noalloc: rows=" + std::to_string(rows) + ", C=" +
                                        std::to_string(C) + " needs " + std::to_string(p.need) +
                                        " bytes of scratch, more than the " +
                                        std::to_string(VH_NOALLOC_SCRATCH_BYTES) +
                                        "-byte device-resident scratch; use vh_layernorm_bwd");
  void* part = vh_rt::noalloc_scratch(g_rt.device);
  if (!part) return fail(VH_ERR_NOT_INIT, "vh_layernorm_bwd_noalloc: device-resident scratch not set up");
  return ln_bwd_launch(p, x, w, dy, dx, dw, db, rows, C, eps, static_cast<float*>(part), s);
}

// ------------------------------------------------------------------ gelu --

static int gelu_flat(const char* base, const float* x, const float* dy, float* y, int64_t n,
                     hipStream_t s) {
  const bool vec = n % 4 == 0 && aligned16(x) && aligned16(y) && (!dy || aligned16(dy));
  const int vw = vec ? 4 : 1;
  EltArgs a{x, nullptr, dy, y, n, 0};
  const int64_t blocks = std::min<int64_t>(cdiv(n / vw, 256), 16384);
  return launch(std::string(base) + (vec ? "_v4" : "_v1"), blocks, 1, 256, 0, s, a);
}

int vh_gelu_fwd(const float* x, float* y, int64_t n, void* stream) {
  VH_TRY(require_init());
  if (n < 0) return fail(VH_ERR_INVALID, "vh_gelu_fwd: negative size");
  if (n == 0) return VH_OK;
  if (!x || !y) return fail(VH_ERR_INVALID, "vh_gelu_fwd: null pointer");
  return gelu_flat("vh_gelu_fwd", x, nullptr, y, n, S(stream));
}

int vh_gelu_grad_mul(const float* x, const float* dy, float* dx, int64_t n, void* stream) {
  VH_TRY(require_init());
  if (n < 0) return fail(VH_ERR_INVALID, "vh_gelu_grad_mul: negative size");
  if (n == 0) return VH_OK;
  if (!x || !dy || !dx) return fail(VH_ERR_INVALID, "vh_gelu_grad_mul: null pointer");
  return gelu_flat("vh_gelu_gradmul", x, dy, dx, n, S(stream));
}

static bool gb_cfg(int64_t C, bool vec, int* nv, int* vw) {
  *vw = (vec && C % 4 == 0) ? 4 : 1;
  *nv = pick_nv(cdiv(C / *vw, 256), 16);
  return *nv > 0;
}

int vh_gelu_bias_fwd(const float* x, const float* bias, float* y, int64_t rows, int64_t C,
                     void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || C < 0) return fail(VH_ERR_INVALID, "vh_gelu_bias_fwd: negative size");
  if (rows == 0 || C == 0) return VH_OK;
  if (!x || !bias || !y) return fail(VH_ERR_INVALID, "vh_gelu_bias_fwd: null pointer");
  if (C > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_gelu_bias_fwd: C too large");
  int nv, vw;
  if (!gb_cfg(C, aligned16(x) && aligned16(bias) && aligned16(y), &nv, &vw)) {
    // Rows wider than a workgroup's registers: 64-unit column tiles by row
    // blocks (the backward's grid), the same bits.
    const int64_t G0 = gb_blocks(rows);
    const int64_t rpb = cdiv(rows, G0);
    GeluBiasBwdArgs a{x, bias, nullptr, y, nullptr, rows, rpb, (int32_t)C};
    return launch("vh_gelu_bias_fwd_tile_v" + std::to_string(vw), cdiv(C / vw, 64), cdiv(rows, rpb), 256, 0,
                  S(stream), a);
  }
  // One row per workgroup: 68.5 us at [16384, 3072] against 80 us for 4096
  // workgroups of 4 rows each (measured; the bias is re-read from L2 per row).
  const int64_t G = std::max<int64_t>(1, std::min<int64_t>(rows, INT32_MAX));
  const int64_t rpb = cdiv(rows, G);
  GeluBiasBwdArgs a{x, bias, nullptr, y, nullptr, rows, rpb, (int32_t)C};
  return launch("vh_gelu_bias_fwd_n" + std::to_string(nv) + "_v" + std::to_string(vw),
                cdiv(rows, rpb), 1, 256, 0, S(stream), a);
}

size_t vh_gelu_bias_bwd_scratch_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return 0;
  return align256((size_t)gb_blocks(rows) * (size_t)C * sizeof(float));
}

int vh_gelu_bias_bwd(const float* x, const float* bias, const float* dy, float* dx, float* dbias,
                     int64_t rows, int64_t C, void* scratch, size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || C < 0) return fail(VH_ERR_INVALID, "vh_gelu_bias_bwd: negative size");
  hipStream_t s = S(stream);
  if (C == 0) return VH_OK;
  if (!dbias) return fail(VH_ERR_INVALID, "vh_gelu_bias_bwd: null pointer");
  if (rows == 0) return fill(dbias, 0.0f, C, s);
  if (!x || !bias || !dy || !dx) return fail(VH_ERR_INVALID, "vh_gelu_bias_bwd: null pointer");
  if (C > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_gelu_bias_bwd: C too large");
  // The column-tile kernel takes any width.
  const int vw = (aligned16(x) && aligned16(bias) && aligned16(dy) && aligned16(dx) && C % 4 == 0) ? 4 : 1;
  const int64_t G0 = gb_blocks(rows);
  const int64_t rpb = cdiv(rows, G0);
  const int64_t G = cdiv(rows, rpb);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, align256((size_t)G0 * (size_t)C * sizeof(float))));
  GeluBiasBwdArgs a{x, bias, dy, dx, static_cast<float*>(sc.p), rows, rpb, (int32_t)C};
  // Grid: 64-unit column tiles by row blocks. At [16384, 3072] 101 us against
  // 122 us for one workgroup walking each row block (measured on MI355X).
  VH_TRY(launch("vh_gelu_bias_bwd_tile_v" + std::to_string(vw), cdiv(C / vw, 64), G, 256,
                0, s, a));
  ColReduceArgs r{static_cast<float*>(sc.p), dbias, nullptr, (int32_t)G, (int32_t)C, 1};
  return launch("vh_col_reduce", cdiv(C, VH_COLR_COLS), 1, VH_COLR_COLS * 16, 0, s, r);
}

// --------------------------------------------------------------- softmax --

// A device flag (vh_attn_decide's verdict) that the attention's products and
// softmax passes read to choose their causal or dense form on the device; set
// for the launches of one attention call on this thread (no host wait for the
// probe's answer).
static thread_local const int32_t* g_causal_flag = nullptr;
struct CausalFlagScope {
  explicit CausalFlagScope(const int32_t* f) { g_causal_flag = f; }
  ~CausalFlagScope() { g_causal_flag = nullptr; }
};

static int softmax_common(const char* base, int cap, int rpw, const float* in, const float* dy,
                          float* out, int64_t rows, int64_t T, int causal, int input_is_x, hipStream_t s,
                          int attn = 0, int ztile = 0) {
  RowCfg c;
  const bool vec = aligned16(in) && aligned16(out) && (!dy || aligned16(dy));
  if (!pick_row_cfg(T, vec, cap, &c)) {
    // Longer rows: one workgroup per row streams it (kernels/rowwide.h).
    if (rows > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, std::string(base) + ": too many rows");
    SoftmaxArgs a{in, dy, out, rows, (int32_t)T, causal ? 1 : 0, input_is_x ? 1 : 0, attn, ztile, g_causal_flag};
    return launch(std::string(base) + "_wide_v" + (vec && T % 4 == 0 ? "4" : "1"), rows, 1, RW_TEAM_HOST,
                  0, s, a);
  }
  // Rows of 129-256 units on two-wave teams holding 2 units per lane instead of
  // one wave holding 3-4: at T = 1024 (MI355X, warm clocks) the forward 204.7
  // against 216.9 us and the backward 271.2 against 278.9 us.
  if (c.team == 64 && (c.nv == 3 || c.nv == 4)) c = RowCfg{128, 2, c.vw};
  set_rpw(&c, rpw);
  const int bs = block_of(c);
  const int64_t rpb = (int64_t)(bs / c.team) * c.rpw;
  SoftmaxArgs a{in, dy, out, rows, (int32_t)T, causal ? 1 : 0, input_is_x ? 1 : 0, attn, ztile, g_causal_flag};
  return launch(fwd_kernel(base, c), cdiv(rows, rpb), 1, bs, 0, s, a);
}

int vh_softmax_fwd(const float* x, float* y, int64_t rows, int64_t T, int causal, void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || T < 0) return fail(VH_ERR_INVALID, "vh_softmax_fwd: negative size");
  if (rows == 0 || T == 0) return VH_OK;
  if (!x || !y) return fail(VH_ERR_INVALID, "vh_softmax_fwd: null pointer");
  if (T > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_softmax_fwd: T too large");
  return softmax_common("vh_sm_fwd", 16, kSmFwdRpw, x, nullptr, y, rows, T, causal, 0, S(stream));
}

int vh_softmax_bwd(const float* in, const float* dy, float* dx, int64_t rows, int64_t T,
                   int input_is_x, int causal, void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || T < 0) return fail(VH_ERR_INVALID, "vh_softmax_bwd: negative size");
  if (rows == 0 || T == 0) return VH_OK;
  if (!in || !dy || !dx) return fail(VH_ERR_INVALID, "vh_softmax_bwd: null pointer");
  if (T > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_softmax_bwd: T too large");
  return softmax_common("vh_sm_bwd", 8, kSmBwdRpw, in, dy, dx, rows, T, causal, input_is_x, S(stream));
}

// ------------------------------------------------------------- embedding --

int vh_embedding_fwd(const float* ids, const float* W, float* out, int64_t n, int64_t V, int64_t D,
                     void* stream) {
  VH_TRY(require_init());
  if (n < 0 || V < 0 || D < 0) return fail(VH_ERR_INVALID, "vh_embedding_fwd: negative size");
  if (n == 0) return VH_OK;
  // D == 0 still launches: the ids are validated as the reference does.
  if (!ids || (D > 0 && !out) || (V > 0 && D > 0 && !W))
    return fail(VH_ERR_INVALID, "vh_embedding_fwd: null pointer");
  if (V > INT32_MAX || D > INT32_MAX || n > INT32_MAX)
    return fail(VH_ERR_UNSUPPORTED, "vh_embedding_fwd: size exceeds int32");
  const bool vec = D % 4 == 0 && aligned16(W) && aligned16(out);
  EmbFwdArgs a{ids, W, out, g_rt.err, n, (int32_t)V, (int32_t)D};
  return launch(vec ? "vh_emb_fwd_v4" : "vh_emb_fwd_v1", cdiv(n, 4), 1, 256, 0, S(stream), a);
}

namespace {
// Heavy tokens have more than 16 hits, so at most n/17 of them; each gets
// ceil(hits/32) tasks, so at most n/32 + n/17 + 1 tasks in all.
constexpr int64_t kEmbLight = 16, kEmbChunkHits = 32;
// Heavy hits are counted per block of 2^blk_shift positions: 512 unless the
// [heavy entries][blocks] table would pass 4M entries, then larger.
constexpr int kEmbMinBlkShift = 9;
constexpr int64_t kEmbMaxBlkTable = int64_t(1) << 22;
struct EmbScratchLayout {
  size_t tok, counts, cursor, ctr, zero_end, heavy_index, heavy, taskmap, blkcnt, pos, partial, total;
  int64_t nblk;
  int blk_shift;
};
EmbScratchLayout emb_layout(int64_t n, int64_t V, int64_t D) {
  EmbScratchLayout L;
  const int64_t heavy_max = n / (kEmbLight + 1) + 1;
  const int64_t tasks_max = n / kEmbChunkHits + heavy_max + 1;
  L.blk_shift = kEmbMinBlkShift;
  while (heavy_max * cdiv(n, int64_t(1) << L.blk_shift) > kEmbMaxBlkTable) ++L.blk_shift;
  L.nblk = cdiv(n, int64_t(1) << L.blk_shift);
  size_t o = 0;
  auto take = [&](size_t elems) {
    size_t at = o;
    o += align256(elems * 4);
    return at;
  };
  L.tok = take((size_t)n);
  L.counts = take((size_t)V);
  L.cursor = take((size_t)V);
  L.ctr = take(4);
  L.zero_end = o;  // counts .. ctr are zeroed per call
  L.heavy_index = take((size_t)V);
  L.heavy = take(4 * (size_t)heavy_max);
  L.taskmap = take((size_t)tasks_max);
  L.blkcnt = take((size_t)heavy_max * (size_t)L.nblk);
  L.pos = take((size_t)V * kEmbLight);
  L.partial = take((size_t)tasks_max * (size_t)D);
  L.total = o;
  return L;
}

// The sorted path: each of EMB_RANGES workgroups sorts the keys of the tokens
// t % EMB_RANGES == k in LDS ((t / EMB_RANGES) << 14 | position: n <= 16384,
// t / EMB_RANGES < 4096).
constexpr int64_t kEmbSortMaxN = 16384;
constexpr int64_t kEmbSortMaxV = EMB_SORT_MAXV;
bool emb_sorted_path(int64_t n, int64_t V, int64_t D) {
  return n > 0 && n <= kEmbSortMaxN && V > 0 && V <= kEmbSortMaxV && D > 0;
}
struct EmbSortLayout {
  size_t spos, seg, heavy, heavy_start, taskmap, counts, ctr, partial, total;
  int64_t hmax, tmax;
};
EmbSortLayout emb_sort_layout(int64_t n, int64_t D) {
  EmbSortLayout L;
  L.hmax = n / (kEmbLight + 1) + 1;              // heavy tokens have > 16 hits
  L.tmax = n / kEmbChunkHits + L.hmax + 1;       // ceil(hits / 32) tasks each
  const int64_t slices_max = cdiv(D, 64);        // column slices of a heavy row (1-float units)
  size_t o = 0;
  auto take = [&](size_t elems) {
    size_t at = o;
    o += align256(elems * 4);
    return at;
  };
  L.spos = take((size_t)EMB_RANGES * n);
  L.seg = take((size_t)EMB_RANGES * n * EMB_REC);
  L.heavy = take((size_t)EMB_RANGES * L.hmax * 4);
  L.heavy_start = take((size_t)EMB_RANGES * L.hmax);
  L.taskmap = take((size_t)EMB_RANGES * L.tmax);
  L.counts = take(3 * EMB_RANGES);
  L.ctr = take((size_t)EMB_RANGES * (L.hmax + L.tmax) * slices_max);
  L.partial = take((size_t)L.tmax * (size_t)D);
  L.total = o;
  return L;
}
}  // namespace

size_t vh_embedding_bwd_scratch_bytes(int64_t n, int64_t V, int64_t D) {
  if (n <= 0 || V < 0 || D < 0) return 0;
  if (emb_sorted_path(n, V, D)) return emb_sort_layout(n, D).total;
  return emb_layout(n, V, D).total;
}

namespace {
// Sorted path: range sorts + zero fill, then segment sums and heavy partials with
// each heavy row slice finished by its last task.
int emb_bwd_sorted(const float* ids, const float* dy, float* dW, int64_t n, int64_t V, int64_t D, void* base_p,
                   hipStream_t s) {
  const EmbSortLayout L = emb_sort_layout(n, D);
  char* base = static_cast<char*>(base_p);
  auto I = [&](size_t off) { return reinterpret_cast<int32_t*>(base + off); };
  const bool vec = D % 4 == 0 && aligned16(dy) && aligned16(dW);
  const int64_t fill_n = V * D / (vec ? 4 : 1);
  // One workgroup per CU (the sort's LDS): the range sorts plus fills on the rest.
  const int64_t fill_blocks =
      std::max<int64_t>(1, std::min<int64_t>(std::max(g_rt.cu_count, EMB_RANGES + 1) - EMB_RANGES,
                                             cdiv(fill_n, 8192)));
  const int32_t slices = (int32_t)cdiv(D / (vec ? 4 : 1), 64);
  EmbSortArgs k1{ids, dW, I(L.spos), I(L.seg), I(L.heavy), I(L.heavy_start), I(L.taskmap), I(L.counts),
                 I(L.ctr), g_rt.err, fill_n, (int32_t)n, (int32_t)V, (int32_t)L.hmax,
                 (int32_t)L.tmax, vec ? 1 : 0, slices};
  VH_TRY(launch("vh_emb_sort", (EMB_RANGES + fill_blocks), 1, 1024, 0, s, k1));
  EmbSumArgs k2{I(L.spos), I(L.seg), I(L.heavy), I(L.heavy_start), I(L.taskmap), I(L.counts), I(L.ctr),
                reinterpret_cast<float*>(base + L.partial), dy, dW, (int32_t)n, (int32_t)L.hmax, (int32_t)L.tmax,
                (int32_t)D, slices};
  // A wave per item (heavy tasks' slices, then segments) up to 16384 waves;
  // the last tasks of each heavy row's slice write that slice of dW.
  return launch(vec ? "vh_emb_sum_v4" : "vh_emb_sum_v1",
                std::min<int64_t>(4096, cdiv(n + L.tmax * slices, 4)), 1, 256, 0, s, k2);
}
}  // namespace

int vh_embedding_bwd(const float* ids, const float* dy, float* dW, int64_t n, int64_t V, int64_t D,
                     void* scratch, size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  if (n < 0 || V < 0 || D < 0) return fail(VH_ERR_INVALID, "vh_embedding_bwd: negative size");
  hipStream_t s = S(stream);
  if (V * D > 0 && !dW) return fail(VH_ERR_INVALID, "vh_embedding_bwd: null pointer");
  if (n == 0) return fill(dW, 0.0f, V * D, s);
  if (!ids || (D > 0 && !dy)) return fail(VH_ERR_INVALID, "vh_embedding_bwd: null pointer");
  if (V >= INT32_MAX || D > INT32_MAX || n >= INT32_MAX / 2)
    return fail(VH_ERR_UNSUPPORTED, "vh_embedding_bwd: size exceeds int32");
  if (emb_sorted_path(n, V, D)) {
    Scratch sc;
    VH_TRY(sc.get(S(stream), scratch, scratch_bytes, emb_sort_layout(n, D).total));
    return emb_bwd_sorted(ids, dy, dW, n, V, D, sc.p, s);
  }
  const EmbScratchLayout L = emb_layout(n, V, D);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, L.total));
  char* base = static_cast<char*>(sc.p);
  auto I = [&](size_t off) { return reinterpret_cast<int32_t*>(base + off); };
  // counts, cursor and the counters are contiguous: one fill of zeros
  // (0.0f has the bits of int 0).
  VH_TRY(fill(I(L.counts), 0.0f, (int64_t)((L.zero_end - L.counts) / 4), s));
  EmbTokArgs k1{ids, I(L.tok), I(L.counts), g_rt.err, n, (int32_t)V};
  VH_TRY(launch("vh_emb_tokens", cdiv(n, 256), 1, 256, 0, s, k1));
  if (V == 0 || D == 0) return VH_OK;  // ids validated, nothing to write
  const bool vec = D % 4 == 0 && aligned16(dy) && aligned16(dW);
  const int32_t slices = (int32_t)cdiv(D / (vec ? 4 : 1), 64);  // 64-unit column slices of a heavy row
  EmbAllocArgs k2{I(L.counts), I(L.heavy_index), I(L.heavy), I(L.taskmap), I(L.blkcnt), I(L.ctr), (int32_t)V,
                  (int32_t)L.nblk};
  VH_TRY(launch("vh_emb_alloc", cdiv(V, 256), 1, 256, 0, s, k2));
  EmbPlaceArgs k3{I(L.tok), I(L.heavy_index), I(L.cursor), I(L.pos), I(L.blkcnt), n, (int32_t)L.nblk,
                  L.blk_shift};
  VH_TRY(launch("vh_emb_place", cdiv(n, 256), 1, 256, 0, s, k3));
  // Up to 1024 worker waves for the heavy work items (at most tasks_max x slices).
  const int64_t heavy_blocks =
      std::min<int64_t>(256, cdiv((n / kEmbChunkHits + n / (kEmbLight + 1) + 2) * slices, 4));
  float* partial = reinterpret_cast<float*>(base + L.partial);
  EmbSegArgs k4{I(L.counts), I(L.pos), I(L.tok), I(L.heavy), I(L.taskmap), I(L.blkcnt), I(L.ctr), partial,
                dy, dW, n, (int32_t)V, (int32_t)D, (int32_t)L.nblk, L.blk_shift, (int32_t)heavy_blocks, slices};
  VH_TRY(launch(vec ? "vh_emb_rows_v4" : "vh_emb_rows_v1", (heavy_blocks + cdiv(V, 4)), 1, 256, 0,
                s, k4));
  // Up to 512 waves striding over the (heavy entry, slice) items the device counted.
  const int64_t heavy_max = n / (kEmbLight + 1) + 1;
  EmbFinalArgs k5{I(L.heavy), I(L.ctr), partial, dW, (int32_t)D, slices};
  return launch(vec ? "vh_emb_heavy_final_v4" : "vh_emb_heavy_final_v1",
                std::min<int64_t>(128, cdiv(heavy_max * slices, 4)), 1, 256, 0, s, k5);
}

// --------------------------------------------------------- cross-entropy --

static const int kXE[] = {8, 16, 24, 32, 40, 48, 56, 64, 72, 80, 88, 96, 99, 104, 112, 120, 128};
constexpr int kXeTeam = 512;  // threads per row of the row-cached kernels
constexpr int kXeMask = 8;    // trailing units they mask

// The row-cached kernels hold NV values per thread of a 512-thread team and
// mask only their last 8 units, so NV - 8 < ceil(V / 512) <= NV; longer rows
// take the streaming kernel (1024 threads).
static std::string xent_kernel(const char* dir, int64_t V) {
  const int64_t need = cdiv(V, kXeTeam);
  for (int v : kXE)
    if (v >= need && v - kXeMask < need) return std::string("vh_xent_") + dir + "_n" + std::to_string(v);
  return std::string("vh_xent_") + dir + "_stream";
}
static unsigned xent_threads(const std::string& kernel) {
  return kernel.compare(kernel.size() - 7, 7, "_stream") == 0 ? 1024u : (unsigned)kXeTeam;
}

size_t vh_cross_entropy_fwd_scratch_bytes(int64_t B) {
  return B <= 0 ? 0 : align256((size_t)B * sizeof(float));
}

int vh_cross_entropy_fwd_ld(const float* logits, int64_t ld, const float* targets, float* loss, int64_t B,
                            int64_t V, void* scratch, size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  if (B <= 0) return fail(VH_ERR_INVALID, "Batch size must be greater than 0");
  if (V <= 0) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd: vocabulary must be > 0");
  if (ld < V) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd: row stride below V");
  if (!logits || !targets || !loss) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd: null pointer");
  if (V > INT32_MAX || B > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_fwd: size exceeds int32");
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_cross_entropy_fwd_scratch_bytes(B)));
  XentArgs a{logits, targets, nullptr, static_cast<float*>(sc.p), nullptr, g_rt.err, B, ld, (int32_t)V, nullptr};
  VH_TRY(launch(xent_kernel("fwd", V), B, 1, xent_threads(xent_kernel("fwd", V)), 0, s, a));
  XentReduceArgs r{static_cast<float*>(sc.p), loss, B};
  return launch("vh_xent_reduce", 1, 1, 1024, 0, s, r);
}

int vh_cross_entropy_fwd(const float* logits, const float* targets, float* loss, int64_t B,
                         int64_t V, void* scratch, size_t scratch_bytes, void* stream) {
  return vh_cross_entropy_fwd_ld(logits, V, targets, loss, B, V, scratch, scratch_bytes, stream);
}

int vh_cross_entropy_fwd_rs_ld(const float* logits, int64_t ld, const float* targets, float* loss,
                               float* row_stats, int64_t B, int64_t V, void* scratch, size_t scratch_bytes,
                               void* stream) {
  VH_TRY(require_init());
  if (B <= 0) return fail(VH_ERR_INVALID, "Batch size must be greater than 0");
  if (V <= 0) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_rs: vocabulary must be > 0");
  if (ld < V) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_rs: row stride below V");
  if (!logits || !targets || !loss || !row_stats)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_rs: null pointer");
  if (reinterpret_cast<uintptr_t>(row_stats) % 8 != 0)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_rs: row_stats must be 8-byte aligned");
  if (V > INT32_MAX || B > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_fwd_rs: size exceeds int32");
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_cross_entropy_fwd_scratch_bytes(B)));
  XentArgs a{logits, targets, nullptr, static_cast<float*>(sc.p), nullptr, g_rt.err, B, ld, (int32_t)V, row_stats};
  VH_TRY(launch(xent_kernel("fwd", V), B, 1, xent_threads(xent_kernel("fwd", V)), 0, s, a));
  XentReduceArgs r{static_cast<float*>(sc.p), loss, B};
  return launch("vh_xent_reduce", 1, 1, 1024, 0, s, r);
}

int vh_cross_entropy_bwd_ld(const float* logits, int64_t ld, const float* targets, const float* grad_out,
                            float* dlogits, int64_t B, int64_t V, void* stream) {
  VH_TRY(require_init());
  if (B <= 0) return fail(VH_ERR_INVALID, "Batch size must be greater than 0");
  if (V <= 0) return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd: vocabulary must be > 0");
  if (ld < V) return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd: row stride below V");
  if (!logits || !targets || !grad_out || !dlogits)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd: null pointer");
  if (V > INT32_MAX || B > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_bwd: size exceeds int32");
  XentArgs a{logits, targets, grad_out, dlogits, nullptr, g_rt.err, B, ld, (int32_t)V, nullptr};
  return launch(xent_kernel("bwd", V), B, 1, xent_threads(xent_kernel("bwd", V)), 0, S(stream), a);
}

// Chunks of the row-statistics backward: 256 threads x 2 16-byte units
// (XR4_CHUNK) when logits and dlogits are 16-byte aligned, else 256 threads x
// 16 elements (XR_CHUNK).
constexpr int64_t kXr4Chunk = 512;
constexpr int64_t kXrChunk = 4096;

int vh_cross_entropy_bwd_rs_ld(const float* logits, int64_t ld, const float* targets, const float* row_stats,
                               const float* grad_out, float* dlogits, int64_t B, int64_t V, void* stream) {
  VH_TRY(require_init());
  if (B <= 0) return fail(VH_ERR_INVALID, "Batch size must be greater than 0");
  if (V <= 0) return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd_rs: vocabulary must be > 0");
  if (ld < V) return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd_rs: row stride below V");
  if (!logits || !targets || !row_stats || !grad_out || !dlogits)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd_rs: null pointer");
  if (reinterpret_cast<uintptr_t>(row_stats) % 8 != 0)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_bwd_rs: row_stats must be 8-byte aligned");
  if (V > INT32_MAX || B > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_bwd_rs: size exceeds int32");
  XentArgs a{logits, targets, grad_out, dlogits, nullptr, g_rt.err, B, ld, (int32_t)V, const_cast<float*>(row_stats)};
  const bool v4 = (reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(dlogits)) % 16 == 0;
  const int64_t grid = B * (v4 ? cdiv(V / 4 + 1, kXr4Chunk) : cdiv(V, kXrChunk));
  if (grid > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_bwd_rs: grid exceeds int32");
  return launch(v4 ? "vh_xent_bwd_rs4" : "vh_xent_bwd_rs", grid, 1, 256, 0, S(stream), a);
}

int vh_cross_entropy_fwd_bwd_ld(const float* logits, int64_t ld, const float* targets, const float* grad_out,
                                float* loss, float* dlogits, int64_t B, int64_t V, void* scratch,
                                size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  if (B <= 0) return fail(VH_ERR_INVALID, "Batch size must be greater than 0");
  if (V <= 0) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_bwd: vocabulary must be > 0");
  if (ld < V) return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_bwd: row stride below V");
  if (!logits || !targets || !grad_out || !loss || !dlogits)
    return fail(VH_ERR_INVALID, "vh_cross_entropy_fwd_bwd: null pointer");
  if (V > INT32_MAX || B > INT32_MAX)
    return fail(VH_ERR_UNSUPPORTED, "vh_cross_entropy_fwd_bwd: size exceeds int32");
  const std::string fk = xent_kernel("fwd", V);
  if (fk.find("_stream") != std::string::npos) {  // rows too long to cache: two passes
    VH_TRY(vh_cross_entropy_fwd_ld(logits, ld, targets, loss, B, V, scratch, scratch_bytes, stream));
    return vh_cross_entropy_bwd_ld(logits, ld, targets, grad_out, dlogits, B, V, stream);
  }
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_cross_entropy_fwd_scratch_bytes(B)));
  float* rows = static_cast<float*>(sc.p);
  XentArgs a{logits, targets, grad_out, dlogits, rows, g_rt.err, B, ld, (int32_t)V, nullptr};
  VH_TRY(launch(xent_kernel("fb", V), B, 1, xent_threads(xent_kernel("fb", V)), 0, s, a));
  XentReduceArgs r{rows, loss, B};
  return launch("vh_xent_reduce", 1, 1, 1024, 0, s, r);
}

int vh_cross_entropy_bwd(const float* logits, const float* targets, const float* grad_out,
                         float* dlogits, int64_t B, int64_t V, void* stream) {
  return vh_cross_entropy_bwd_ld(logits, V, targets, grad_out, dlogits, B, V, stream);
}

// ------------------------------------------------------------ composites --

int vh_binary(int op, const float* l, const vh_layout* ll, const float* r, const vh_layout* rl,
              float* out, void* stream) {
  VH_TRY(require_init());
  if (op < 0 || op > 3) return fail(VH_ERR_INVALID, "vh_binary: unknown op");
  VH_TRY(check_layout(ll, "vh_binary lhs"));
  VH_TRY(check_layout(rl, "vh_binary rhs"));
  const int R = std::max(ll->rank, rl->rank);
  StridedLayout ol{}, lk{}, rk{};
  ol.rank = lk.rank = rk.rank = R;
  for (int i = 0; i < R; ++i) {
    const int li = ll->rank - R + i, ri = rl->rank - R + i;
    const int64_t ld = li >= 0 ? ll->dims[li] : 1, rd = ri >= 0 ? rl->dims[ri] : 1;
    int64_t od;
    if (ld == rd) od = ld;
    else if (ld == 1) od = rd;
    else if (rd == 1) od = ld;
    else return fail(VH_ERR_INVALID, "Shapes are not broadcastable");
    ol.dims[i] = od;
    lk.dims[i] = rk.dims[i] = od;
    lk.strides[i] = (li >= 0 && ll->dims[li] != 1) ? ll->strides[li] : 0;
    rk.strides[i] = (ri >= 0 && rl->dims[ri] != 1) ? rl->strides[ri] : 0;
  }
  int64_t n = 1;
  for (int i = 0; i < R; ++i) n *= ol.dims[i];
  if (n == 0) return VH_OK;
  if (!l || !r || !out) return fail(VH_ERR_INVALID, "vh_binary: null pointer");
  bool same = ll->rank == rl->rank;
  for (int i = 0; same && i < ll->rank; ++i) same = ll->dims[i] == rl->dims[i];
  BinaryArgs a{l, r, out, ol, lk, rk, n, op, 0, 0, 0};
  hipStream_t s = S(stream);
  if (same && is_contig(ll) && is_contig(rl)) {
    const bool vec = n % 4 == 0 && aligned16(l) && aligned16(r) && aligned16(out);
    const int64_t blocks = std::min<int64_t>(cdiv(n / (vec ? 4 : 1), 256), 16384);
    return launch(vec ? "vh_binary_contig_v4" : "vh_binary_contig_v1", blocks, 1, 256, 0, s, a);
  }
  // A contiguous operand covering the whole output and a contiguous vector
  // that repeats along it: over the output's trailing dims (a bias, the
  // attention mask, or one value) -- the row-broadcast stream -- or over its
  // leading dims with size-1 trailing dims (a kept-dim row sum) -- the
  // column-broadcast stream. The vector's own leading (or trailing) size-1
  // dims do not matter.
  auto covers = [&](const vh_layout* t) { return is_contig(t) && numel(t) == n; };
  // Elements per repeat of t over the output's trailing dims (0: not such a vector).
  auto suffix_len = [&](const vh_layout* t) -> int64_t {
    if (!is_contig(t)) return 0;
    int lo = 0;
    while (lo < t->rank && t->dims[lo] == 1) ++lo;
    const int k = t->rank - lo;
    if (k > R) return 0;
    int64_t len = 1;
    for (int i = 0; i < k; ++i) {
      if (t->dims[lo + i] != ol.dims[R - k + i]) return 0;
      len *= t->dims[lo + i];
    }
    return len;
  };
  // Output elements per element of t when t spans the output's leading dims.
  auto prefix_run = [&](const vh_layout* t) -> int64_t {
    if (!is_contig(t)) return 0;
    int hi = t->rank;
    while (hi > 0 && t->dims[hi - 1] == 1) --hi;
    const int off = R - t->rank;  // t right-aligned; its leading dims must be the output's
    for (int i = 0; i < off; ++i)
      if (ol.dims[i] != 1) return 0;
    for (int i = 0; i < hi; ++i)
      if (t->dims[i] != ol.dims[off + i]) return 0;
    int64_t run = 1;
    for (int i = off + hi; i < R; ++i) run *= ol.dims[i];
    return run;
  };
  const bool small_grid = cdiv(n, 256) < (int64_t(1) << 31);
  for (int side = 0; side < 2 && small_grid; ++side) {  // side 0: vector on the right
    const vh_layout* full = side == 0 ? ll : rl;
    const vh_layout* vt = side == 0 ? rl : ll;
    if (!covers(full) || numel(vt) >= n) continue;
    a.vec_lhs = side;
    const int64_t bn = suffix_len(vt);
    if (bn > 0 && n / bn > 1) {
      a.bn = bn;
      const bool vec = (bn % 4 == 0 || bn == 1) && n % 4 == 0 && aligned16(l) && aligned16(r) && aligned16(out);
      const int vw = vec ? 4 : 1;
      return launch(vec ? "vh_binary_rowbcast_v4" : "vh_binary_rowbcast_v1", cdiv(n / vw, 256), 1, 256, 0,
                    s, a);
    }
    const int64_t run = prefix_run(vt);
    if (run > 1) {
      a.bn = run;
      const bool vec = run % 4 == 0 && aligned16(full == ll ? l : r) && aligned16(out);
      const int vw = vec ? 4 : 1;
      return launch(vec ? "vh_binary_colbcast_v4" : "vh_binary_colbcast_v1", cdiv(n / vw, 256), 1, 256, 0,
                    s, a);
    }
  }
  const int64_t blocks = std::min<int64_t>(cdiv(n, 256), 16384);
  return launch(n < INT32_MAX ? "vh_binary_strided_i32" : "vh_binary_strided_i64", blocks, 1,
                256, 0, s, a);
}

int vh_reduce(int mean, const float* x, const vh_layout* xl, int dim, float* out, void* stream) {
  VH_TRY(require_init());
  VH_TRY(check_layout(xl, "vh_reduce"));
  if (dim < 0 || dim >= xl->rank) return fail(VH_ERR_INVALID, "Reduction dim out of range");
  StridedLayout ol{};
  ol.rank = xl->rank - 1;
  int64_t n_out = 1;
  for (int i = 0, j = 0; i < xl->rank; ++i) {
    if (i == dim) continue;
    ol.dims[j] = xl->dims[i];
    ol.strides[j] = xl->strides[i];
    n_out *= xl->dims[i];
    ++j;
  }
  if (n_out == 0) return VH_OK;
  if (!x || !out) return fail(VH_ERR_INVALID, "vh_reduce: null pointer");
  const int64_t red_len = xl->dims[dim];
  const int64_t red_stride = xl->strides[dim];
  // A sum over the outermost dim of a contiguous tensor is the column sum of a
  // [red_len, n_out] matrix (a bias gradient's reduce_to): two passes over row
  // groups instead of one thread walking each column.
  if (!mean && red_len >= 64 && is_contig(xl) && n_out <= INT32_MAX) {
    bool outer = true;
    for (int i = 0; i < dim; ++i) outer = outer && xl->dims[i] == 1;
    if (outer) return vh_sum_rows(x, red_len, n_out, out, nullptr, 0, stream);
  }
  ReduceArgs a{x, out, ol, n_out, red_len, red_stride, mean ? 1 : 0};
  hipStream_t s = S(stream);
  if ((red_stride == 1 || red_len == 1) && red_len >= 128)
    return launch("vh_reduce_wave", cdiv(n_out, 4), 1, 256, 0, s, a);
  const int64_t blocks = std::min<int64_t>(cdiv(n_out, 256), 16384);
  return launch("vh_reduce_thread", blocks, 1, 256, 0, s, a);
}

int vh_strided_copy(const float* src, const vh_layout* sl, float* dst, void* stream) {
  VH_TRY(require_init());
  VH_TRY(check_layout(sl, "vh_strided_copy"));
  const int64_t n = numel(sl);
  if (n == 0) return VH_OK;
  if (!src || !dst) return fail(VH_ERR_INVALID, "vh_strided_copy: null pointer");
  hipStream_t s = S(stream);
  if (is_contig(sl)) {
    VH_HIP(hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice, s));
    return VH_OK;
  }
  // A transposed view (last dim strided, the one before it unit-stride; up to
  // two leading dims): the LDS-tiled transpose, coalesced on both sides.
  const int r = sl->rank;
  if (r >= 2 && r <= 4 && sl->strides[r - 2] == 1 && sl->strides[r - 1] != 1 && sl->dims[r - 2] >= 16 &&
      sl->dims[r - 1] >= 16) {
    TransposeArgs t{src, dst, sl->dims[r - 2], sl->dims[r - 1], sl->strides[r - 1], 1, 0, 0};
    int64_t nb = 1;
    if (r == 3) {
      nb = sl->dims[0];
      t.nb1 = sl->dims[0];
      t.sb1 = sl->strides[0];
    } else if (r == 4) {
      nb = sl->dims[0] * sl->dims[1];
      t.nb1 = sl->dims[1];
      t.sb0 = sl->strides[0];
      t.sb1 = sl->strides[1];
    }
    const bool v4 = t.R % 4 == 0 && t.C % 4 == 0 && t.sc % 4 == 0 && t.sb0 % 4 == 0 && t.sb1 % 4 == 0 &&
                    aligned16(src) && aligned16(dst);
    if (cdiv(t.C, 64) < (int64_t(1) << 31) && cdiv(t.R, 64) < 65536 && nb < 65536)
      return launch(v4 ? "vh_transpose_v4" : "vh_transpose", cdiv(t.C, 64), cdiv(t.R, 64), 256, 0, s, t, nb);
  }
  CopyArgs a{src, dst, to_kl(*sl), n};
  const int64_t blocks = std::min<int64_t>(cdiv(n, 256), 16384);
  return launch(n < INT32_MAX ? "vh_strided_copy_i32" : "vh_strided_copy_i64", blocks, 1, 256, 0,
                s, a);
}


// ---------------------------------------------------------------- row sums --

static int64_t sum_rows_groups(int64_t rows) { return std::max<int64_t>(1, std::min<int64_t>(rows, 256)); }

size_t vh_sum_rows_scratch_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return 0;
  return align256((size_t)sum_rows_groups(rows) * (size_t)C * sizeof(float));
}

int vh_sum_rows(const float* x, int64_t rows, int64_t C, float* out, void* scratch, size_t scratch_bytes,
                void* stream) {
  VH_TRY(require_init());
  if (rows < 0 || C < 0) return fail(VH_ERR_INVALID, "vh_sum_rows: negative size");
  hipStream_t s = S(stream);
  if (C == 0) return VH_OK;
  if (!out) return fail(VH_ERR_INVALID, "vh_sum_rows: null pointer");
  if (rows == 0) return fill(out, 0.0f, C, s);
  if (!x) return fail(VH_ERR_INVALID, "vh_sum_rows: null pointer");
  if (C > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_sum_rows: C too large");
  const int64_t G0 = sum_rows_groups(rows);
  const int64_t rpb = cdiv(rows, G0);
  const int64_t G = cdiv(rows, rpb);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, align256((size_t)G0 * (size_t)C * sizeof(float))));
  float* part = static_cast<float*>(sc.p);
  ColPartialArgs a{x, part, rows, rpb, (int32_t)C};
  VH_TRY(launch("vh_col_partial", G, cdiv(C, 256), 256, 0, s, a));
  ColReduceArgs r{part, out, nullptr, (int32_t)G, (int32_t)C, 1};
  return launch("vh_col_reduce", cdiv(C, VH_COLR_COLS), 1, VH_COLR_COLS * 16, 0, s, r);
}

// ------------------------------------------------------------------ gemm --

static bool gemm_vec_ok(const float* p, int64_t ld, int64_t ext, const int64_t* sb) {
  return aligned16(p) && ld % 4 == 0 && ext % 4 == 0 && sb[0] % 4 == 0 && sb[1] % 4 == 0;
}

namespace {
struct GemmPlan {
  bool narrow;     // 128 x 64 C tiles instead of 128 x 128
  int64_t ksplit;  // K ranges, each its own workgroups; 1 = no split
  int64_t kchunk;  // k per range, a multiple of the 32-wide k tile
};

// Tile width and split-K for a product: the shape whose estimated time is
// least. A split or a narrow tile pays where the C tiles leave the chip's
// resident workgroups (2 per CU) idle -- a last wave mostly empty (768 tiles on
// 512 slots) or too few tiles to fill it (the weight gradients, 768 x 768
// outputs over K = 16384 rows). Time is counted in k steps of one 128-wide
// tile: waves x tile width x (k per range + a fixed cost for the prologue and
// epilogue), a narrow tile at 0.88 of the wide one's matrix-core rate (its B
// fragments feed half as many products), plus the fixed-order reduce of the
// split partials ((ks + 1) M N floats through HBM). Batched and causal
// products do not split. N <= 64 (attention's P v and its gradients,
// N = Dk = 64) always takes the narrow tile.
GemmPlan gemm_plan(int64_t M, int64_t N, int64_t K, bool may_split) {
  const int64_t slots = 2 * std::max(g_rt.cu_count, 1);
  GemmPlan best{N <= VH_GEMM_TILE_N / 2, 1, K};
  if (!may_split || K == 0) return best;
  double best_t = -1.0;
  for (int tn : {VH_GEMM_TILE_N, VH_GEMM_TILE_N / 2}) {
    if (N <= VH_GEMM_TILE_N / 2 && tn != VH_GEMM_TILE_N / 2) continue;
    const int64_t tiles = cdiv(M, VH_GEMM_TILE_M) * cdiv(N, tn);
    for (int64_t want = 1; want <= 32; ++want) {
      if (want > 1 && K / want < 256) break;
      const int64_t kchunk = cdiv(cdiv(K, want), 32) * 32;
      const int64_t ks = cdiv(K, kchunk);
      if (ks != want) continue;
      const int64_t n = tiles * ks;
      const double waves = (double)cdiv(n, slots);  // a part-filled last wave costs a whole one
      double t = waves * ((double)tn / VH_GEMM_TILE_N) * ((double)kchunk + 48.0) /
                 (tn == VH_GEMM_TILE_N ? 1.0 : 0.88);
      if (ks > 1) t += (double)(ks + 1) * (double)M * (double)N * 4.0 / 536e3;
      if (best_t < 0.0 || t < best_t) {
        best_t = t;
        best = GemmPlan{tn != VH_GEMM_TILE_N, ks, kchunk};
      }
    }
  }
  return best;
}
}  // namespace

namespace {
// Kernel arguments for descriptor d from outer batch index b0 on (the pointers
// advanced to it; the kernel walks the batches from there).
GemmArgs gemm_args(const vh_gemm_desc* d, int64_t lda, int64_t ldb, int64_t tiles_m, int64_t tiles_n,
                   int64_t b0 = 0) {
  GemmArgs g{};
  g.causal_flag = g_causal_flag;
  g.A = d->a ? d->a + b0 * d->a_sb[0] : nullptr;
  g.B = d->b ? d->b + b0 * d->b_sb[0] : nullptr;
  g.C = d->c + b0 * d->c_sb[0];
  g.E = d->e ? d->e + b0 * d->e_sb[0] : nullptr;
  g.M = d->M;
  g.N = d->N;
  g.K = d->K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = d->c_sm;
  g.sa1 = d->a_sb[0];
  g.sa2 = d->a_sb[1];
  g.sb1 = d->b_sb[0];
  g.sb2 = d->b_sb[1];
  g.sc1 = d->c_sb[0];
  g.sc2 = d->c_sb[1];
  g.se1 = d->e_sb[0];
  g.se2 = d->e_sb[1];
  g.sem = d->e_sm;
  g.sen = d->e_sn;
  g.nb2 = (int32_t)d->batch[1];
  g.tiles_m = (int32_t)tiles_m;
  g.tiles_n = (int32_t)tiles_n;
  g.accumulate = d->accumulate ? 1 : 0;
  g.causal = d->causal;
  g.alpha = d->alpha;
  g.ksplit = 1;
  return g;
}
}  // namespace

namespace {
thread_local int g_gemm_path = VH_GEMM_PATH_NONE;

// The persistent 256 x BN-tile kernel (kernels/gemm_big.h) for a large dense
// product, when its conditions hold; *taken reports whether it ran. BN = 256
// when B is row-contiguous, the k loop is long (K >= VH_GEMMB_WIDE_K) and the
// wide tiles fill at least one round of workgroups: a wider tile does a third
// more products per k-tile barrier and loads 14 % fewer operand bytes per
// product (on MI355X, the lm_head dW as [50260, 768] 9.16 -> 8.93 ms, as
// [768, 50260] 9.07 -> 8.92), while its epilogue keeps fewer registers free
// (it spills), which short k loops pay for (fc2 forward, K = 3072: 544 -> 593
// us), and a product of fewer wide tiles than workgroups runs all of them in
// the stream-K round (the [768, 768] weight gradient, K = 16384: 180 -> 196
// us). With both operands k-contiguous the narrow tile stays ahead even on
// long k loops (lm_head dx, K = 50260: 8.65 against 9.00 ms).
// Conditions: 4-byte-aligned operand bases (its 128-bit loads need no more); a
// tile's reads within 2^32 bytes of its origin (leading dimensions < 2^22); k
// tile and tile counts below 2^31 (K < 2^26). A k-contiguous operand with
// K % 32 != 0 splits K: the kernel takes the whole 32-wide k tiles and the
// tiled kernel adds the rest (alpha times the tail product) into C. A
// row-contiguous operand's reads past K land past its buffer bound, and so read
// 0, only when its leading dimension covers its extent (lda >= M, ldb >= N):
// one broadcast along k (stride 0) or with overlapping rows leaves a partial
// last k tile to the tiled kernel, which tests k < K.
int gemm_big(const vh_gemm_desc* d, bool akc, bool bkc, int64_t lda, int64_t ldb, hipStream_t s, bool* taken) {
  *taken = false;
  const int64_t M = d->M, N = d->N, K = d->K, nb = d->batch[0] * d->batch[1];
  if (d->causal != VH_GEMM_DENSE || K <= 0) return VH_OK;
  // Batched products need k loops long enough for a persistent walk (short-K
  // batched products, such as attention's scores, have their own kernel).
  if (nb > 1 && K < 512) return VH_OK;
  if (M < VH_GEMMB_TM || N < VH_GEMMB_TN || (double)M * (double)N * (double)K * (double)nb < 67108864.0)
    return VH_OK;
  if (reinterpret_cast<uintptr_t>(d->a) % 4 != 0 || reinterpret_cast<uintptr_t>(d->b) % 4 != 0) return VH_OK;
  if (lda >= (int64_t(1) << 22) || ldb >= (int64_t(1) << 22) || K >= (int64_t(1) << 26)) return VH_OK;
  const int G = std::max(8, g_rt.cu_count / 8 * 8);
  const int64_t K32 = (akc || bkc) ? K / 32 * 32 : K;
  if (K32 == 0) return VH_OK;
  if (K32 % 32 != 0 && ((!akc && lda < M) || (!bkc && ldb < N))) return VH_OK;
  const bool wide = (d->engine == VH_GEMM_ENGINE_WIDE && N >= VH_GEMMB_TN_WIDE) ||
                    (!bkc && K32 >= VH_GEMMB_WIDE_K && N >= VH_GEMMB_TN_WIDE &&
                     cdiv(M, VH_GEMMB_TM) * cdiv(N, VH_GEMMB_TN_WIDE) * nb >= G);
  const int64_t BN = wide ? VH_GEMMB_TN_WIDE : VH_GEMMB_TN;
  const int64_t tiles_m = cdiv(M, VH_GEMMB_TM), tiles_n = cdiv(N, BN);
  if (tiles_m * tiles_n * nb >= INT32_MAX) return VH_OK;
  const int64_t tiles = tiles_m * tiles_n * nb, rem = tiles % G;
  GemmArgs g = gemm_args(d, lda, ldb, tiles_m, tiles_n);
  g.K = K32;
  g.nbat = nb;
  void* ws = nullptr;
  if (rem > 0) {
    VH_TRY(g_arena.alloc((size_t)G * VH_GEMMB_SLOTS * VH_GEMMB_TM * BN * sizeof(float), s, &ws));
    g.ws = static_cast<float*>(ws);
  }
  const std::string bn = std::to_string(BN);
  const std::string name = std::string("vh_gemmb_") + (akc ? "k" : "m") + (bkc ? "k" : "n") + "_" + bn;
  int rc = launch(name, G, 1, 512, 0, s, g);
  if (rc == VH_OK && rem > 0) {
    GemmArgs f = g;
    f.ksplit = G;
    rc = launch("vh_gemmb_fix_" + bn, (rem * (VH_GEMMB_TM / 16)), 1, 256, 0, s, f);
  }
  if (ws) g_arena.free(ws, s);
  VH_TRY(rc);
  *taken = true;
  if (K32 < K) {
    vh_gemm_desc t = *d;
    t.K = K - K32;
    t.a = d->a + K32 * d->a_sk;
    t.b = d->b + K32 * d->b_sk;
    t.e = nullptr;
    t.accumulate = 1;
    t.engine = VH_GEMM_ENGINE_TILED;
    VH_TRY(vh_gemm(&t, s));
  }
  g_gemm_path = VH_GEMM_PATH_PERSISTENT;
  return VH_OK;
}
}  // namespace

int vh_gemm_last_path(void) { return g_gemm_path; }

int vh_gemm(const vh_gemm_desc* d, void* stream) {
  g_gemm_path = VH_GEMM_PATH_NONE;
  VH_TRY(require_init());
  if (!d) return fail(VH_ERR_INVALID, "vh_gemm: null descriptor");
  const int64_t M = d->M, N = d->N, K = d->K;
  if (M < 0 || N < 0 || K < 0 || d->batch[0] < 0 || d->batch[1] < 0)
    return fail(VH_ERR_INVALID, "vh_gemm: negative size");
  const int64_t strides[] = {d->a_sm, d->a_sk, d->b_sk, d->b_sn, d->c_sm, d->a_sb[0], d->a_sb[1],
                             d->b_sb[0], d->b_sb[1], d->c_sb[0], d->c_sb[1], d->e_sm, d->e_sn,
                             d->e_sb[0], d->e_sb[1]};
  for (int64_t st : strides)
    if (st < 0) return fail(VH_ERR_INVALID, "vh_gemm: negative stride");
  if (M == 0 || N == 0 || d->batch[0] == 0 || d->batch[1] == 0) return VH_OK;
  if (!d->c || (K > 0 && (!d->a || !d->b))) return fail(VH_ERR_INVALID, "vh_gemm: null pointer");
  if (d->causal < 0 || d->causal > 3) return fail(VH_ERR_INVALID, "vh_gemm: unknown causal mode");
  if ((d->causal == VH_GEMM_K_LE_M || d->causal == VH_GEMM_K_GE_M) && M != K)
    return fail(VH_ERR_INVALID, "vh_gemm: causal k ranges need M == K");
  // A unit stride along k (k-contiguous) or along m; the same for B along k or n.
  const bool akc = d->a_sk == 1 || K == 1;
  const bool bkc = d->b_sk == 1 || K == 1;
  if (!akc && d->a_sm != 1 && M != 1)
    return fail(VH_ERR_UNSUPPORTED, "vh_gemm: A needs a unit stride along m or k");
  if (!bkc && d->b_sn != 1 && N != 1)
    return fail(VH_ERR_UNSUPPORTED, "vh_gemm: B needs a unit stride along k or n");
  const int64_t lda = akc ? (M == 1 ? 0 : d->a_sm) : d->a_sk;
  const int64_t ldb = bkc ? (N == 1 ? 0 : d->b_sn) : d->b_sk;
  if (d->engine < VH_GEMM_ENGINE_DEFAULT || d->engine > VH_GEMM_ENGINE_WIDE)
    return fail(VH_ERR_INVALID, "vh_gemm: unknown engine");
  // LIBRARY: large unbatched dense products, with no addend or a bias over
  // the output columns, go to hipBLASLt when it has an algorithm (the A/B
  // reference); everything else as DEFAULT.
  // Under a device causal flag (an attention call) the product keeps one
  // launch whose grid serves both forms: no library, large-product kernel or
  // split of K.
  const bool dflag = g_causal_flag != nullptr;
  if (!dflag && d->engine == VH_GEMM_ENGINE_LIBRARY && d->batch[0] * d->batch[1] == 1 && d->causal == VH_GEMM_DENSE &&
      (!d->e || (d->e_sm == 0 && d->e_sn == 1)) && K > 0 && (double)M * (double)N * (double)K >= 67108864.0) {
    bool taken = false;
    VH_TRY(vh_rt::blaslt_gemm(d, akc, bkc, stream, &taken));
    if (taken) {
      g_gemm_path = VH_GEMM_PATH_LIBRARY;
      return VH_OK;
    }
  }
  if (!dflag && d->engine != VH_GEMM_ENGINE_TILED) {
    bool taken = false;
    VH_TRY(gemm_big(d, akc, bkc, lda, ldb, S(stream), &taken));
    if (taken) return VH_OK;
  }
  const bool avec = K > 0 && gemm_vec_ok(d->a, lda, akc ? K : M, d->a_sb);
  const bool bvec = K > 0 && gemm_vec_ok(d->b, ldb, bkc ? K : N, d->b_sb);
  const GemmPlan plan = gemm_plan(M, N, K, !dflag && d->batch[0] * d->batch[1] == 1 && d->causal == VH_GEMM_DENSE);
  const int64_t tiles_m = cdiv(M, VH_GEMM_TILE_M), tiles_n = cdiv(N, plan.narrow ? 64 : VH_GEMM_TILE_N);
  if (tiles_m * tiles_n > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_gemm: too many tiles");
  const std::string name = std::string("vh_gemm_") + (akc ? "k" : "m") + (avec ? "4" : "1") + "_" +
                           (bkc ? "k" : "n") + (bvec ? "4" : "1") + (plan.narrow ? "_t64" : "");
  hipStream_t s = S(stream);
  const int64_t tiles = tiles_m * tiles_n;
  {
    const int64_t ks = plan.ksplit, kchunk = plan.kchunk;
    if (ks > 1) {
      void* ws = nullptr;
      VH_TRY(g_arena.alloc((size_t)(ks * M * N) * sizeof(float), s, &ws));
      // Raw partials: the reduce applies alpha, the addend and accumulation.
      GemmArgs g = gemm_args(d, lda, ldb, tiles_m, tiles_n);
      g.E = nullptr;
      g.accumulate = 0;
      g.ksplit = (int32_t)ks;
      g.kchunk = kchunk;
      g.ws = static_cast<float*>(ws);
      int rc = launch(name, tiles, ks, 256, 0, s, g);
      if (rc == VH_OK) {
        GemmReduceArgs r{g.ws, d->c, d->e, M, N, d->c_sm, d->e_sm, d->e_sn, (int32_t)ks,
                         d->accumulate ? 1 : 0, d->alpha};
        const int64_t blocks = std::min<int64_t>(cdiv(M * N, 256), 8192);
        rc = launch("vh_gemm_reduce", blocks, 1, 256, 0, s, r);
      }
      g_arena.free(ws, s);
      if (rc == VH_OK) g_gemm_path = VH_GEMM_PATH_SPLIT_K;
      return rc;
    }
  }
  // Batched products with a short k range (attention's q k^T and dO v^T,
  // K = Dk): one workgroup per resident slot walks the tiles of all batches,
  // loading each tile's operands under the previous tile's products
  // (gemm_f32_persist). A workgroup per tile spends most of its short life
  // waiting for its first loads there.
  const int64_t nbat = d->batch[0] * d->batch[1];
  if (nbat > 1 && K > 0 && K <= 256 && avec && bvec && !plan.narrow &&
      (d->causal == VH_GEMM_DENSE || (d->causal == VH_GEMM_SKIP_UPPER && tiles_n >= tiles_m))) {
    GemmArgs g = gemm_args(d, lda, ldb, tiles_m, tiles_n);
    g.nbat = nbat;
    // Under a device flag the product may run dense: size the grid for that.
    const int64_t live = (d->causal == VH_GEMM_SKIP_UPPER && !dflag) ? tiles_m * (tiles_m + 1) / 2 : tiles;
    const int64_t slots = 8 * std::max<int64_t>(1, 2 * std::max(g_rt.cu_count, 1) / 8);
    const int64_t grid = std::min<int64_t>(slots, 8 * cdiv(live * nbat, 8));
    const std::string pname = std::string("vh_gemmp_") + (akc ? "k4" : "m4") + "_" + (bkc ? "k4" : "n4");
    VH_TRY(launch(pname, grid, 1, 256, 0, s, g));
    g_gemm_path = VH_GEMM_PATH_BATCHED;
    return VH_OK;
  }
  // Grid y covers both batch dims; runs of the outer one keep it under 65535.
  const int64_t outer_chunk = std::max<int64_t>(1, 65535 / d->batch[1]);
  if (d->batch[1] > 65535) return fail(VH_ERR_UNSUPPORTED, "vh_gemm: inner batch too large");
  for (int64_t b0 = 0; b0 < d->batch[0]; b0 += outer_chunk) {
    const int64_t nb = std::min(outer_chunk, d->batch[0] - b0);
    const GemmArgs g = gemm_args(d, lda, ldb, tiles_m, tiles_n, b0);
    VH_TRY(launch(name, (tiles_m * tiles_n), (nb * d->batch[1]), 256, 0, s, g));
  }
  g_gemm_path = VH_GEMM_PATH_TILED;
  return VH_OK;
}

namespace {
// A contiguous copy of a strided operand whose last two dims have no unit
// stride (the reference makes every matmul operand contiguous, cpu:307-308).
struct Contig {
  void* p = nullptr;
  hipStream_t s = nullptr;
  ~Contig() {
    if (p) g_arena.free(p, s);
  }
};

int matmul_operand(const float* x, const vh_layout* l, Contig* tmp, const float** out, vh_layout* ol,
                   hipStream_t s) {
  *ol = *l;
  *out = x;
  const int r = l->rank;
  const bool ok = l->strides[r - 1] == 1 || l->strides[r - 2] == 1 || l->dims[r - 1] == 1 ||
                  l->dims[r - 2] == 1;
  if (ok) return VH_OK;
  const int64_t n = numel(l);
  tmp->s = s;
  VH_TRY(g_arena.alloc((size_t)n * sizeof(float), s, &tmp->p));
  VH_TRY(vh_strided_copy(x, l, static_cast<float*>(tmp->p), s));
  int64_t acc = 1;
  for (int i = r - 1; i >= 0; --i) {
    ol->strides[i] = acc;
    acc *= l->dims[i];
  }
  *out = static_cast<const float*>(tmp->p);
  return VH_OK;
}
}  // namespace

int vh_matmul(const float* lhs, const vh_layout* ll, const float* rhs, const vh_layout* rl, float* out,
              void* stream) {
  VH_TRY(require_init());
  VH_TRY(check_layout(ll, "vh_matmul lhs"));
  VH_TRY(check_layout(rl, "vh_matmul rhs"));
  if (ll->rank < 2 || rl->rank < 2) return fail(VH_ERR_INVALID, "Matmul requires rank >= 2");
  const int lr = ll->rank, rr = rl->rank;
  const int64_t M = ll->dims[lr - 2], K = ll->dims[lr - 1], K2 = rl->dims[rr - 2], N = rl->dims[rr - 1];
  if (K != K2) return fail(VH_ERR_INVALID, "Incompatible dimensions for matmul");
  const int lb = lr - 2, rb = rr - 2, ob = std::max(lb, rb);
  int64_t odims[VH_MAX_RANK], as[VH_MAX_RANK], bs[VH_MAX_RANK];
  for (int i = 0; i < ob; ++i) {
    const int li = i - (ob - lb), ri = i - (ob - rb);
    const int64_t a = li >= 0 ? ll->dims[li] : 1, b = ri >= 0 ? rl->dims[ri] : 1;
    if (a != b && a != 1 && b != 1) return fail(VH_ERR_INVALID, "Batch shapes are not broadcastable");
    odims[i] = std::max(a, b);
  }
  int64_t nout = M * N;
  for (int i = 0; i < ob; ++i) nout *= odims[i];
  if (nout == 0) return VH_OK;
  if (!lhs || !rhs || !out) return fail(VH_ERR_INVALID, "vh_matmul: null pointer");
  hipStream_t s = S(stream);
  Contig ta, tb;
  const float *A, *B;
  vh_layout al, bl;
  VH_TRY(matmul_operand(lhs, ll, &ta, &A, &al, s));
  VH_TRY(matmul_operand(rhs, rl, &tb, &B, &bl, s));
  for (int i = 0; i < ob; ++i) {
    const int li = i - (ob - lb), ri = i - (ob - rb);
    as[i] = (li >= 0 && al.dims[li] != 1) ? al.strides[li] : 0;
    bs[i] = (ri >= 0 && bl.dims[ri] != 1) ? bl.strides[ri] : 0;
  }
  // Output batch strides (contiguous [batch..., M, N]).
  int64_t cs[VH_MAX_RANK], acc = M * N;
  for (int i = ob - 1; i >= 0; --i) {
    cs[i] = acc;
    acc *= odims[i];
  }
  // A right operand shared by every batch (a Linear weight applied to [B, S, K]
  // input) whose left batches are evenly spaced rows folds into one product of
  // batch * M rows: the same multiply-adds in the same order per element, one
  // launch of the large-product kernel instead of a batched one.
  bool fold = ob > 0;
  int64_t rows = M;
  for (int i = ob - 1; i >= 0 && fold; --i) {
    if (odims[i] == 1) continue;
    fold = bs[i] == 0 && as[i] == rows * al.strides[lr - 2];
    rows *= odims[i];
  }
  vh_gemm_desc d{};
  if (fold) {
    d.M = rows;
    d.N = N;
    d.K = K;
    d.a = A;
    d.a_sm = al.strides[lr - 2];
    d.a_sk = al.strides[lr - 1];
    d.b = B;
    d.b_sk = bl.strides[rr - 2];
    d.b_sn = bl.strides[rr - 1];
    d.c = out;
    d.c_sm = N;
    d.alpha = 1.0f;
    d.batch[0] = d.batch[1] = 1;
    return vh_gemm(&d, stream);
  }
  d.M = M;
  d.N = N;
  d.K = K;
  d.a_sm = al.strides[lr - 2];
  d.a_sk = al.strides[lr - 1];
  d.b_sk = bl.strides[rr - 2];
  d.b_sn = bl.strides[rr - 1];
  d.c_sm = N;
  d.alpha = 1.0f;
  // The last two batch dims go to the kernel; any others are looped here.
  const int inner = std::min(ob, 2), lead = ob - inner;
  for (int j = 0; j < 2; ++j) {
    const int i = lead + j - (2 - inner);
    d.batch[j] = i >= lead ? odims[i] : 1;
    d.a_sb[j] = i >= lead ? as[i] : 0;
    d.b_sb[j] = i >= lead ? bs[i] : 0;
    d.c_sb[j] = i >= lead ? cs[i] : 0;
  }
  int64_t nlead = 1;
  for (int i = 0; i < lead; ++i) nlead *= odims[i];
  for (int64_t t = 0; t < nlead; ++t) {
    int64_t rem = t, ao = 0, bo = 0, co = 0;
    for (int i = lead - 1; i >= 0; --i) {
      const int64_t c = rem % odims[i];
      rem /= odims[i];
      ao += c * as[i];
      bo += c * bs[i];
      co += c * cs[i];
    }
    d.a = A + ao;
    d.b = B + bo;
    d.c = out + co;
    VH_TRY(vh_gemm(&d, stream));
  }
  return VH_OK;
}

// ------------------------------------------------------- fused attention --

namespace {
struct AttnShape {
  int64_t B, H, S, Dk;
};

int attn_layout(const vh_layout* l, const char* what, AttnShape* sh, bool first) {
  if (!l || l->rank != 4) return fail(VH_ERR_INVALID, std::string(what) + ": expected a rank-4 [B, H, S, Dk] layout");
  VH_TRY(check_layout(l, what));
  if (first) {
    *sh = AttnShape{l->dims[0], l->dims[1], l->dims[2], l->dims[3]};
  } else if (l->dims[0] != sh->B || l->dims[1] != sh->H || l->dims[2] != sh->S || l->dims[3] != sh->Dk) {
    return fail(VH_ERR_INVALID, std::string(what) + ": shape differs from q");
  }
  if (l->strides[3] != 1 && l->dims[3] != 1)
    return fail(VH_ERR_UNSUPPORTED, std::string(what) + ": the last dim must have unit stride");
  return VH_OK;
}

// The mask right-aligned to [B, H, S, S] with broadcasting (cpu:2395-2404).
int attn_mask(const vh_layout* ml, const AttnShape& sh, int64_t st[4]) {
  if (ml->rank > 4) return fail(VH_ERR_INVALID, "fused attention: mask rank above 4");
  VH_TRY(check_layout(ml, "fused attention mask"));
  const int64_t tgt[4] = {sh.B, sh.H, sh.S, sh.S};
  for (int i = 0; i < 4; ++i) {
    const int mi = i - (4 - ml->rank);
    const int64_t dim = mi >= 0 ? ml->dims[mi] : 1;
    if (dim != 1 && dim != tgt[i]) return fail(VH_ERR_INVALID, "fused attention: mask does not broadcast");
    st[i] = (mi >= 0 && dim != 1) ? ml->strides[mi] : 0;
  }
  return VH_OK;
}

// scores[b, h] = q k^T * scale (+ mask) into P, then P = softmax(scores) in place.
int attn_probs(const float* q, const vh_layout* ql, const float* k, const vh_layout* kl, const float* mask,
               const int64_t* mst, int causal, const AttnShape& sh, float* P, hipStream_t s) {
  const float scale = 1.0f / std::sqrt((float)sh.Dk);
  vh_gemm_desc d{};
  d.M = sh.S;
  d.N = sh.S;
  d.K = sh.Dk;
  d.a = q;
  d.a_sm = ql->strides[2];
  d.a_sk = 1;
  d.b = k;  // B[k=d][n=j] = k[j][d]
  d.b_sk = 1;
  d.b_sn = kl->strides[2];
  d.c = P;
  d.c_sm = sh.S;
  d.batch[0] = sh.B;
  d.batch[1] = sh.H;
  d.a_sb[0] = ql->strides[0];
  d.a_sb[1] = ql->strides[1];
  d.b_sb[0] = kl->strides[0];
  d.b_sb[1] = kl->strides[1];
  d.c_sb[0] = sh.H * sh.S * sh.S;
  d.c_sb[1] = sh.S * sh.S;
  if (mask) {
    d.e = mask;
    d.e_sb[0] = mst[0];
    d.e_sb[1] = mst[1];
    d.e_sm = mst[2];
    d.e_sn = mst[3];
  }
  d.alpha = scale;
  d.causal = causal ? VH_GEMM_SKIP_UPPER : VH_GEMM_DENSE;
  VH_TRY(vh_gemm(&d, s));
  // The causal products read P only up to the end of each row's C tile.
  return softmax_common("vh_sm_fwd", 16, kSmFwdRpw, P, nullptr, P, sh.B * sh.H * sh.S, sh.S, causal, 0, s, 1,
                        VH_GEMM_TILE_M);
}
}  // namespace

namespace {
// The backward from the probabilities P [B, H, S, S] (contiguous): G is a
// score-sized workspace.
int attn_bwd_from_probs(const float* P, float* G, const float* q, const vh_layout* ql, const float* k,
                        const vh_layout* kl, const float* v, const vh_layout* vl, int causal, const float* dout,
                        const vh_layout* dol, float* dq, const vh_layout* dql, float* dk, const vh_layout* dkl,
                        float* dv, const vh_layout* dvl, const AttnShape& sh, hipStream_t s) {
  const float scale = 1.0f / std::sqrt((float)sh.Dk);
  const int64_t pb0 = sh.H * sh.S * sh.S, pb1 = sh.S * sh.S;
  // 2. dP = dO v^T into G.
  vh_gemm_desc d{};
  d.M = sh.S;
  d.N = sh.S;
  d.K = sh.Dk;
  d.a = dout;
  d.a_sm = dol->strides[2];
  d.a_sk = 1;
  d.b = v;  // B[k=d][n=j] = v[j][d]
  d.b_sk = 1;
  d.b_sn = vl->strides[2];
  d.c = G;
  d.c_sm = sh.S;
  d.batch[0] = sh.B;
  d.batch[1] = sh.H;
  d.a_sb[0] = dol->strides[0];
  d.a_sb[1] = dol->strides[1];
  d.b_sb[0] = vl->strides[0];
  d.b_sb[1] = vl->strides[1];
  d.c_sb[0] = pb0;
  d.c_sb[1] = pb1;
  d.alpha = 1.0f;
  d.causal = causal ? VH_GEMM_SKIP_UPPER : VH_GEMM_DENSE;
  VH_TRY(vh_gemm(&d, s));
  // 3. dS = P * (dP - sum(dP * P)) in place over G.
  VH_TRY(softmax_common("vh_sm_bwd", 8, kSmBwdRpw, P, G, G, sh.B * sh.H * sh.S, sh.S, causal, 0, s, 1,
                        VH_GEMM_TILE_M));
  // 4. dq = (dS k) * scale.
  vh_gemm_desc e{};
  e.M = sh.S;
  e.N = sh.Dk;
  e.K = sh.S;
  e.a = G;
  e.a_sm = sh.S;
  e.a_sk = 1;
  e.b = k;  // B[k=j][n=d] = k[j][d]
  e.b_sk = kl->strides[2];
  e.b_sn = 1;
  e.c = dq;
  e.c_sm = dql->strides[2];
  e.batch[0] = sh.B;
  e.batch[1] = sh.H;
  e.a_sb[0] = pb0;
  e.a_sb[1] = pb1;
  e.b_sb[0] = kl->strides[0];
  e.b_sb[1] = kl->strides[1];
  e.c_sb[0] = dql->strides[0];
  e.c_sb[1] = dql->strides[1];
  e.alpha = scale;
  e.causal = causal ? VH_GEMM_K_LE_M : VH_GEMM_DENSE;
  VH_TRY(vh_gemm(&e, s));
  // 5. dk = (dS^T q) * scale: A[m=j][k=i] = dS[i][j].
  e.a_sm = 1;
  e.a_sk = sh.S;
  e.b = q;
  e.b_sk = ql->strides[2];
  e.b_sb[0] = ql->strides[0];
  e.b_sb[1] = ql->strides[1];
  e.c = dk;
  e.c_sm = dkl->strides[2];
  e.c_sb[0] = dkl->strides[0];
  e.c_sb[1] = dkl->strides[1];
  e.causal = causal ? VH_GEMM_K_GE_M : VH_GEMM_DENSE;
  VH_TRY(vh_gemm(&e, s));
  // 6. dv = P^T dO.
  e.a = P;
  e.b = dout;
  e.b_sk = dol->strides[2];
  e.b_sb[0] = dol->strides[0];
  e.b_sb[1] = dol->strides[1];
  e.c = dv;
  e.c_sm = dvl->strides[2];
  e.c_sb[0] = dvl->strides[0];
  e.c_sb[1] = dvl->strides[1];
  e.alpha = 1.0f;
  return vh_gemm(&e, s);
}
}  // namespace

size_t vh_fused_attention_scratch_bytes(int64_t B, int64_t H, int64_t S, int backward) {
  if (B <= 0 || H <= 0 || S <= 0) return 0;
  const size_t one = align256((size_t)B * (size_t)H * (size_t)S * (size_t)S * sizeof(float));
  return backward ? 2 * one : one;
}

namespace {
constexpr size_t kProbeWords = 64 * 8;  // the probe's 64 slots of 8 words
constexpr size_t kProbeBytes = kProbeWords * sizeof(uint32_t) + 256;  // + the verdict

// Launches the probe of an attention call's mask and operands (vh_attn_probe)
// and its verdict (vh_attn_decide) into flag, a device int32: 1 when skipping
// the masked blocks gives the dense masked form's bits (the conditions are
// in attn_decide_impl). words: kProbeWords of device scratch. *usable is false,
// and nothing is launched, when the call is outside what the probe handles
// (no [S, S] block in the mask, or a grid beyond its limits): the dense form
// must run then.
int attn_probe_decide(const float* q, const vh_layout* ql, const float* k, const vh_layout* kl, const float* v,
                      const vh_layout* vl, const float* g, const vh_layout* gl, const float* mask,
                      const vh_layout* ml, const AttnShape& sh, uint32_t* words, int32_t* flag, hipStream_t s,
                      bool* usable) {
  *usable = false;
  // The mask must carry the [S, S] block itself (a broadcast row or column
  // cannot hold the triangle), each leading dim either its own or broadcast.
  if (ml->rank < 2 || ml->dims[ml->rank - 1] != sh.S || ml->dims[ml->rank - 2] != sh.S) return VH_OK;
  if (sh.S > INT32_MAX || sh.Dk > INT32_MAX || sh.B * sh.H > INT32_MAX) return VH_OK;
  AttnProbeArgs a{};
  const vh_layout* ls[5] = {ml, ql, kl, vl, g ? gl : nullptr};
  const float* ts[5] = {mask, q, k, v, g};
  for (int i = 0; i < 5; ++i) {
    a.t[i] = ts[i];
    if (!ts[i]) continue;
    const vh_layout* l = ls[i];
    int64_t dm[4], st[4];
    for (int j = 0; j < 4; ++j) {
      const int lj = j - (4 - l->rank);
      dm[j] = lj >= 0 ? l->dims[lj] : 1;
      st[j] = lj >= 0 ? l->strides[lj] : 0;
    }
    a.d0[i] = (int32_t)dm[0]; a.d1[i] = (int32_t)dm[1]; a.d2[i] = (int32_t)dm[2]; a.d3[i] = (int32_t)dm[3];
    a.s0[i] = st[0]; a.s1[i] = st[1]; a.s2[i] = st[2]; a.s3[i] = st[3];
  }
  a.Y = (int32_t)std::max<int64_t>(sh.B * sh.H, (int64_t)a.d0[0] * a.d1[0]);
  if ((int64_t)a.Y * 5 > 65535) return VH_OK;  // grid y limit: leave such calls on the dense path
  VH_TRY(fill(reinterpret_cast<float*>(words), 0.0f, (int64_t)kProbeWords, s));
  a.words = words;
  VH_TRY(launch("vh_attn_probe", cdiv(sh.S, 16), (5 * a.Y), 256, 0, s, a));
  AttnDecideArgs dcs{words, flag, (double)(1.0f / std::sqrt((float)sh.Dk)), (int32_t)sh.Dk, g ? 1 : 0};
  VH_TRY(launch("vh_attn_decide", 1, 1, 64, 0, s, dcs));
  *usable = true;
  return VH_OK;
}
}  // namespace

int vh_attention_mask_is_causal(const float* q, const vh_layout* ql, const float* k, const vh_layout* kl,
                                const float* v, const vh_layout* vl, const float* g, const vh_layout* gl,
                                const float* mask, const vh_layout* ml, int* is_causal, void* stream) {
  VH_TRY(require_init());
  if (!is_causal) return fail(VH_ERR_INVALID, "vh_attention_mask_is_causal: null result pointer");
  *is_causal = 0;
  AttnShape sh;
  VH_TRY(attn_layout(ql, "attention mask probe q", &sh, true));
  VH_TRY(attn_layout(kl, "attention mask probe k", &sh, false));
  VH_TRY(attn_layout(vl, "attention mask probe v", &sh, false));
  if (g) VH_TRY(attn_layout(gl, "attention mask probe grad", &sh, false));
  if (!mask || !ml) return fail(VH_ERR_INVALID, "vh_attention_mask_is_causal: no mask");
  int64_t mst[4];
  VH_TRY(attn_mask(ml, sh, mst));
  if (sh.B * sh.H * sh.S * sh.Dk == 0 || !q || !k || !v) return VH_OK;
  hipStream_t s = S(stream);
  // The answer needs a host wait, which a stream under graph capture cannot
  // make: answer "no" (the dense form is always right) without launching.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  VH_HIP(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone) return VH_OK;
  Scratch sc;
  VH_TRY(sc.get(s, nullptr, 0, kProbeBytes));
  uint32_t* words = static_cast<uint32_t*>(sc.p);
  int32_t* flag = reinterpret_cast<int32_t*>(words + kProbeWords);
  bool usable = false;
  VH_TRY(attn_probe_decide(q, ql, k, kl, v, vl, g, gl, mask, ml, sh, words, flag, s, &usable));
  if (!usable) return VH_OK;
  int32_t f = 0;
  VH_HIP(hipMemcpyAsync(&f, flag, sizeof(f), hipMemcpyDeviceToHost, s));
  VH_HIP(hipStreamSynchronize(s));
  *is_causal = f == 1 ? 1 : 0;
  return VH_OK;
}

int vh_fused_attention_fwd(const float* q, const vh_layout* ql, const float* k, const vh_layout* kl,
                           const float* v, const vh_layout* vl, const float* mask, const vh_layout* ml,
                           int causal, float* out, const vh_layout* ol, void* scratch, size_t scratch_bytes,
                           void* stream) {
  VH_TRY(require_init());
  AttnShape sh;
  VH_TRY(attn_layout(ql, "fused attention q", &sh, true));
  VH_TRY(attn_layout(kl, "fused attention k", &sh, false));
  VH_TRY(attn_layout(vl, "fused attention v", &sh, false));
  VH_TRY(attn_layout(ol, "fused attention out", &sh, false));
  int64_t mst[4] = {0, 0, 0, 0};
  if (mask) VH_TRY(attn_mask(ml, sh, mst));
  if (sh.B * sh.H * sh.S * sh.Dk == 0) return VH_OK;
  if (!q || !k || !v || !out) return fail(VH_ERR_INVALID, "vh_fused_attention_fwd: null pointer");
  if (sh.S > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_fused_attention_fwd: S too large");
  if (causal < 0 || causal > VH_ATTN_CAUSAL_AUTO) return fail(VH_ERR_INVALID, "vh_fused_attention_fwd: bad causal mode");
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_fused_attention_scratch_bytes(sh.B, sh.H, sh.S, 0)));
  float* P = static_cast<float*>(sc.p);
  // AUTO: the probe's verdict stays on the device; the launches below read it.
  Scratch pb;
  const int32_t* dflag = nullptr;
  if (causal == VH_ATTN_CAUSAL_AUTO) {
    causal = 0;
    if (mask) {
      VH_TRY(pb.get(s, nullptr, 0, kProbeBytes));
      uint32_t* words = static_cast<uint32_t*>(pb.p);
      int32_t* flag = reinterpret_cast<int32_t*>(words + kProbeWords);
      bool usable = false;
      VH_TRY(attn_probe_decide(q, ql, k, kl, v, vl, nullptr, nullptr, mask, ml, sh, words, flag, s, &usable));
      if (usable) {
        causal = 1;
        dflag = flag;
      }
    }
  }
  CausalFlagScope fs(dflag);
  VH_TRY(attn_probs(q, ql, k, kl, mask, mst, causal, sh, P, s));
  vh_gemm_desc d{};  // out = P v
  d.M = sh.S;
  d.N = sh.Dk;
  d.K = sh.S;
  d.a = P;
  d.a_sm = sh.S;
  d.a_sk = 1;
  d.b = v;  // B[k=j][n=d] = v[j][d]
  d.b_sk = vl->strides[2];
  d.b_sn = 1;
  d.c = out;
  d.c_sm = ol->strides[2];
  d.batch[0] = sh.B;
  d.batch[1] = sh.H;
  d.a_sb[0] = sh.H * sh.S * sh.S;
  d.a_sb[1] = sh.S * sh.S;
  d.b_sb[0] = vl->strides[0];
  d.b_sb[1] = vl->strides[1];
  d.c_sb[0] = ol->strides[0];
  d.c_sb[1] = ol->strides[1];
  d.alpha = 1.0f;
  d.causal = causal ? VH_GEMM_K_LE_M : VH_GEMM_DENSE;
  return vh_gemm(&d, s);
}

int vh_fused_attention_bwd(const float* q, const vh_layout* ql, const float* k, const vh_layout* kl,
                           const float* v, const vh_layout* vl, const float* mask, const vh_layout* ml,
                           int causal, const float* dout, const vh_layout* dol, float* dq,
                           const vh_layout* dql, float* dk, const vh_layout* dkl, float* dv,
                           const vh_layout* dvl, void* scratch, size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  AttnShape sh;
  VH_TRY(attn_layout(ql, "fused attention q", &sh, true));
  VH_TRY(attn_layout(kl, "fused attention k", &sh, false));
  VH_TRY(attn_layout(vl, "fused attention v", &sh, false));
  VH_TRY(attn_layout(dol, "fused attention grad_out", &sh, false));
  VH_TRY(attn_layout(dql, "fused attention dq", &sh, false));
  VH_TRY(attn_layout(dkl, "fused attention dk", &sh, false));
  VH_TRY(attn_layout(dvl, "fused attention dv", &sh, false));
  int64_t mst[4] = {0, 0, 0, 0};
  if (mask) VH_TRY(attn_mask(ml, sh, mst));
  if (sh.B * sh.H * sh.S * sh.Dk == 0) return VH_OK;
  if (!q || !k || !v || !dout || !dq || !dk || !dv)
    return fail(VH_ERR_INVALID, "vh_fused_attention_bwd: null pointer");
  if (sh.S > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_fused_attention_bwd: S too large");
  if (causal < 0 || causal > VH_ATTN_CAUSAL_AUTO) return fail(VH_ERR_INVALID, "vh_fused_attention_bwd: bad causal mode");
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_fused_attention_scratch_bytes(sh.B, sh.H, sh.S, 1)));
  float* P = static_cast<float*>(sc.p);
  float* G = P + vh_fused_attention_scratch_bytes(sh.B, sh.H, sh.S, 0) / sizeof(float);
  Scratch pb;
  const int32_t* dflag = nullptr;
  if (causal == VH_ATTN_CAUSAL_AUTO) {
    causal = 0;
    if (mask) {
      VH_TRY(pb.get(s, nullptr, 0, kProbeBytes));
      uint32_t* words = static_cast<uint32_t*>(pb.p);
      int32_t* flag = reinterpret_cast<int32_t*>(words + kProbeWords);
      bool usable = false;
      VH_TRY(attn_probe_decide(q, ql, k, kl, v, vl, dout, dol, mask, ml, sh, words, flag, s, &usable));
      if (usable) {
        causal = 1;
        dflag = flag;
      }
    }
  }
  CausalFlagScope fs(dflag);
  // P, recomputed from q and k as the reference does (cpu:2520-2569).
  VH_TRY(attn_probs(q, ql, k, kl, mask, mst, causal, sh, P, s));
  return attn_bwd_from_probs(P, G, q, ql, k, kl, v, vl, causal, dout, dol, dq, dql, dk, dkl, dv, dvl, sh, s);
}

int vh_fused_attention_bwd_probs(const float* P, const float* q, const vh_layout* ql, const float* k,
                                 const vh_layout* kl, const float* v, const vh_layout* vl, int causal,
                                 const float* dout, const vh_layout* dol, float* dq, const vh_layout* dql,
                                 float* dk, const vh_layout* dkl, float* dv, const vh_layout* dvl, void* scratch,
                                 size_t scratch_bytes, void* stream) {
  VH_TRY(require_init());
  AttnShape sh;
  VH_TRY(attn_layout(ql, "fused attention q", &sh, true));
  VH_TRY(attn_layout(kl, "fused attention k", &sh, false));
  VH_TRY(attn_layout(vl, "fused attention v", &sh, false));
  VH_TRY(attn_layout(dol, "fused attention grad_out", &sh, false));
  VH_TRY(attn_layout(dql, "fused attention dq", &sh, false));
  VH_TRY(attn_layout(dkl, "fused attention dk", &sh, false));
  VH_TRY(attn_layout(dvl, "fused attention dv", &sh, false));
  if (sh.B * sh.H * sh.S * sh.Dk == 0) return VH_OK;
  if (!P || !q || !k || !v || !dout || !dq || !dk || !dv)
    return fail(VH_ERR_INVALID, "vh_fused_attention_bwd_probs: null pointer");
  if (sh.S > INT32_MAX) return fail(VH_ERR_UNSUPPORTED, "vh_fused_attention_bwd_probs: S too large");
  hipStream_t s = S(stream);
  Scratch sc;
  VH_TRY(sc.get(S(stream), scratch, scratch_bytes, vh_fused_attention_scratch_bytes(sh.B, sh.H, sh.S, 0)));
  return attn_bwd_from_probs(P, static_cast<float*>(sc.p), q, ql, k, kl, v, vl, causal, dout, dol, dq, dql, dk,
                             dkl, dv, dvl, sh, s);
}

// ----------------------------------------------------------------- AdamW --

// f32::powi lowers to compiler-rt's __powisf2: binary exponentiation in f32.
static float powi_f32(float a, int b) {
  const bool recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

namespace {
// AdamW's hyper-parameters as the kernels take them (f32 roundings of the
// reference's: 1 - beta, 1 - beta^t, lr * weight_decay).
AdamArgs adam_hyper(int32_t t, float lr, float beta1, float beta2, float eps, float weight_decay) {
  AdamArgs a{};
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.omb1 = 1.0f - beta1;
  a.omb2 = 1.0f - beta2;
  a.bc1 = 1.0f - powi_f32(beta1, t);
  a.bc2 = 1.0f - powi_f32(beta2, t);
  a.lr = lr;
  a.lrwd = lr * weight_decay;
  a.eps = eps;
  return a;
}
}  // namespace

int vh_adamw_step_multi(int count, float* const* params, const float* const* grads, float* const* ms,
                        float* const* vs, const int64_t* ns, int32_t t, float lr, float beta1, float beta2, float eps,
                        float weight_decay, void* stream) {
  VH_TRY(require_init());
  if (count < 0) return fail(VH_ERR_INVALID, "vh_adamw_step_multi: negative count");
  if (t < 1) return fail(VH_ERR_INVALID, "vh_adamw_step: step count t must be >= 1");
  if (count > 0 && (!params || !grads || !ms || !vs || !ns))
    return fail(VH_ERR_INVALID, "vh_adamw_step_multi: null array");
  for (int i = 0; i < count; ++i) {
    if (ns[i] < 0) return fail(VH_ERR_INVALID, "vh_adamw_step: negative size");
    if (ns[i] > 0 && (!params[i] || !grads[i] || !ms[i] || !vs[i]))
      return fail(VH_ERR_INVALID, "vh_adamw_step: null pointer");
  }
  AdamMultiArgs a{};
  a.h = adam_hyper(t, lr, beta1, beta2, eps, weight_decay);
  hipStream_t s = S(stream);
  // Tensors in groups of up to VH_ADAMW_MULTI_MAX per launch, one unit per
  // thread as vh_adamw_step; empty tensors take no blocks.
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (a.count == 0) return VH_OK;
    const int rc = launch("vh_adamw_multi", blocks, 1, 256, 0, s, a);
    a.count = 0;
    blocks = 0;
    return rc;
  };
  for (int i = 0; i < count; ++i) {
    const int64_t n = ns[i];
    if (n == 0) continue;
    const bool vec = n % 4 == 0 && aligned16(params[i]) && aligned16(grads[i]) && aligned16(ms[i]) && aligned16(vs[i]);
    const int64_t nb = cdiv(vec ? n / 4 : n, 256);
    if (nb > INT32_MAX / 2) return fail(VH_ERR_UNSUPPORTED, "vh_adamw_step_multi: tensor too large");
    if (a.count == VH_ADAMW_MULTI_MAX || blocks + nb > INT32_MAX / 2) VH_TRY(flush());
    a.seg[a.count] = AdamSeg{params[i], grads[i], ms[i], vs[i], n, (int32_t)blocks, vec ? 1 : 0};
    ++a.count;
    blocks += nb;
  }
  return flush();
}

int vh_adamw_step(float* param, const float* grad, float* m, float* v, int64_t n, int32_t t, float lr,
                  float beta1, float beta2, float eps, float weight_decay, void* stream) {
  VH_TRY(require_init());
  if (n < 0) return fail(VH_ERR_INVALID, "vh_adamw_step: negative size");
  if (t < 1) return fail(VH_ERR_INVALID, "vh_adamw_step: step count t must be >= 1");
  if (n == 0) return VH_OK;
  if (!param || !grad || !m || !v) return fail(VH_ERR_INVALID, "vh_adamw_step: null pointer");
  AdamArgs a = adam_hyper(t, lr, beta1, beta2, eps, weight_decay);
  a.p = param;
  a.g = grad;
  a.m = m;
  a.v = v;
  a.n = n;
  const bool vec = n % 4 == 0 && aligned16(param) && aligned16(grad) && aligned16(m) && aligned16(v);
  // One unit per thread: over the 85 M parameters of the block step this runs
  // at 6.1 TB/s, against 5.3 TB/s for a grid of 8192 workgroups striding
  // (measured). The kernel keeps its stride loop for sizes past the grid limit.
  const int64_t blocks = std::min<int64_t>(cdiv(n / (vec ? 4 : 1), 256), INT32_MAX);
  return launch(vec ? "vh_adamw_v4" : "vh_adamw_v1", blocks, 1, 256, 0, S(stream), a);
}

}  // extern "C"
