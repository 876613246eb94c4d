// checkpoint.cpp -- `.ve` weight checkpoints of device tensors
// (crates/vearo/src/checkpoint.rs:9-91).
//
// File layout, little-endian throughout (checkpoint.rs:12-27):
//   u32 count; per tensor: u32 rank, u32 dims[rank], u32 numel, f32 data[numel].
//
// The reference pulls each tensor to a host Vec (to_vec_f32) and writes it
// through a BufWriter; on load it reads a whole Vec and copy_from_slice()s it
// to the device. Here the data streams in chunks through two pinned host
// buffers: while one chunk is copied between device and host on the stream,
// the other is written to (or read from) the file, so a 340 MB parameter set
// moves at the slower of PCIe and the file system instead of their sum.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/vearo_hip.h"
#include "rt_internal.h"

namespace {

using vh_rt::fail;

constexpr size_t kChunk = size_t(32) << 20;  // bytes per staging buffer

#define CK_HIP(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(VH_ERR_HIP, std::string(#expr) + " failed: " + hipGetErrorString(e_)); \
  } while (0)

#define CK_TRY(expr)                \
  do {                              \
    int rc_ = (expr);               \
    if (rc_ != VH_OK) return rc_;   \
  } while (0)

// Two pinned staging buffers and an event per buffer marking when the copy
// that last used it has finished. Released on scope exit after the copies.
struct Staging {
  unsigned char* buf[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};

  int init() {
    for (int i = 0; i < 2; ++i) {
      CK_HIP(hipHostMalloc(reinterpret_cast<void**>(&buf[i]), kChunk, hipHostMallocDefault));
      CK_HIP(hipEventCreateWithFlags(&done[i], hipEventDisableTiming));
    }
    return VH_OK;
  }
  // Waits for the copy that last used buffer i.
  int wait(int i) {
    if (pending[i]) {
      pending[i] = false;
      CK_HIP(hipEventSynchronize(done[i]));
    }
    return VH_OK;
  }
  ~Staging() {
    for (int i = 0; i < 2; ++i) {
      if (done[i]) {
        if (pending[i]) (void)hipEventSynchronize(done[i]);
        (void)hipEventDestroy(done[i]);
      }
      if (buf[i]) (void)hipHostFree(buf[i]);
    }
  }
};

struct File {
  std::FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

int io_error(const char* what, const char* path) {
  return fail(VH_ERR_IO, std::string(what) + " " + path + ": " + std::strerror(errno));
}

// The reference's Tensor::is_contiguous: strides equal to the row-major ones
// of the dims (tensor.rs:335-337, shape.rs:68-79).
bool contiguous(const vh_layout& l) {
  int64_t acc = 1;
  for (int i = l.rank - 1; i >= 0; --i) {
    if (l.strides[i] != acc) return false;
    acc *= l.dims[i];
  }
  return true;
}

int check_layout(const vh_layout* l, int i, const char* what) {
  if (l->rank < 0 || l->rank > VH_MAX_RANK)
    return fail(VH_ERR_INVALID, std::string(what) + ": tensor " + std::to_string(i) + " has rank out of range");
  for (int d = 0; d < l->rank; ++d)
    if (l->dims[d] < 0 || l->strides[d] < 0)
      return fail(VH_ERR_INVALID, std::string(what) + ": tensor " + std::to_string(i) + " has a negative dim or stride");
  return VH_OK;
}

int64_t numel_of(const vh_layout& l) {
  int64_t n = 1;
  for (int d = 0; d < l.rank; ++d) n *= l.dims[d];
  return n;
}

int put_u32(File& f, uint32_t v, const char* path) {
  unsigned char b[4] = {(unsigned char)(v & 0xff), (unsigned char)((v >> 8) & 0xff),
                        (unsigned char)((v >> 16) & 0xff), (unsigned char)(v >> 24)};
  if (std::fwrite(b, 1, 4, f.f) != 4) return io_error("write", path);
  return VH_OK;
}

// Reads a u32; a short file is the reference's read_exact error.
int get_u32(File& f, uint32_t* v, const char* path) {
  unsigned char b[4];
  if (std::fread(b, 1, 4, f.f) != 4) {
    if (std::ferror(f.f)) return io_error("read", path);
    return fail(VH_ERR_IO, std::string("read ") + path + ": unexpected end of file");
  }
  *v = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
  return VH_OK;
}

}  // namespace

extern "C" {

int vh_checkpoint_save(const char* path, int32_t n, const float* const* tensors, const vh_layout* layouts,
                       void* stream) {
  CK_TRY(vh_rt::require_init());
  if (!path) return fail(VH_ERR_INVALID, "vh_checkpoint_save: null path");
  if (n < 0) return fail(VH_ERR_INVALID, "vh_checkpoint_save: negative tensor count");
  if (n > 0 && (!tensors || !layouts)) return fail(VH_ERR_INVALID, "vh_checkpoint_save: null tensor list");
  // Every argument is checked before the file is created.
  for (int i = 0; i < n; ++i) {
    CK_TRY(check_layout(&layouts[i], i, "vh_checkpoint_save"));
    if (!contiguous(layouts[i])) return fail(VH_ERR_INVALID, "to_vec_f32 requires contiguous tensor");
    const int64_t ne = numel_of(layouts[i]);
    if (ne > 0 && !tensors[i]) return fail(VH_ERR_INVALID, "vh_checkpoint_save: null tensor pointer");
    bool fits = ne <= (int64_t)UINT32_MAX;
    for (int d = 0; d < layouts[i].rank; ++d) fits = fits && layouts[i].dims[d] <= (int64_t)UINT32_MAX;
    if (!fits)
      return fail(VH_ERR_UNSUPPORTED, "vh_checkpoint_save: tensor " + std::to_string(i) +
                                          " has a dim or element count beyond the format's u32");
  }
  const hipStream_t s = vh_rt::stream_of(stream);
  Staging st;
  CK_TRY(st.init());
  File f;
  f.f = std::fopen(path, "wb");
  if (!f.f) return io_error("create", path);
  CK_TRY(put_u32(f, (uint32_t)n, path));
  int next = 0;  // staging buffer the next chunk goes to
  for (int i = 0; i < n; ++i) {
    const vh_layout& l = layouts[i];
    CK_TRY(put_u32(f, (uint32_t)l.rank, path));
    for (int d = 0; d < l.rank; ++d) CK_TRY(put_u32(f, (uint32_t)l.dims[d], path));
    const size_t bytes = (size_t)numel_of(l) * sizeof(float);
    CK_TRY(put_u32(f, (uint32_t)numel_of(l), path));
    // Chunk c is copied into buffer `next` while chunk c-1 (in the other
    // buffer) is written to the file.
    const unsigned char* src = reinterpret_cast<const unsigned char*>(tensors[i]);
    size_t prev_len = 0;
    int prev = -1;
    for (size_t off = 0; off < bytes || prev >= 0;) {
      int cur = -1;
      size_t len = 0;
      if (off < bytes) {
        cur = next;
        len = bytes - off < kChunk ? bytes - off : kChunk;
        CK_TRY(st.wait(cur));
        CK_HIP(hipMemcpyAsync(st.buf[cur], src + off, len, hipMemcpyDeviceToHost, s));
        CK_HIP(hipEventRecord(st.done[cur], s));
        st.pending[cur] = true;
        next ^= 1;
        off += len;
      }
      if (prev >= 0) {
        CK_TRY(st.wait(prev));
        if (std::fwrite(st.buf[prev], 1, prev_len, f.f) != prev_len) return io_error("write", path);
      }
      prev = cur;
      prev_len = len;
    }
  }
  const int closed = std::fclose(f.f);
  f.f = nullptr;
  if (closed != 0) return io_error("close", path);
  return VH_OK;
}

int vh_checkpoint_load(const char* path, int32_t n, float* const* tensors, const vh_layout* layouts, void* stream) {
  CK_TRY(vh_rt::require_init());
  if (!path) return fail(VH_ERR_INVALID, "vh_checkpoint_load: null path");
  if (n < 0) return fail(VH_ERR_INVALID, "vh_checkpoint_load: negative tensor count");
  if (n > 0 && (!tensors || !layouts)) return fail(VH_ERR_INVALID, "vh_checkpoint_load: null tensor list");
  for (int i = 0; i < n; ++i) CK_TRY(check_layout(&layouts[i], i, "vh_checkpoint_load"));
  const hipStream_t s = vh_rt::stream_of(stream);
  File f;
  f.f = std::fopen(path, "rb");
  if (!f.f) return io_error("open", path);
  Staging st;
  CK_TRY(st.init());
  uint32_t count = 0;
  CK_TRY(get_u32(f, &count, path));
  if ((int64_t)count != (int64_t)n)
    return fail(VH_ERR_INVALID, "Checkpoint tensor count does not match model parameter count");
  int next = 0;
  for (int i = 0; i < n; ++i) {
    const vh_layout& l = layouts[i];
    uint32_t rank = 0;
    CK_TRY(get_u32(f, &rank, path));
    // The dims are all read before they are compared (checkpoint.rs:56-68).
    bool same = (int64_t)rank == l.rank;
    for (uint32_t d = 0; d < rank; ++d) {
      uint32_t v = 0;
      CK_TRY(get_u32(f, &v, path));
      same = same && (int)d < l.rank && (int64_t)v == l.dims[d];
    }
    if (!same) return fail(VH_ERR_INVALID, "Checkpoint shape does not match parameter shape");
    uint32_t len = 0;
    CK_TRY(get_u32(f, &len, path));
    const int64_t ne = numel_of(l);
    if (!contiguous(l) || (int64_t)len != ne) {
      // The reference reads the whole data block first (an I/O error if the
      // file is short), then copy_from_slice asserts (tensor.rs:817-826).
      // The earlier tensors' last copies still read the staging buffers: let
      // them finish before buffer 0 takes the discarded block, so those
      // tensors end fully loaded, as the reference leaves them.
      CK_TRY(st.wait(0));
      CK_TRY(st.wait(1));
      for (uint64_t left = (uint64_t)len * 4; left > 0;) {
        const size_t step = left < kChunk ? (size_t)left : kChunk;
        if (std::fread(st.buf[0], 1, step, f.f) != step) {
          if (std::ferror(f.f)) return io_error("read", path);
          return fail(VH_ERR_IO, std::string("read ") + path + ": unexpected end of file");
        }
        left -= step;
      }
      if (!contiguous(l)) return fail(VH_ERR_INVALID, "copy_from_slice requires contiguous tensor");
      return fail(VH_ERR_INVALID, "Source slice length must match tensor numel");
    }
    if (ne > 0 && !tensors[i]) return fail(VH_ERR_INVALID, "vh_checkpoint_load: null tensor pointer");
    // Chunk c is read from the file into buffer `next` while the copy of chunk
    // c-1 (from the other buffer) to the device runs.
    unsigned char* dst = reinterpret_cast<unsigned char*>(tensors[i]);
    const size_t bytes = (size_t)ne * sizeof(float);
    for (size_t off = 0; off < bytes;) {
      const int cur = next;
      const size_t step = bytes - off < kChunk ? bytes - off : kChunk;
      CK_TRY(st.wait(cur));
      if (std::fread(st.buf[cur], 1, step, f.f) != step) {
        if (std::ferror(f.f)) return io_error("read", path);
        return fail(VH_ERR_IO, std::string("read ") + path + ": unexpected end of file");
      }
      CK_HIP(hipMemcpyAsync(dst + off, st.buf[cur], step, hipMemcpyHostToDevice, s));
      CK_HIP(hipEventRecord(st.done[cur], s));
      st.pending[cur] = true;
      next ^= 1;
      off += step;
    }
  }
  CK_TRY(st.wait(0));
  CK_TRY(st.wait(1));
  return VH_OK;
}

}  // extern "C"
