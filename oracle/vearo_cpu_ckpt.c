/*
 * vearo_cpu_ckpt.c -- CPU oracle for the `.ve` weight checkpoint
 * (crates/vearo/src/checkpoint.rs:9-91). TEST INFRASTRUCTURE ONLY, like the
 * rest of oracle/: tests compare the device checkpoint path's files and loaded
 * tensors with this one.
 *
 * Host tensors: data pointers with vo_layout dims/strides. Values go through
 * the file one u32 / f32 at a time, little-endian, in the reference's order.
 */
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "vearo_cpu_ref.h"

static int ck_fail(int code, char* err, size_t errlen, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return code;
}

/* Tensor::is_contiguous: strides equal the row-major ones (tensor.rs:335-337). */
static int ck_contiguous(const vo_layout* l) {
  int64_t acc = 1;
  for (int i = l->rank - 1; i >= 0; --i) {
    if (l->strides[i] != acc) return 0;
    acc *= l->dims[i];
  }
  return 1;
}

static int64_t ck_numel(const vo_layout* l) {
  int64_t n = 1;
  for (int i = 0; i < l->rank; ++i) n *= l->dims[i];
  return n;
}

static int w32(FILE* f, uint32_t v) {
  const unsigned char b[4] = {v & 0xff, (v >> 8) & 0xff, (v >> 16) & 0xff, v >> 24};
  return fwrite(b, 1, 4, f) == 4;
}

static int r32(FILE* f, uint32_t* v) {
  unsigned char b[4];
  if (fread(b, 1, 4, f) != 4) return 0;
  *v = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
  return 1;
}

/* save_checkpoint (checkpoint.rs:9-33): count, then per tensor rank, dims,
 * numel and the values of to_vec_f32() (which asserts contiguity,
 * tensor.rs:751-755). */
int vo_checkpoint_save(const char* path, int n, const float* const* data, const vo_layout* layouts, char* err,
                       size_t errlen) {
  FILE* f = fopen(path, "wb");
  if (!f) return ck_fail(VO_IOERR, err, errlen, "create %s: %s", path, strerror(errno));
  int ok = w32(f, (uint32_t)n);
  for (int i = 0; ok && i < n; ++i) {
    const vo_layout* l = &layouts[i];
    ok = w32(f, (uint32_t)l->rank);
    for (int d = 0; ok && d < l->rank; ++d) ok = w32(f, (uint32_t)l->dims[d]);
    if (!ck_contiguous(l)) {
      fclose(f);
      return ck_fail(VO_PANIC, err, errlen, "to_vec_f32 requires contiguous tensor");
    }
    const int64_t ne = ck_numel(l);
    ok = ok && w32(f, (uint32_t)ne);
    for (int64_t k = 0; ok && k < ne; ++k) {
      uint32_t bits;
      memcpy(&bits, &data[i][k], 4);
      ok = w32(f, bits);
    }
  }
  if (fclose(f) != 0) ok = 0;
  if (!ok) return ck_fail(VO_IOERR, err, errlen, "write %s failed", path);
  return VO_OK;
}

/* load_checkpoint (checkpoint.rs:40-91): count check, then per tensor the dims
 * (all read, then compared), numel, the values (read in full first), and
 * copy_from_slice's checks (tensor.rs:816-826). */
int vo_checkpoint_load(const char* path, int n, float* const* data, const vo_layout* layouts, char* err,
                       size_t errlen) {
  FILE* f = fopen(path, "rb");
  if (!f) return ck_fail(VO_IOERR, err, errlen, "open %s: %s", path, strerror(errno));
  int rc = VO_OK;
  uint32_t count;
  if (!r32(f, &count)) {
    rc = ck_fail(VO_IOERR, err, errlen, "read %s: unexpected end of file", path);
    goto out;
  }
  if ((int64_t)count != n) {
    rc = ck_fail(VO_PANIC, err, errlen, "Checkpoint tensor count does not match model parameter count");
    goto out;
  }
  for (int i = 0; i < n; ++i) {
    const vo_layout* l = &layouts[i];
    uint32_t rank, v, len;
    if (!r32(f, &rank)) {
      rc = ck_fail(VO_IOERR, err, errlen, "read %s: unexpected end of file", path);
      goto out;
    }
    int same = (int64_t)rank == l->rank;
    for (uint32_t d = 0; d < rank; ++d) {
      if (!r32(f, &v)) {
        rc = ck_fail(VO_IOERR, err, errlen, "read %s: unexpected end of file", path);
        goto out;
      }
      same = same && (int)d < l->rank && (int64_t)v == l->dims[d];
    }
    if (!same) {
      rc = ck_fail(VO_PANIC, err, errlen, "Checkpoint shape does not match parameter shape");
      goto out;
    }
    if (!r32(f, &len)) {
      rc = ck_fail(VO_IOERR, err, errlen, "read %s: unexpected end of file", path);
      goto out;
    }
    const int64_t ne = ck_numel(l);
    const int fits = ck_contiguous(l) && (int64_t)len == ne;
    for (uint32_t k = 0; k < len; ++k) {
      if (!r32(f, &v)) {
        rc = ck_fail(VO_IOERR, err, errlen, "read %s: unexpected end of file", path);
        goto out;
      }
      if (fits) memcpy(&data[i][k], &v, 4);
    }
    if (!ck_contiguous(l)) {
      rc = ck_fail(VO_PANIC, err, errlen, "copy_from_slice requires contiguous tensor");
      goto out;
    }
    if ((int64_t)len != ne) {
      rc = ck_fail(VO_PANIC, err, errlen, "Source slice length must match tensor numel");
      goto out;
    }
  }
out:
  fclose(f);
  return rc;
}
