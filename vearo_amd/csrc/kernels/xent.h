// xent.h -- cross-entropy forward / backward over [B, V] logits for gfx950.
//
// Semantics: vearo-backend-cpu cross_entropy (crates/vearo-backend-cpu/src/lib.rs:982-1051):
// per row max (from -inf), sum of exp(l - max), log_softmax = l[t] - max - ln(sum);
// loss = -(sum over rows of log_softmax) / B, returned as one float.
// cross_entropy_backward (lib.rs:1053-1127): dl = go * (p - 1[c == t]) / B with
// p = exp(l - max) / sum. Targets are f32 class ids, rounded like Rust's round().
// The kernels evaluate it as (p - 1[c == t]) * (go / B) with go / B rounded once
// per row: one correctly rounded division per element (p) instead of two. The
// same bits as the reference's order when B is a power of two (the scaling is
// then exact), within one rounding of it otherwise. Measured at [16384, 50257]
// the second division cost about 8% of the backward's time.
//
// Layout: logits / dlogits [B, V] with row stride ld (>= V), targets [B], one
// 512-thread workgroup (8 waves) per row. When V <= 512*128 the row is held in
// VGPRs and read from HBM once (fwd 4 B/elem read; bwd 4 B read + 4 B write). Longer rows
// take the streaming variant: one online max/sum pass, plus a write pass in bwd.
// The scalar per-row log_softmax values are reduced by xent_reduce in a fixed
// order, so the loss is deterministic. MODE 2 does forward and backward in one
// read of the row (for a caller that knows grad_out before the forward, as the
// training step does: the seed gradient of backward() is 1): the same row
// loss and the same dlogits as MODE 0 and MODE 1. The forwards can also write
// each row's (max, sum-exp); xent_bwd_rs*_impl is then the backward as a flat
// stream from them, with MODE 1's bits.
#pragma once
#include "common.h"

VH_DEV int32_t xent_target(const XentArgs& a, int64_t row) {
  const float tv = a.targets[row];
  const int32_t t = checked_index(tv, a.V);
  if (t < 0 && threadIdx.x == 0) {
    atomicMin(&a.err->target, err_pack(row, tv));
    a.err->target_bound = (unsigned)a.V;
  }
  return t;
}

// Word 3 of a raw (untyped, stride 0) buffer resource on CDNA: bounds-checked
// by byte offset against num_records, out-of-range loads return 0 and
// out-of-range stores are dropped.
#define VH_BUF_WORD3 0x00020000

// Row-cached kernels: a team of XE_TEAM threads per row, each holding NV
// values in VGPRs (two rows in flight per CU at the GPT-2 vocabulary). Units
// 0 .. NV - XE_MASK - 1 lie inside the row for every thread (the host picks NV
// with NV - XE_MASK < ceil(V / XE_TEAM) <= NV); only the last XE_MASK are
// masked (-inf, so exp gives 0).
#define XE_TEAM 512
#define XE_MASK 8
template <int NV, int MODE>  // 0 forward, 1 backward, 2 both
VH_DEV void xent_cached_impl(const XentArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int V = a.V;
  const float* lr = a.logits + row * a.ld;
  // One buffer resource per row: base and bound live in SGPRs, the unit offset
  // k * XE_TEAM * 4 goes in the scalar offset field, so the cached row costs
  // one VGPR per float and no per-load address registers.
  const __amdgpu_buffer_rsrc_t rin =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(lr), 0, V * 4, VH_BUF_WORD3);
  const int voff = threadIdx.x * 4;
  float v[NV];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    // The builtin returns the raw 32 bits: reinterpret, do not convert.
    // Unit offset k * 2048 B as (k / 2) * 4096 in the scalar offset plus
    // (k % 2) * 2048 folded into the instruction's immediate: half as many
    // scalar constants live across the burst of loads.
    const float x = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rin, voff + (k & 1) * XE_TEAM * 4, (k >> 1) * XE_TEAM * 8, 0));
    // tid < V - k * XE_TEAM: the bound is a scalar, no per-unit index register.
    v[k] = (k < NV - XE_MASK || (int)threadIdx.x < V - k * XE_TEAM) ? x : -INFINITY;
  }
  // Every load issued before the max chain starts consuming them.
  __builtin_amdgcn_sched_barrier(0);
  const int32_t t = xent_target(a, row);
  // MODE 2 reads the target logit here, before the team barriers below: the
  // row's gradient stores come after them, so dlogits may alias logits.
  float lt = 0.0f;
  if constexpr (MODE == 2) {
    if (threadIdx.x == 0 && t >= 0) lt = lr[t];
  }
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if (v[k] > m) m = v[k];
  m = team_max<XE_TEAM>(m, red);
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const float e = expf(v[k] - m);
    v[k] = e;
    s += e;
  }
  s = team_sum<XE_TEAM>(s, red);
  if constexpr (MODE == 0) {
    if (threadIdx.x == 0) {
      a.out[row] = t >= 0 ? lr[t] - m - logf(s) : 0.0f;
      if (a.stats) *reinterpret_cast<float2*>(a.stats + 2 * row) = make_float2(m, s);
    }
  }
  if constexpr (MODE != 0) {
    __builtin_amdgcn_sched_barrier(0);
    const float c = *a.grad_out / (float)a.B;
    const __amdgpu_buffer_rsrc_t rout =
        __builtin_amdgcn_make_buffer_rsrc(a.out + row * a.ld, 0, V * 4, VH_BUF_WORD3);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const float p = v[k] / s;
      const float ind = (int)threadIdx.x == t - k * XE_TEAM ? 1.0f : 0.0f;
      // Units past the row end fall outside the resource and are dropped.
      const float g = (p - ind) * c;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, g), rout, voff + (k & 1) * XE_TEAM * 4,
                                            (k >> 1) * XE_TEAM * 8, 0);
      // At most 2 elements' correctly rounded divisions in flight: their
      // temporaries then fit beside the cached row without spilling.
      if (k & 1) __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (MODE == 2) {  // after the row's registers are free
    if (threadIdx.x == 0) a.row_loss[row] = t >= 0 ? lt - m - logf(s) : 0.0f;
  }
}

// Any V: per-thread online max / rescaled sum, merged across the workgroup.
template <bool BWD>
VH_DEV void xent_stream_impl(const XentArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int V = a.V;
  const float* lr = a.logits + row * a.ld;
  float m = -INFINITY, s = 0.0f;
  for (int c = threadIdx.x; c < V; c += 1024) {
    const float x = lr[c];
    if (x > m) {
      s = s * expf(m - x) + 1.0f;
      m = x;
    } else if (x != -INFINITY) {
      s += expf(x - m);
    }
  }
  const float M = team_max<1024>(m, red);
  s = (m == -INFINITY) ? 0.0f : s * expf(m - M);
  s = team_sum<1024>(s, red);
  const int32_t t = xent_target(a, row);
  if constexpr (!BWD) {
    if (threadIdx.x == 0) {
      a.out[row] = t >= 0 ? lr[t] - M - logf(s) : 0.0f;
      if (a.stats) *reinterpret_cast<float2*>(a.stats + 2 * row) = make_float2(M, s);
    }
  } else {
    const float gs = *a.grad_out / (float)a.B;
    float* o = a.out + row * a.ld;
    for (int c = threadIdx.x; c < V; c += 1024) {
      const float p = expf(lr[c] - M) / s;
      const float ind = c == t ? 1.0f : 0.0f;
      o[c] = (p - ind) * gs;
    }
  }
}

// Backward from the forward's row statistics (stats[2 r] = the row max m,
// stats[2 r + 1] = the row's sum of exp(l - m), as the forward kernel of the
// same V computed them): dl = (expf(l - m) / s - 1[c == t]) * (go / B), the
// operations the backward kernels above apply after their reductions, so the
// same bits. Nothing is left to reduce, so the row need not be held in
// registers: a flat stream of short-lived workgroups, one per (row, chunk).
VH_DEV float xent_rs_grad(float x, int i, int32_t t, float2 st, float c) {
  const float p = expf(x - st.x) / st.y;
  const float ind = i == t ? 1.0f : 0.0f;
  return (p - ind) * c;
}

// 16-byte form (logits and dlogits 16-byte aligned): per row, the head
// elements before the first 16-byte boundary and the 0-3 tail elements are
// done by threads 0-7 of chunk 0; the rest as 16-byte units, XR4_PER per
// thread, streaming (non-temporal) loads and stores. At [16384, 50257]
// (MI355X): 256 threads x 2 units 1131 us; 4 units 1178, 8 units 1247, 1 unit
// 1358; 512 threads x 2 units 1164; cached-hint loads and stores 1159 us.
#define XR4_THREADS 256
#define XR4_PER 2
#define XR4_CHUNK (XR4_THREADS * XR4_PER)  // 16-byte units per workgroup
VH_DEV void xent_bwd_rs4_impl(const XentArgs& a) {
  const int V = a.V;
  const uint32_t nch = (uint32_t)((V / 4 + 1 + XR4_CHUNK - 1) / XR4_CHUNK);
  const uint32_t row32 = blockIdx.x / nch;
  const int u0 = (int)(blockIdx.x - row32 * nch) * XR4_CHUNK;
  const int64_t row = row32;
  const float2 st = *reinterpret_cast<const float2*>(a.stats + 2 * row);
  const int32_t t = xent_target(a, row);
  const float c = *a.grad_out / (float)a.B;
  const int64_t base = row * a.ld;
  const int hv = min((int)((4 - (base & 3)) & 3), V);  // head elements
  const int nvec = (V - hv) / 4;
  const float* lr = a.logits + base;
  float* o = a.out + base;
  const int tid = threadIdx.x;
  if (u0 == 0 && tid < 8) {
    const int i = tid < 4 ? tid : hv + 4 * nvec + (tid - 4);
    if (tid < 4 ? tid < hv : i < V) o[i] = xent_rs_grad(lr[i], i, t, st, c);
  }
  const float* l4 = lr + hv;
  float* o4 = o + hv;
  Unit<4> x[XR4_PER];
#pragma unroll
  for (int k = 0; k < XR4_PER; ++k) {
    const int u = u0 + k * XR4_THREADS + tid;
    x[k] = u < nvec ? load_stream<4>(l4 + 4 * u) : zero_unit<4>();
  }
#pragma unroll
  for (int k = 0; k < XR4_PER; ++k) {
    const int u = u0 + k * XR4_THREADS + tid;
    if (u < nvec) {
      Unit<4> r;
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[j] = xent_rs_grad(x[k].v[j], hv + 4 * u + j, t, st, c);
      store_stream<4>(o4 + 4 * u, r);
    }
  }
}

// Any alignment: 32-bit elements, XR_PER per thread, lane-contiguous.
#define XR_THREADS 256
#define XR_PER 16
#define XR_CHUNK (XR_THREADS * XR_PER)  // elements per workgroup
VH_DEV void xent_bwd_rs_impl(const XentArgs& a) {
  const int V = a.V;
  const uint32_t nch = (uint32_t)((V + XR_CHUNK - 1) / XR_CHUNK);
  const uint32_t row32 = blockIdx.x / nch;
  const int c0 = (int)(blockIdx.x - row32 * nch) * XR_CHUNK;
  const int64_t row = row32;
  const float2 st = *reinterpret_cast<const float2*>(a.stats + 2 * row);
  const int32_t t = xent_target(a, row);
  const float c = *a.grad_out / (float)a.B;
  const float* lr = a.logits + row * a.ld;
  float* o = a.out + row * a.ld;
  const int n = V - c0;
  float x[XR_PER];
#pragma unroll
  for (int k = 0; k < XR_PER; ++k) {
    const int i = k * XR_THREADS + (int)threadIdx.x;
    x[k] = i < n ? lr[c0 + i] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < XR_PER; ++k) {
    const int i = k * XR_THREADS + (int)threadIdx.x;
    if (i < n) o[c0 + i] = xent_rs_grad(x[k], c0 + i, t, st, c);
  }
}

// loss = -(sum of per-row log_softmax) / B; one 1024-thread workgroup, each
// thread sums a strided subset in order, then a fixed tree.
VH_DEV void xent_reduce_impl(const XentReduceArgs& a) {
  __shared__ float red[16];
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < a.B; i += 1024) s += a.row_loss[i];
  s = team_sum<1024>(s, red);
  if (threadIdx.x == 0) a.loss[0] = -s / (float)a.B;
}
