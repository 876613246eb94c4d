// softmax.h -- row softmax forward / fused backward for gfx950, with an optional
// causal row structure.
//
// Forward semantics: vearo-backend-cpu softmax (crates/vearo-backend-cpu/src/lib.rs:499-563):
// max (strict >, from -inf), sum of exp(v-max), y = exp(v-max)/sum (a division).
// Backward semantics: the autograd Softmax arm (crates/vearo-autograd/src/lib.rs:547-553)
// y = softmax(x); s = sum(dy*y); dx = y*(dy - s), fused into one pass.
//
// Layout: [rows, T] row-major; a TEAM of lanes owns one row held in VGPRs and
// takes RPW rows, issuing all their loads before the reductions.
// causal = 1: row r is query (r % T) of a T x T score block, so only columns
// [0, r % T] are live; the masked tail is never read and written as exact 0,
// which is what exp() gives the reference for -inf (or -1e9 additive) entries.
// Traffic: fwd reads the live prefix and writes the row (4f+4 B/elem, f = live
// fraction); bwd reads the live prefix of y (or x) and dy, writes dx. All row
// traffic is non-temporal (single use). Rows are held whole in registers before
// anything is written, so in == out (in place) is allowed.
// ztile > 0 (the fused attention's own score block only): the masked zeros of a
// causal row are written only up to the end of its ztile-row tile, the part
// the causal products read; the tiles wholly above the diagonal are left as
// they are (44 % of the row writes at T = 1024).
// attn = 1 follows the CPU fused attention instead (cpu:2451-2458, 2583-2590):
// p = e * inv with inv = 1/(sum + 1e-9), and the backward's sum of dy*y is a
// fused multiply-add chain.
#pragma once
#include "common.h"

// The launch's causal mode: a.causal, unless a device flag says the rows are dense.
VH_DEV int sm_causal(const SoftmaxArgs& a) { return (a.causal_flag && *a.causal_flag == 0) ? 0 : a.causal; }

// End of the columns a row writes, given its live length L (causal: L - 1 is
// the row's index in its T x T block).
VH_DEV int zero_end(const SoftmaxArgs& a, int causal, int L) {
  if (!causal || a.ztile <= 0) return a.T;
  const int e = ((L - 1) / a.ztile + 1) * a.ztile;
  return e < a.T ? e : a.T;
}

template <int TEAM, int NV, int VW, int RPW>
VH_DEV void softmax_fwd_impl(const SoftmaxArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int TPB = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row0 = ((int64_t)blockIdx.x * TPB + threadIdx.x / TEAM) * RPW;
  const int T = a.T;
  const int U = T / VW;
  const int causal = sm_causal(a);

  Unit<VW> v[RPW][NV];
  int L[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool active = row < a.rows;
    L[r] = causal ? (int)(row % T) + 1 : T;  // live length
    const float* xr = a.x + (active ? row : 0) * (int64_t)T;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      const bool live = active && u < U && u * VW < L[r];
      v[r][k] = live ? load_stream<VW>(xr + u * VW) : zero_unit<VW>();
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool active = row < a.rows;
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      const bool live = active && u < U && u * VW < L[r];
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        if (!live || u * VW + j >= L[r]) v[r][k].v[j] = -INFINITY;
        if (v[r][k].v[j] > m) m = v[r][k].v[j];
      }
    }
    m = team_max<TEAM>(m, red);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U && u * VW < L[r]) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float e = (u * VW + j < L[r]) ? expf(v[r][k].v[j] - m) : 0.0f;
          v[r][k].v[j] = e;
          s += e;
        }
      }
    }
    s = team_sum<TEAM>(s, red);
    const float inv = 1.0f / (s + 1e-9f);
    if (active) {
      float* yr = a.y + row * (int64_t)T;
      const int Z = zero_end(a, causal, L[r]);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int u = lane + k * TEAM;
        if (u < U && u * VW < Z) {
          Unit<VW> o;
#pragma unroll
          for (int j = 0; j < VW; ++j)
            o.v[j] = (u * VW + j < L[r]) ? (a.attn ? v[r][k].v[j] * inv : v[r][k].v[j] / s) : 0.0f;
          store_stream<VW>(yr + u * VW, o);
        }
      }
    }
  }
}

template <int TEAM, int NV, int VW, int RPW>
VH_DEV void softmax_bwd_impl(const SoftmaxArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int TPB = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row0 = ((int64_t)blockIdx.x * TPB + threadIdx.x / TEAM) * RPW;
  const int T = a.T;
  const int U = T / VW;
  const int causal = sm_causal(a);

  Unit<VW> y[RPW][NV], g[RPW][NV];
  int L[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool active = row < a.rows;
    L[r] = causal ? (int)(row % T) + 1 : T;
    const int64_t off = (active ? row : 0) * (int64_t)T;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      const bool live = active && u < U && u * VW < L[r];
      y[r][k] = live ? load_stream<VW>(a.x + off + u * VW) : zero_unit<VW>();
      g[r][k] = live ? load_stream<VW>(a.dy + off + u * VW) : zero_unit<VW>();
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool active = row < a.rows;
    if (a.input_is_x) {
      // Recompute y exactly as the forward does.
      float m = -INFINITY;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int u = lane + k * TEAM;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          if (u < U && u * VW + j < L[r] && y[r][k].v[j] > m) m = y[r][k].v[j];
        }
      }
      m = team_max<TEAM>(m, red);
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int u = lane + k * TEAM;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float e = (u < U && u * VW + j < L[r]) ? expf(y[r][k].v[j] - m) : 0.0f;
          y[r][k].v[j] = e;
          s += e;
        }
      }
      s = team_sum<TEAM>(s, red);
      const float inv = 1.0f / (s + 1e-9f);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
#pragma unroll
        for (int j = 0; j < VW; ++j) y[r][k].v[j] = a.attn ? y[r][k].v[j] * inv : y[r][k].v[j] / s;
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        if (u < U && u * VW + j < L[r])
          dot = a.attn ? __builtin_fmaf(g[r][k].v[j], y[r][k].v[j], dot) : dot + g[r][k].v[j] * y[r][k].v[j];
      }
    }
    dot = team_sum<TEAM>(dot, red);
    if (active) {
      float* dxr = a.y + row * (int64_t)T;
      const int Z = zero_end(a, causal, L[r]);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int u = lane + k * TEAM;
        if (u < U && u * VW < Z) {
          Unit<VW> o;
#pragma unroll
          for (int j = 0; j < VW; ++j)
            o.v[j] = (u * VW + j < L[r]) ? y[r][k].v[j] * (g[r][k].v[j] - dot) : 0.0f;
          store_stream<VW>(dxr + u * VW, o);
        }
      }
    }
  }
}
