// softmax.h -- row softmax forward / fused backward for gfx950, with an optional
// causal row structure.
//
// Forward semantics: vearo-backend-cpu softmax (crates/vearo-backend-cpu/src/lib.rs:499-563):
// max (strict >, from -inf), sum of exp(v-max), y = exp(v-max)/sum (a division).
// Backward semantics: the autograd Softmax arm (crates/vearo-autograd/src/lib.rs:547-553)
// y = softmax(x); s = sum(dy*y); dx = y*(dy - s), fused into one pass.
//
// Layout: [rows, T] row-major; a TEAM of lanes owns one row held in VGPRs.
// causal = 1: row r is query (r % T) of a T x T score block, so only columns
// [0, r % T] are live; the masked tail is never read and written as exact 0,
// which is what exp() gives the reference for -inf (or -1e9 additive) entries.
// Traffic: fwd reads the live prefix and writes the row (4f+4 B/elem, f = live
// fraction); bwd reads the live prefix of y (or x) and dy, writes dx.
#pragma once
#include "common.h"

template <int TEAM, int NV, int VW>
VH_DEV void softmax_fwd_impl(const SoftmaxArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int RPB = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TEAM;
  const bool active = row < a.rows;
  const int T = a.T;
  const int U = T / VW;
  const int L = a.causal ? (int)(row % T) + 1 : T;  // live length
  const float* xr = a.x + (active ? row : 0) * (int64_t)T;

  Unit<VW> v[NV];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    const bool live = active && u < U && u * VW < L;
    v[k] = live ? load_unit<VW>(xr + u * VW) : zero_unit<VW>();
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      if (!live || u * VW + j >= L) v[k].v[j] = -INFINITY;
      if (v[k].v[j] > m) m = v[k].v[j];
    }
  }
  m = team_max<TEAM>(m, red);
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    if (u < U && u * VW < L) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float e = (u * VW + j < L) ? expf(v[k].v[j] - m) : 0.0f;
        v[k].v[j] = e;
        s += e;
      }
    }
  }
  s = team_sum<TEAM>(s, red);
  if (!active) return;
  float* yr = a.y + row * (int64_t)T;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    if (u < U) {
      Unit<VW> o;
#pragma unroll
      for (int j = 0; j < VW; ++j) o.v[j] = (u * VW + j < L) ? v[k].v[j] / s : 0.0f;
      store_unit<VW>(yr + u * VW, o);
    }
  }
}

template <int TEAM, int NV, int VW>
VH_DEV void softmax_bwd_impl(const SoftmaxArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int RPB = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TEAM;
  const bool active = row < a.rows;
  const int T = a.T;
  const int U = T / VW;
  const int L = a.causal ? (int)(row % T) + 1 : T;
  const int64_t off = (active ? row : 0) * (int64_t)T;

  Unit<VW> y[NV], g[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    const bool live = active && u < U && u * VW < L;
    y[k] = live ? load_unit<VW>(a.x + off + u * VW) : zero_unit<VW>();
    g[k] = live ? load_unit<VW>(a.dy + off + u * VW) : zero_unit<VW>();
  }
  if (a.input_is_x) {
    // Recompute y exactly as the forward does.
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        if (u < U && u * VW + j < L && y[k].v[j] > m) m = y[k].v[j];
      }
    }
    m = team_max<TEAM>(m, red);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float e = (u < U && u * VW + j < L) ? expf(y[k].v[j] - m) : 0.0f;
        y[k].v[j] = e;
        s += e;
      }
    }
    s = team_sum<TEAM>(s, red);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
      for (int j = 0; j < VW; ++j) y[k].v[j] = y[k].v[j] / s;
    }
  }
  float dot = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      if (u < U && u * VW + j < L) dot += g[k].v[j] * y[k].v[j];
    }
  }
  dot = team_sum<TEAM>(dot, red);
  if (!active) return;
  float* dxr = a.y + row * (int64_t)T;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    if (u < U) {
      Unit<VW> o;
#pragma unroll
      for (int j = 0; j < VW; ++j)
        o.v[j] = (u * VW + j < L) ? y[k].v[j] * (g[k].v[j] - dot) : 0.0f;
      store_unit<VW>(dxr + u * VW, o);
    }
  }
}
