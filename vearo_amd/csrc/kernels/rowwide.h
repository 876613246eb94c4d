// rowwide.h -- LayerNorm and softmax over rows too long for the register-held
// row kernels (layernorm.h, softmax.h): one 1024-thread workgroup per row
// streams the row from memory once per reduction it needs, so any row length
// runs (the reference's CPU loops have no limit: crates/vearo-backend-cpu/src/
// lib.rs:499-563, 665-858) and no kernel holds more of a row than a few units
// per lane (the register forms of 24K-32K-float rows spill).
//
// Per element the arithmetic is the register kernels' (the same expressions
// in the same order); the row sums are the same sums with lanes owning
// strided units, reduced by team_sum in a fixed order, so results are
// deterministic. Rows are read 2-4 times (a row of up to ~1 MB is read back
// from L2 / MALL soon after): for the forward softmax, 3 reads + 1 write.
//
// LayerNorm backward takes two kernels plus the column reduce: ln_stats_wide
// computes each row's mean, 1/std, sum(dy*w) and sum(dy*w*xhat) (one workgroup
// per row); ln_tile_wide then walks a column tile over a block of rows,
// writing dx and summing dgamma / dbeta partials per (row block, column),
// which col_reduce adds in row-block order.
#pragma once
#include "common.h"
#include "softmax.h"

#define RW_TEAM 1024

// Softmax forward (softmax_fwd_impl's per-element math): max over the live
// prefix, sum of exp(v - max), then y = e / sum (attn: e * 1/(sum + 1e-9));
// masked columns written as 0 up to zero_end.
template <int VW>
VH_DEV void sm_fwd_wide_impl(const SoftmaxArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  if (row >= a.rows) return;
  const int T = a.T;
  const int U = T / VW;
  const int causal = sm_causal(a);
  const int L = causal ? (int)(row % T) + 1 : T;
  const float* xr = a.x + row * (int64_t)T;
  float m = -INFINITY;
  for (int u = threadIdx.x; u < U && u * VW < L; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j)
      if (u * VW + j < L && v.v[j] > m) m = v.v[j];
  }
  m = team_max<RW_TEAM>(m, red);
  float s = 0.0f;
  for (int u = threadIdx.x; u < U && u * VW < L; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j)
      if (u * VW + j < L) s += expf(v.v[j] - m);
  }
  s = team_sum<RW_TEAM>(s, red);
  const float inv = 1.0f / (s + 1e-9f);
  float* yr = a.y + row * (int64_t)T;
  const int Z = zero_end(a, causal, L);
  for (int u = threadIdx.x; u < U && u * VW < Z; u += RW_TEAM) {
    const bool live = u * VW < L;
    Unit<VW> v = live ? load_unit<VW>(xr + u * VW) : zero_unit<VW>();
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float e = (u * VW + j < L) ? expf(v.v[j] - m) : 0.0f;
      o.v[j] = (u * VW + j < L) ? (a.attn ? e * inv : e / s) : 0.0f;
    }
    store_unit<VW>(yr + u * VW, o);
  }
}

// Softmax backward (softmax_bwd_impl's math): y recomputed from x as the
// forward does (input_is_x) or read; dot = sum(dy * y) over the live prefix
// (attn: a fused multiply-add chain); dx = y * (dy - dot), masked columns 0.
// In place (dx over x or dy) is safe: each element's last reads precede its
// write in the same thread.
template <int VW>
VH_DEV void sm_bwd_wide_impl(const SoftmaxArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  if (row >= a.rows) return;
  const int T = a.T;
  const int U = T / VW;
  const int causal = sm_causal(a);
  const int L = causal ? (int)(row % T) + 1 : T;
  const int64_t off = row * (int64_t)T;
  const float* xr = a.x + off;
  const float* gr = a.dy + off;
  float m = 0.0f, s = 1.0f, inv = 1.0f;
  if (a.input_is_x) {
    m = -INFINITY;
    for (int u = threadIdx.x; u < U && u * VW < L; u += RW_TEAM) {
      const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j)
        if (u * VW + j < L && v.v[j] > m) m = v.v[j];
    }
    m = team_max<RW_TEAM>(m, red);
    s = 0.0f;
    for (int u = threadIdx.x; u < U && u * VW < L; u += RW_TEAM) {
      const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j)
        if (u * VW + j < L) s += expf(v.v[j] - m);
    }
    s = team_sum<RW_TEAM>(s, red);
    inv = 1.0f / (s + 1e-9f);
  }
  auto y_of = [&](float v) -> float {
    if (!a.input_is_x) return v;
    const float e = expf(v - m);
    return a.attn ? e * inv : e / s;
  };
  float dot = 0.0f;
  for (int u = threadIdx.x; u < U && u * VW < L; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW), g = load_unit<VW>(gr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j)
      if (u * VW + j < L) {
        const float y = y_of(v.v[j]);
        dot = a.attn ? __builtin_fmaf(g.v[j], y, dot) : dot + g.v[j] * y;
      }
  }
  dot = team_sum<RW_TEAM>(dot, red);
  float* dxr = a.y + off;
  const int Z = zero_end(a, causal, L);
  for (int u = threadIdx.x; u < U && u * VW < Z; u += RW_TEAM) {
    const bool live = u * VW < L;
    const Unit<VW> v = live ? load_unit<VW>(xr + u * VW) : zero_unit<VW>();
    const Unit<VW> g = live ? load_unit<VW>(gr + u * VW) : zero_unit<VW>();
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) o.v[j] = (u * VW + j < L) ? y_of(v.v[j]) * (g.v[j] - dot) : 0.0f;
    store_unit<VW>(dxr + u * VW, o);
  }
}

// LayerNorm forward (ln_fwd_impl's math): mean, then the sum of squared
// deviations, then y = ((x - mean) * inv_std) * w + b.
template <int VW>
VH_DEV void ln_fwd_wide_impl(const LnFwdArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  if (row >= a.rows) return;
  const int C = a.C;
  const int U = C / VW;
  const float Cf = (float)C;
  const float* xr = a.x + row * (int64_t)C;
  float s = 0.0f;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) s += v.v[j];
  }
  s = team_sum<RW_TEAM>(s, red);
  const float mean = s / Cf;
  float q = 0.0f;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float d = v.v[j] - mean;
      q += d * d;
    }
  }
  q = team_sum<RW_TEAM>(q, red);
  const float inv_std = 1.0f / sqrtf(q / Cf + a.eps);
  float* yr = a.y + row * (int64_t)C;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
    const Unit<VW> w = load_unit<VW>(a.w + u * VW), b = load_unit<VW>(a.b + u * VW);
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float xh = (v.v[j] - mean) * inv_std;
      o.v[j] = xh * w.v[j] + b.v[j];
    }
    store_unit<VW>(yr + u * VW, o);
  }
}

// LayerNorm backward, stage 1: per row mean, inv_std, sum(dy * w) and
// sum((dy * w) * xhat) into stats[row][0..3] (ln_bwd_impl's row math).
template <int VW>
VH_DEV void ln_stats_wide_impl(const LnWideArgs& a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  if (row >= a.rows) return;
  const int C = a.C;
  const int U = C / VW;
  const float Cf = (float)C;
  const float* xr = a.x + row * (int64_t)C;
  const float* gr = a.dy + row * (int64_t)C;
  float s = 0.0f;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) s += v.v[j];
  }
  s = team_sum<RW_TEAM>(s, red);
  const float mean = s / Cf;
  float q = 0.0f;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float d = v.v[j] - mean;
      q += d * d;
    }
  }
  q = team_sum<RW_TEAM>(q, red);
  const float inv_std = 1.0f / sqrtf(q / Cf + a.eps);
  float sgw = 0.0f, sgwx = 0.0f;
  for (int u = threadIdx.x; u < U; u += RW_TEAM) {
    const Unit<VW> v = load_unit<VW>(xr + u * VW), g = load_unit<VW>(gr + u * VW);
    const Unit<VW> w = load_unit<VW>(a.w + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float xh = (v.v[j] - mean) * inv_std;
      const float gow = g.v[j] * w.v[j];
      sgw += gow;
      sgwx += gow * xh;
    }
  }
  sgw = team_sum<RW_TEAM>(sgw, red);
  sgwx = team_sum<RW_TEAM>(sgwx, red);
  if (threadIdx.x == 0) {
    float* st = a.stats + row * 4;
    st[0] = mean;
    st[1] = inv_std;
    st[2] = sgw;
    st[3] = sgwx;
  }
}

// LayerNorm backward, stage 2: workgroup (column tile of 256 units, row block
// blockIdx.y of rpb rows). Each lane owns one unit of columns: dx for every
// row of the block, and its dgamma / dbeta sums over the block's rows in row
// order into part[blockIdx.y][0 | 1][columns].
template <int VW>
VH_DEV void ln_tile_wide_impl(const LnWideArgs& a) {
  const int C = a.C;
  const int U = C / VW;
  const int u = blockIdx.x * 256 + threadIdx.x;
  if (u >= U) return;
  const float Cf = (float)C;
  const float rC = 1.0f / Cf;
  const int64_t r0 = (int64_t)blockIdx.y * a.rpb;
  const int64_t r1 = r0 + a.rpb < a.rows ? r0 + a.rpb : a.rows;
  const Unit<VW> w = load_unit<VW>(a.w + u * VW);
  Unit<VW> gw = zero_unit<VW>(), gb = zero_unit<VW>();
  for (int64_t row = r0; row < r1; ++row) {
    const float* st = a.stats + row * 4;
    const float mean = st[0], inv_std = st[1], sgw = st[2], sgwx = st[3];
    const Unit<VW> v = load_stream<VW>(a.x + row * (int64_t)C + u * VW);
    const Unit<VW> g = load_stream<VW>(a.dy + row * (int64_t)C + u * VW);
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float xh = (v.v[j] - mean) * inv_std;
      gw.v[j] += g.v[j] * xh;
      gb.v[j] += g.v[j];
      const float t1 = Cf * g.v[j] * w.v[j];
      o.v[j] = div_rn((t1 - sgw - xh * sgwx) * inv_std, Cf, rC);
    }
    store_stream<VW>(a.dx + row * (int64_t)C + u * VW, o);
  }
  float* p = a.part + (size_t)blockIdx.y * 2 * C;
  store_unit<VW>(p + u * VW, gw);
  store_unit<VW>(p + C + u * VW, gb);
}
