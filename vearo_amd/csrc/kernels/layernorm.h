// layernorm.h -- LayerNorm forward / backward for gfx950.
//
// Semantics follow vearo-backend-cpu layernorm (crates/vearo-backend-cpu/src/lib.rs:665-740)
// and layernorm_backward (lib.rs:742-858): mean = sum/C, var = sum((x-mean)^2)/C,
// inv_std = 1/sqrt(var+eps), y = ((x-mean)*inv_std)*w + b;
// dx = ((C*go)*w - sum(go*w) - x_hat*sum((go*w)*x_hat)) * inv_std / C,
// dgamma = sum_rows go*x_hat, dbeta = sum_rows go.
//
// Layout: x, y, dy, dx are [rows, C] row-major in HBM; w, b are [C].
// Forward: a TEAM of lanes owns one row, the row lives in VGPRs (NV units of VW
// floats per lane), so x is read exactly once and y written once (8 B/elem).
// Backward: x and dy read once, dx written once (12 B/elem). dgamma/dbeta are
// deterministic and atomic-free: each lane accumulates its fixed columns over the
// rows its team visits, the row-groups of a workgroup are folded in a fixed LDS
// tree, one partial row per workgroup goes to scratch, and col_reduce sums the
// partials in a fixed order.
#pragma once
#include "common.h"

template <int TEAM, int NV, int VW>
VH_DEV void ln_fwd_impl(const LnFwdArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int RPB = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TEAM;
  const bool active = row < a.rows;
  const int C = a.C;
  const int U = C / VW;
  const float* xr = a.x + (active ? row : 0) * (int64_t)C;

  Unit<VW> v[NV];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    v[k] = (active && u < U) ? load_unit<VW>(xr + u * VW) : zero_unit<VW>();
#pragma unroll
    for (int j = 0; j < VW; ++j) s += v[k].v[j];
  }
  s = team_sum<TEAM>(s, red);
  const float Cf = (float)C;
  const float mean = s / Cf;
  float q = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    if (u < U) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float d = v[k].v[j] - mean;
        q += d * d;
      }
    }
  }
  q = team_sum<TEAM>(q, red);
  const float var = q / Cf;
  const float inv_std = 1.0f / sqrtf(var + a.eps);
  if (!active) return;
  float* yr = a.y + row * (int64_t)C;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = lane + k * TEAM;
    if (u < U) {
      const Unit<VW> w = load_unit<VW>(a.w + u * VW);
      const Unit<VW> b = load_unit<VW>(a.b + u * VW);
      Unit<VW> o;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float xh = (v[k].v[j] - mean) * inv_std;
        o.v[j] = xh * w.v[j] + b.v[j];
      }
      store_unit<VW>(yr + u * VW, o);
    }
  }
}

// Backward stage 1. Workgroup = BS threads = G row-groups of TEAM lanes. The
// workgroup owns rows [blockIdx.x*rows_per_block, +rows_per_block); group g
// visits rows g, g+G, ... of that range. Dynamic LDS: (G/2)*2*C floats.
template <int TEAM, int NV, int VW>
VH_DEV void ln_bwd_impl(const LnBwdArgs& a, float* lds) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int G = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int g = threadIdx.x / TEAM;
  const int C = a.C;
  const int U = C / VW;
  const float Cf = (float)C;
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_block;
  int64_t r1 = r0 + a.rows_per_block;
  if (r1 > a.rows) r1 = a.rows;

  Unit<VW> gw[NV], gb[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    gw[k] = zero_unit<VW>();
    gb[k] = zero_unit<VW>();
  }

  for (int64_t row = r0 + g; row < r1; row += G) {
    const float* xr = a.x + row * (int64_t)C;
    const float* dyr = a.dy + row * (int64_t)C;
    Unit<VW> xv[NV], gv[NV];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U) {
        xv[k] = load_unit<VW>(xr + u * VW);
        gv[k] = load_unit<VW>(dyr + u * VW);
      } else {
        xv[k] = zero_unit<VW>();
        gv[k] = zero_unit<VW>();
      }
#pragma unroll
      for (int j = 0; j < VW; ++j) s += xv[k].v[j];
    }
    s = team_sum<TEAM>(s, red);
    const float mean = s / Cf;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float d = xv[k].v[j] - mean;
          q += d * d;
        }
      }
    }
    q = team_sum<TEAM>(q, red);
    const float inv_std = 1.0f / sqrtf(q / Cf + a.eps);

    float sgw = 0.0f, sgwx = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U) {
        const Unit<VW> w = load_unit<VW>(a.w + u * VW);
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float xh = (xv[k].v[j] - mean) * inv_std;
          const float gow = gv[k].v[j] * w.v[j];
          sgw += gow;
          sgwx += gow * xh;
          gw[k].v[j] += gv[k].v[j] * xh;
          gb[k].v[j] += gv[k].v[j];
        }
      }
    }
    sgw = team_sum<TEAM>(sgw, red);
    sgwx = team_sum<TEAM>(sgwx, red);

    float* dxr = a.dx + row * (int64_t)C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U) {
        const Unit<VW> w = load_unit<VW>(a.w + u * VW);
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float xh = (xv[k].v[j] - mean) * inv_std;
          const float t1 = Cf * gv[k].v[j] * w.v[j];
          o.v[j] = (t1 - sgw - xh * sgwx) * inv_std / Cf;
        }
        store_unit<VW>(dxr + u * VW, o);
      }
    }
  }

  // Fold the G row-groups in a fixed tree: at each step the upper half parks its
  // partials in LDS and the lower half adds them (group g += group g+half).
  if constexpr (G > 1) {
#pragma unroll
    for (int half = G / 2; half >= 1; half /= 2) {
      if (g >= half && g < 2 * half) {
        float* dst = lds + (size_t)(g - half) * 2 * C;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int u = lane + k * TEAM;
          if (u < U) {
#pragma unroll
            for (int j = 0; j < VW; ++j) {
              dst[u * VW + j] = gw[k].v[j];
              dst[C + u * VW + j] = gb[k].v[j];
            }
          }
        }
      }
      __syncthreads();
      if (g < half) {
        const float* src = lds + (size_t)g * 2 * C;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int u = lane + k * TEAM;
          if (u < U) {
#pragma unroll
            for (int j = 0; j < VW; ++j) {
              gw[k].v[j] += src[u * VW + j];
              gb[k].v[j] += src[C + u * VW + j];
            }
          }
        }
      }
      __syncthreads();
    }
  }
  if (g == 0) {
    float* p = a.part + (size_t)blockIdx.x * 2 * C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (u < U) {
        store_unit<VW>(p + u * VW, gw[k]);
        store_unit<VW>(p + C + u * VW, gb[k]);
      }
    }
  }
}

// Stage 2: out_c[col] = sum over p of part[p][c][col], p ascending within each of
// 16 waves (wave w takes p = w, w+16, ...), then the 16 wave sums in order.
// Grid: (ceil(C/64), ncomp), 1024 threads.
VH_DEV void col_reduce_impl(const ColReduceArgs& a) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int comp = blockIdx.y;
  const int col = blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (col < a.C) {
    const float* base = a.part + (size_t)comp * a.C + col;
    const size_t pstride = (size_t)a.ncomp * a.C;
    int p = w;
    for (; p + 48 < a.P; p += 64) {
      const float v0 = base[(size_t)p * pstride];
      const float v1 = base[(size_t)(p + 16) * pstride];
      const float v2 = base[(size_t)(p + 32) * pstride];
      const float v3 = base[(size_t)(p + 48) * pstride];
      s += v0;
      s += v1;
      s += v2;
      s += v3;
    }
    for (; p < a.P; p += 16) s += base[(size_t)p * pstride];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < a.C) {
    float t = red[0][lane];
#pragma unroll
    for (int i = 1; i < 16; ++i) t += red[i][lane];
    (comp == 0 ? a.out0 : a.out1)[col] = t;
  }
}
