// layernorm.h -- LayerNorm forward / backward for gfx950.
//
// Semantics follow vearo-backend-cpu layernorm (crates/vearo-backend-cpu/src/lib.rs:665-740)
// and layernorm_backward (lib.rs:742-858): mean = sum/C, var = sum((x-mean)^2)/C,
// inv_std = 1/sqrt(var+eps), y = ((x-mean)*inv_std)*w + b;
// dx = ((C*go)*w - sum(go*w) - x_hat*sum((go*w)*x_hat)) * inv_std / C,
// dgamma = sum_rows go*x_hat, dbeta = sum_rows go.
//
// Layout: x, y, dy, dx are [rows, C] row-major in HBM; w, b are [C].
// Forward: a TEAM of lanes owns a row held in VGPRs (NV units of VW floats per
// lane); each team takes RPW rows and issues all their loads before any math,
// so x is read once and y written once (8 B/elem) with enough bytes in flight.
// Backward: x and dy read once, dx written once (12 B/elem); the next row of a
// team is prefetched while the current one is reduced. dgamma/dbeta are
// deterministic and atomic-free: each lane accumulates its fixed columns over
// the rows its team visits, the G row-groups of a workgroup fold in a fixed LDS
// tree, one partial row per workgroup goes to scratch, and col_reduce sums the
// partials in a fixed order. FULL forms (C exactly TEAM * NV * VW, e.g. 768 =
// 64 lanes x 3 units x 4 floats) drop the per-unit bounds tests: 12 % of the
// backward's time at GPT-2 shape (measured).
#pragma once
#include "common.h"

template <int TEAM, int NV, int VW, int RPW, bool FULL = false>
VH_DEV void ln_fwd_impl(const LnFwdArgs& a) {
  constexpr int BS = TEAM > 256 ? TEAM : 256;
  constexpr int TPB = BS / TEAM;  // teams per block
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int64_t row0 = ((int64_t)blockIdx.x * TPB + threadIdx.x / TEAM) * RPW;
  const int C = a.C;
  const int U = FULL ? TEAM * NV : C / VW;  // FULL: C == TEAM * NV * VW, every unit live
  const float Cf = (float)C;

  Unit<VW> v[RPW][NV];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool active = row < a.rows;
    const float* xr = a.x + (active ? row : 0) * (int64_t)C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      v[r][k] = (active && (FULL || u < U)) ? load_stream<VW>(xr + u * VW) : zero_unit<VW>();
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
      for (int j = 0; j < VW; ++j) s += v[r][k].v[j];
    }
    s = team_sum<TEAM>(s, red);
    const float mean = s / Cf;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (FULL || u < U) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float d = v[r][k].v[j] - mean;
          q += d * d;
        }
      }
    }
    q = team_sum<TEAM>(q, red);
    const float var = q / Cf;
    const float inv_std = 1.0f / sqrtf(var + a.eps);
    if (row < a.rows) {
      float* yr = a.y + row * (int64_t)C;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int u = lane + k * TEAM;
        if (FULL || u < U) {
          const Unit<VW> w = load_unit<VW>(a.w + u * VW);
          const Unit<VW> b = load_unit<VW>(a.b + u * VW);
          Unit<VW> o;
#pragma unroll
          for (int j = 0; j < VW; ++j) {
            const float xh = (v[r][k].v[j] - mean) * inv_std;
            o.v[j] = xh * w.v[j] + b.v[j];
          }
          store_stream<VW>(yr + u * VW, o);
        }
      }
    }
  }
}

// Backward stage 1. Workgroup = BS threads = G row-groups of TEAM lanes. The
// workgroup owns rows [blockIdx.x*rows_per_block, +rows_per_block); group g
// visits rows g, g+G, ... of that range. Dynamic LDS: (G/2)*2*C floats.
template <int TEAM, int NV, int VW, int BS, bool FULL = false>
VH_DEV void ln_bwd_impl(const LnBwdArgs& a, float* lds) {
  static_assert(BS >= TEAM && BS % TEAM == 0, "block must hold whole teams");
  constexpr int G = BS / TEAM;
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int g = threadIdx.x / TEAM;
  const int C = a.C;
  const int U = FULL ? TEAM * NV : C / VW;  // FULL: C == TEAM * NV * VW, every unit live
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

  // Row `row` of this group: x and dy into registers (zeros past the range).
  auto load_row = [&](int64_t row, Unit<VW>* xv, Unit<VW>* gv) {
    const bool ok = row < r1;
    const float* xr = a.x + (ok ? row : 0) * (int64_t)C;
    const float* dyr = a.dy + (ok ? row : 0) * (int64_t)C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (ok && (FULL || u < U)) {
        xv[k] = load_stream<VW>(xr + u * VW);
        gv[k] = load_stream<VW>(dyr + u * VW);
      } else {
        xv[k] = zero_unit<VW>();
        gv[k] = zero_unit<VW>();
      }
    }
  };

  Unit<VW> xv[NV], gv[NV];
  int64_t row = r0 + g;
  load_row(row, xv, gv);
  for (; row < r1; row += G) {
    Unit<VW> xn[NV], gn[NV];
    load_row(row + G, xn, gn);  // prefetch: in flight while this row is reduced

    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
      for (int j = 0; j < VW; ++j) s += xv[k].v[j];
    }
    s = team_sum<TEAM>(s, red);
    const float mean = s / Cf;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (FULL || u < U) {
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
      if (FULL || u < U) {
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
      if (FULL || u < U) {
        const Unit<VW> w = load_unit<VW>(a.w + u * VW);
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float xh = (xv[k].v[j] - mean) * inv_std;
          const float t1 = Cf * gv[k].v[j] * w.v[j];
          o.v[j] = (t1 - sgw - xh * sgwx) * inv_std / Cf;
        }
        store_stream<VW>(dxr + u * VW, o);
      }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      xv[k] = xn[k];
      gv[k] = gn[k];
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
          if (FULL || u < U) {
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
          if (FULL || u < U) {
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
      if (FULL || u < U) {
        store_unit<VW>(p + u * VW, gw[k]);
        store_unit<VW>(p + C + u * VW, gb[k]);
      }
    }
  }
}

// Stage 2: out_c[col] = sum over p of part[p][c][col]. Wave w of the 16 owns the
// contiguous partial range [w*per, (w+1)*per) and sums it in order with up to 16
// loads in flight; the 16 wave sums are then added in wave order, so the result
// is the partials summed in index order with a fixed grouping (deterministic).
// Grid: (ceil(C/64), ncomp), 1024 threads.
VH_DEV void col_reduce_impl(const ColReduceArgs& a) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int comp = blockIdx.y;
  const int col = blockIdx.x * 64 + lane;
  const int per = (a.P + 15) / 16;
  const int p0 = w * per;
  const int p1 = min(p0 + per, a.P);
  float s = 0.0f;
  if (col < a.C) {
    const float* base = a.part + (size_t)comp * a.C + col;
    const size_t pstride = (size_t)a.ncomp * a.C;
    for (int p = p0; p < p1; p += 16) {
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = (p + k < p1) ? base[(size_t)(p + k) * pstride] : 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (p + k < p1) s += v[k];
    }
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
