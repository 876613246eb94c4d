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
// Backward: x and dy read once, dx written once (12 B/elem), rows dealt to the
// grid's teams grid-stride. dgamma/dbeta are deterministic and atomic-free:
// each lane accumulates its fixed columns over the rows its team visits, the G
// teams of a workgroup fold in a fixed order through LDS, one partial row per
// workgroup goes to scratch, and col_reduce sums the partials in a fixed order.
// FULL forms (C exactly TEAM * NV * VW, e.g. 768 = 64 lanes x 3 units x 4
// floats) drop the per-unit bounds tests: 12 % of the backward's time at GPT-2
// shape (measured). An in-kernel finish of the column sums (last workgroup to
// arrive adds the partials) was measured at 150-190 us against 4.5 us for the
// separate col_reduce launch: the device-scope fence it needs writes back an
// XCD's L2 and serialises across the workgroups of the XCD.
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

// Backward stage 1. Workgroup = BS threads = G row-groups (teams) of TEAM
// lanes; the grid's NT = gridDim.x * G teams take rows grid-stride (team t:
// rows t, t + NT, ...), so at any moment the whole grid streams one contiguous
// block of rows (measured on MI355X at [16384, 768]: 30.5 against 34.4 us for
// teams walking private contiguous row ranges, the same arithmetic). w stays in
// registers where the budget allows (HOIST), so the only memory waits in the
// row loop are on x and dy. The row reductions and the dx expression are the
// reference's; the division by C is div_rn (bit-identical, 3 instructions).
// dgamma/dbeta: each lane accumulates its columns over its team's rows; the G
// teams of a workgroup fold through LDS in a fixed order -- FULL forms (C a
// compile-time TEAM*NV*VW, G = 8) in one level (every team parks its partial
// row, one barrier, each thread sums one 4-column unit over the 16 slots in
// team order), the others in a fixed pairwise tree in dynamic LDS of
// (G/2)*2*C floats -- and one partial row per workgroup goes to scratch for
// col_reduce. Row assignment and grouping depend on (rows, C) only, so the
// result is identical run to run.
template <int TEAM, int NV, int VW, int BS, bool FULL = false>
VH_DEV void ln_bwd_impl(const LnBwdArgs& a, float* lds) {
  static_assert(BS >= TEAM && BS % TEAM == 0, "block must hold whole teams");
  constexpr int G = BS / TEAM;
  constexpr bool HOIST = NV * VW <= 12;  // w in VGPRs: 12 more at C = 768 (109 -> 111 in all)
  __shared__ float red[16];
  const int lane = threadIdx.x % TEAM;
  const int g = threadIdx.x / TEAM;
  const int C = FULL ? TEAM * NV * VW : a.C;
  const int U = FULL ? TEAM * NV : C / VW;  // FULL: C == TEAM * NV * VW, every unit live
  const float Cf = (float)C;
  const float rC = 1.0f / Cf;
  const int64_t NT = (int64_t)gridDim.x * G;

  Unit<VW> gw[NV], gb[NV], wv[HOIST ? NV : 1];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    gw[k] = zero_unit<VW>();
    gb[k] = zero_unit<VW>();
    if constexpr (HOIST) {
      const int u = lane + k * TEAM;
      wv[k] = (FULL || u < U) ? load_unit<VW>(a.w + u * VW) : zero_unit<VW>();
    }
  }
  auto wunit = [&](int k, int u) -> Unit<VW> {
    if constexpr (HOIST) return wv[k];
    else return load_unit<VW>(a.w + u * VW);
  };

  for (int64_t row = (int64_t)blockIdx.x * G + g; row < a.rows; row += NT) {
    const float* xr = a.x + row * (int64_t)C;
    const float* dyr = a.dy + row * (int64_t)C;
    Unit<VW> xv[NV], gv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      if (FULL || u < U) {
        xv[k] = load_stream<VW>(xr + u * VW);
        gv[k] = load_stream<VW>(dyr + u * VW);
      } else {
        xv[k] = zero_unit<VW>();
        gv[k] = zero_unit<VW>();
      }
    }

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
        const Unit<VW> w = wunit(k, u);
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
        const Unit<VW> w = wunit(k, u);
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float xh = (xv[k].v[j] - mean) * inv_std;
          const float t1 = Cf * gv[k].v[j] * w.v[j];
          o.v[j] = div_rn((t1 - sgw - xh * sgwx) * inv_std, Cf, rC);
        }
        store_stream<VW>(dxr + u * VW, o);
      }
    }
  }

  float* p = a.part + (size_t)blockIdx.x * 2 * C;
  if constexpr (FULL) {
    // One-level fold: slot g holds team g's [dgamma | dbeta] partial row.
    static_assert(VW == 4, "full forms use 128-bit units");
    __shared__ float fold[G * 2 * TEAM * NV * VW];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = lane + k * TEAM;
      store_unit<VW>(fold + g * 2 * C + u * VW, gw[k]);
      store_unit<VW>(fold + g * 2 * C + C + u * VW, gb[k]);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 2 * C / 4; t += BS) {
      Unit<4> acc = load_unit<4>(fold + t * 4);
#pragma unroll
      for (int i = 1; i < G; ++i) {
        const Unit<4> v = load_unit<4>(fold + i * 2 * C + t * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc.v[j] += v.v[j];
      }
      store_unit<4>(p + t * 4, acc);
    }
  } else {
    // Fixed pairwise tree: at each step the upper half parks its partials in
    // LDS and the lower half adds them (group g += group g+half).
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
}

// Stage 2: out_c[col] = sum over p of part[p][c][col]. A workgroup owns CW =
// VH_COLR_COLS consecutive columns; thread group w of the 16 owns the contiguous
// partial range [w*per, (w+1)*per) and sums it in order with up to 16 loads in
// flight; the 16 range sums are then added in range order, so the result is the
// partials summed in index order with a fixed grouping (deterministic). Narrow
// workgroups spread the 1.5 MiB of LayerNorm partials over 96 CUs instead of
// 24 (LayerNorm backward + reduce 32.2 -> 31.6 us, same bits).
// Grid: (ceil(C/CW), ncomp), CW * 16 threads.
VH_DEV void col_reduce_impl(const ColReduceArgs& a) {
  constexpr int CW = VH_COLR_COLS;
  __shared__ float red[16][CW];
  const int lane = threadIdx.x % CW;
  const int w = threadIdx.x / CW;
  const int comp = blockIdx.y;
  const int col = blockIdx.x * CW + lane;
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
