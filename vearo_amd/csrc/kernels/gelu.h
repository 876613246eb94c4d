// gelu.h -- GELU (tanh approximation) forward / backward, optionally fused with
// the broadcast bias add of a Linear layer, for gfx950.
//
// Formulas follow vearo-backend-cpu gelu (crates/vearo-backend-cpu/src/lib.rs:456-497)
// and the autograd gelu_grad_mask (crates/vearo-autograd/src/lib.rs:377-403), with the
// same f32 constants and the same rounding order (built with -ffp-contract=off).
// The bias add h = x + b[c] is the Linear bias add (cpu lib.rs:183-196 broadcast).
//
// Layout: x, dy, y, dx [rows, C] row-major; bias, dbias [C]. The forward bias
// kernel takes one row per 256-thread workgroup with the row's bias in VGPRs.
// The backward takes a tile of 64 column units by one row block per
// workgroup, one unit per lane, so every wave streams 64 consecutive units of
// a row (the layout a plain copy streams best in) and the dbias partial of the
// tile's columns is summed in the workgroup. Every tensor byte moves once (fwd
// 8 B/elem, bwd 12 B/elem) and dbias needs no atomics. Rows wider than the
// forward's registers hold take a column-tile forward of the backward's shape.
#pragma once
#include "common.h"

#define GELU_SQRT_2_OVER_PI 0.79788456f
#define GELU_COEFF 0.044715f
#define GELU_DERIV_COEFF 0.134145f

VH_DEV float gelu_f(float v) {
  const float v3 = v * v * v;
  const float inner = GELU_SQRT_2_OVER_PI * (v + GELU_COEFF * v3);
  return 0.5f * v * (1.0f + tanhf(inner));
}

VH_DEV float gelu_mask_f(float v) {
  const float v3 = v * v * v;
  const float inner = GELU_SQRT_2_OVER_PI * (v + GELU_COEFF * v3);
  const float t = tanhf(inner);
  const float sech_sq = 1.0f - t * t;
  const float inner_deriv = GELU_SQRT_2_OVER_PI * (1.0f + GELU_DERIV_COEFF * v * v);
  return 0.5f * (1.0f + t) + 0.5f * v * sech_sq * inner_deriv;
}

// Flat elementwise: mode 0 -> y = gelu(x); mode 1 -> y = dy * gelu_mask(x).
template <int MODE, int VW>
VH_DEV void gelu_flat_impl(const EltArgs& a) {
  const int64_t nu = a.n / VW;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < nu; u += stride) {
    const Unit<VW> x = load_stream<VW>(a.x + u * VW);
    Unit<VW> o;
    if constexpr (MODE == 0) {
#pragma unroll
      for (int j = 0; j < VW; ++j) o.v[j] = gelu_f(x.v[j]);
    } else {
      const Unit<VW> g = load_stream<VW>(a.dy + u * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j) o.v[j] = g.v[j] * gelu_mask_f(x.v[j]);
    }
    store_stream<VW>(a.y + u * VW, o);
  }
}

// y[r, c] = gelu(x[r, c] + bias[c]); workgroup = 256 threads, NV units per thread.
template <int NV, int VW>
VH_DEV void gelu_bias_fwd_impl(const GeluBiasBwdArgs& a) {
  const int C = a.C;
  const int U = C / VW;
  Unit<VW> b[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = threadIdx.x + k * 256;
    b[k] = u < U ? load_unit<VW>(a.bias + u * VW) : zero_unit<VW>();
  }
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_block;
  int64_t r1 = r0 + a.rows_per_block;
  if (r1 > a.rows) r1 = a.rows;
  for (int64_t r = r0; r < r1; ++r) {
    const float* xr = a.x + r * C;
    float* yr = a.dx + r * C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = threadIdx.x + k * 256;
      if (u < U) {
        const Unit<VW> x = load_stream<VW>(xr + u * VW);
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) o.v[j] = gelu_f(x.v[j] + b[k].v[j]);
        store_stream<VW>(yr + u * VW, o);
      }
    }
  }
}

// The same forward for rows wider than one workgroup holds in registers
// (past 256 x 16 units): a tile of 64 column units by one row block per
// 256-thread workgroup, one unit per lane, wave w taking rows r0 + w, r0 + w +
// 4, ...; the same gelu(x + b) per element, so the same bits.
template <int VW>
VH_DEV void gelu_bias_fwd_tile_impl(const GeluBiasBwdArgs& a) {
  const int64_t C = a.C;
  const int64_t U = C / VW;
  const int64_t u = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  if (u >= U) return;
  const Unit<VW> b = load_unit<VW>(a.bias + u * VW);
  const int64_t r0 = (int64_t)blockIdx.y * a.rows_per_block;
  int64_t r1 = r0 + a.rows_per_block;
  if (r1 > a.rows) r1 = a.rows;
  for (int64_t r = r0 + (threadIdx.x >> 6); r < r1; r += 4) {
    const Unit<VW> x = load_stream<VW>(a.x + r * C + u * VW);
    Unit<VW> o;
#pragma unroll
    for (int j = 0; j < VW; ++j) o.v[j] = gelu_f(x.v[j] + b.v[j]);
    store_stream<VW>(a.dx + r * C + u * VW, o);
  }
}

// dx[r, c] = dy[r, c] * gelu_mask(x[r, c] + bias[c]); part[blk][c] = sum of
// dx[r, c] over the rows of row block blk = [blk * rpb, blk * rpb + rpb).
// Workgroup (column tile blockIdx.x of 64 VW-float units, row block
// blockIdx.y): each lane holds one unit, so a wave reads and writes 64
// consecutive units of a row; wave w takes rows r0 + w, r0 + w + 4, ... (RPT
// rows' loads issued together), sums them in ascending order, and the four
// waves' sums are added in wave order through LDS. The partials depend on
// (rows, C) only.
template <int VW, int RPT>
VH_DEV void gelu_bias_bwd_tile_impl(const GeluBiasBwdArgs& a) {
  __shared__ Unit<VW> lds[3][64];
  const int C = a.C;
  const int U = C / VW;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int u = blockIdx.x * 64 + lane;
  const bool cu = u < U;
  const Unit<VW> b = cu ? load_unit<VW>(a.bias + u * VW) : zero_unit<VW>();
  Unit<VW> acc = zero_unit<VW>();
  const int64_t r0 = (int64_t)blockIdx.y * a.rows_per_block;
  int64_t r1 = r0 + a.rows_per_block;
  if (r1 > a.rows) r1 = a.rows;
  for (int64_t base = r0 + w; base < r1; base += 4 * RPT) {
    Unit<VW> x[RPT], g[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int64_t r = base + 4 * i;
      x[i] = g[i] = zero_unit<VW>();
      if (cu && r < r1) {
        x[i] = load_stream<VW>(a.x + r * C + u * VW);
        g[i] = load_stream<VW>(a.dy + r * C + u * VW);
      }
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int64_t r = base + 4 * i;
      if (cu && r < r1) {
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          o.v[j] = g[i].v[j] * gelu_mask_f(x[i].v[j] + b.v[j]);
          acc.v[j] += o.v[j];
        }
        store_stream<VW>(a.dx + r * C + u * VW, o);
      }
    }
  }
  if (w > 0) lds[w - 1][lane] = acc;
  __syncthreads();
  if (w == 0 && cu) {
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int j = 0; j < VW; ++j) acc.v[j] += lds[q][lane].v[j];
    store_unit<VW>(a.part + (int64_t)blockIdx.y * C + u * VW, acc);
  }
}
