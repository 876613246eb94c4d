// gelu.h -- GELU (tanh approximation) forward / backward, optionally fused with
// the broadcast bias add of a Linear layer, for gfx950.
//
// Formulas follow vearo-backend-cpu gelu (crates/vearo-backend-cpu/src/lib.rs:456-497)
// and the autograd gelu_grad_mask (crates/vearo-autograd/src/lib.rs:377-403), with the
// same f32 constants and the same rounding order (built with -ffp-contract=off).
// The bias add h = x + b[c] is the Linear bias add (cpu lib.rs:183-196 broadcast).
//
// Layout: x, dy, y, dx [rows, C] row-major; bias, dbias [C]. The bias kernels are
// column-stationary: a 256-thread workgroup keeps its columns' bias (and dbias
// partials) in VGPRs and walks a contiguous range of rows, so every tensor byte
// moves once (fwd 8 B/elem, bwd 12 B/elem) and dbias needs no atomics.
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

// dx[r, c] = dy[r, c] * gelu_mask(x[r, c] + bias[c]); part[blk][c] = sum over the
// workgroup's rows (ascending) of dx[r, c].
template <int NV, int VW>
VH_DEV void gelu_bias_bwd_impl(const GeluBiasBwdArgs& a) {
  const int C = a.C;
  const int U = C / VW;
  Unit<VW> b[NV], acc[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = threadIdx.x + k * 256;
    b[k] = u < U ? load_unit<VW>(a.bias + u * VW) : zero_unit<VW>();
    acc[k] = zero_unit<VW>();
  }
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_block;
  int64_t r1 = r0 + a.rows_per_block;
  if (r1 > a.rows) r1 = a.rows;
  for (int64_t r = r0; r < r1; ++r) {
    const float* xr = a.x + r * C;
    const float* gr = a.dy + r * C;
    float* dr = a.dx + r * C;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int u = threadIdx.x + k * 256;
      if (u < U) {
        const Unit<VW> x = load_stream<VW>(xr + u * VW);
        const Unit<VW> g = load_stream<VW>(gr + u * VW);
        Unit<VW> o;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          o.v[j] = g.v[j] * gelu_mask_f(x.v[j] + b[k].v[j]);
          acc[k].v[j] += o.v[j];
        }
        store_stream<VW>(dr + u * VW, o);
      }
    }
  }
  float* p = a.part + (size_t)blockIdx.x * C;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int u = threadIdx.x + k * 256;
    if (u < U) store_unit<VW>(p + u * VW, acc[k]);
  }
}
