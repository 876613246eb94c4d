// optim.h -- AdamW parameter update on the device.
//
// Semantics: Tensor::adamw_step (crates/vearo-core/src/tensor.rs:931-986) for one
// parameter tensor, in the reference's operation order (built without FMA
// contraction, so each product and sum rounds separately):
//   m = beta1*m + (1-beta1)*g;  v = beta2*v + ((1-beta2)*g)*g;
//   m_hat = m/bc1;  v_hat = v/bc2;  p = p - (lr*wd)*p;  p = p - (lr*m_hat)/(sqrt(v_hat) + eps)
// The reference keeps m and v on the host and copies the parameter both ways
// (tensor.rs:989-1019); here p, g, m and v stay in HBM: one read of each and one
// write of p, m, v (28 bytes per parameter).
#pragma once
#include "common.h"

VH_DEV void adam_one(const AdamArgs& a, float& p, float g, float& m, float& v) {
  m = a.beta1 * m + a.omb1 * g;
  v = a.beta2 * v + a.omb2 * g * g;
  const float mh = m / a.bc1;
  const float vh = v / a.bc2;
  p = p - a.lrwd * p;
  p = p - a.lr * mh / (__builtin_sqrtf(vh) + a.eps);
}

// One launch over up to VH_ADAMW_MULTI_MAX tensors: block b belongs to the
// last tensor whose first block is <= b and updates one unit per thread of it
// with adam_one, so each element gets exactly the bits vh_adamw_v4 / v1 give it.
VH_DEV void adamw_multi_impl(const AdamMultiArgs& a) {
  int s = 0;
  for (int i = 1; i < a.count; ++i)
    if ((int)blockIdx.x >= a.seg[i].blk0) s = i;
  const AdamSeg& sg = a.seg[s];
  const int64_t u = (int64_t)(blockIdx.x - sg.blk0) * blockDim.x + threadIdx.x;
  if (sg.vec) {
    if (u >= sg.n / 4) return;
    Unit<4> p = load_stream<4>(sg.p + u * 4), g = load_stream<4>(sg.g + u * 4);
    Unit<4> m = load_stream<4>(sg.m + u * 4), v = load_stream<4>(sg.v + u * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) adam_one(a.h, p.v[j], g.v[j], m.v[j], v.v[j]);
    store_stream<4>(sg.p + u * 4, p);
    store_stream<4>(sg.m + u * 4, m);
    store_stream<4>(sg.v + u * 4, v);
  } else {
    if (u >= sg.n) return;
    float p = sg.p[u], m = sg.m[u], v = sg.v[u];
    adam_one(a.h, p, sg.g[u], m, v);
    sg.p[u] = p;
    sg.m[u] = m;
    sg.v[u] = v;
  }
}

template <int VW>
VH_DEV void adamw_impl(const AdamArgs& a) {
  const int64_t U = a.n / VW;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < U; u += stride) {
    Unit<VW> p = load_stream<VW>(a.p + u * VW), g = load_stream<VW>(a.g + u * VW);
    Unit<VW> m = load_stream<VW>(a.m + u * VW), v = load_stream<VW>(a.v + u * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) adam_one(a, p.v[j], g.v[j], m.v[j], v.v[j]);
    store_stream<VW>(a.p + u * VW, p);
    store_stream<VW>(a.m + u * VW, m);
    store_stream<VW>(a.v + u * VW, v);
  }
}
