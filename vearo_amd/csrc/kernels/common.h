// common.h -- device helpers shared by the gfx950 kernels: wave64 / multi-wave
// "team" reductions and fixed-width register rows.
//
// A row of a bandwidth-bound op is owned by a TEAM of lanes:
//   TEAM 16/32/64  -> a sub-wave or one wave64; reductions stay in VGPRs via DPP
//                     row ops and two ds_swizzle/bpermute steps.
//   TEAM 256/1024  -> TEAM/64 waves of one workgroup; each wave reduces in
//                     registers, then the per-wave values meet in LDS in a fixed
//                     order (bit-identical result in every lane, deterministic).
// Each lane holds NV "units" of the row in registers, unit k = lane + k*TEAM,
// where a unit is VW consecutive floats (VW = 4 -> one 128-bit load).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../vh_kargs.h"

#define VH_DEV __device__ __forceinline__

// DPP controls (gfx9 encoding).
#define DPP_QUAD_XOR1 0xB1   // quad_perm [1,0,3,2]
#define DPP_QUAD_XOR2 0x4E   // quad_perm [2,3,0,1]
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_MIRROR 0x140

template <int CTRL>
VH_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Row value of 16-lane row `ROW` of the wave (wave-uniform, via v_readlane).
template <int ROW>
VH_DEV float row_value(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), ROW * 16));
}

// Sum / max over aligned groups of W lanes (W = 2..64); every lane of the group
// ends with the same bits (each step combines the two halves commutatively).
// A whole wave (W = 64) combines its four 16-lane row values with v_readlane
// as (r0 + r1) + (r2 + r3) -- the same bits as an xor-16 then xor-32 exchange,
// without the two LDS-unit permutes on the row's critical path.
template <int W>
VH_DEV float group_sum(float v) {
  if constexpr (W >= 2) v += dpp_mov<DPP_QUAD_XOR1>(v);
  if constexpr (W >= 4) v += dpp_mov<DPP_QUAD_XOR2>(v);
  if constexpr (W >= 8) v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
  if constexpr (W >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
  if constexpr (W == 32) v += __shfl_xor(v, 16, 64);
  if constexpr (W == 64) v = (row_value<0>(v) + row_value<1>(v)) + (row_value<2>(v) + row_value<3>(v));
  return v;
}

template <int W>
VH_DEV float group_max(float v) {
  if constexpr (W >= 2) v = fmaxf(v, dpp_mov<DPP_QUAD_XOR1>(v));
  if constexpr (W >= 4) v = fmaxf(v, dpp_mov<DPP_QUAD_XOR2>(v));
  if constexpr (W >= 8) v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
  if constexpr (W >= 16) v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
  if constexpr (W == 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if constexpr (W == 64)
    v = fmaxf(fmaxf(row_value<0>(v), row_value<1>(v)), fmaxf(row_value<2>(v), row_value<3>(v)));
  return v;
}

// Team reductions. For TEAM > 64 a team is TEAM / 64 consecutive waves of the
// workgroup (one or more teams per workgroup); wave w writes its partial to
// lds[w] and each team reads its own NW slots, so `lds` must hold
// blockDim.x / 64 floats and every thread of the block must call (no early
// exit). The partials are combined in wave order.
template <int TEAM>
VH_DEV float team_sum(float v, float* lds) {
  if constexpr (TEAM <= 64) {
    return group_sum<TEAM>(v);
  } else {
    constexpr int NW = TEAM / 64;
    v = group_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    const float* t = lds + (wave / NW) * NW;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    float s = t[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s += t[i];
    __syncthreads();
    return s;
  }
}

template <int TEAM>
VH_DEV float team_max(float v, float* lds) {
  if constexpr (TEAM <= 64) {
    return group_max<TEAM>(v);
  } else {
    constexpr int NW = TEAM / 64;
    v = group_max<64>(v);
    const int wave = threadIdx.x >> 6;
    const float* t = lds + (wave / NW) * NW;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    float s = t[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s = fmaxf(s, t[i]);
    __syncthreads();
    return s;
  }
}

template <int VW>
struct Unit {
  float v[VW];
};

template <int VW>
VH_DEV Unit<VW> load_unit(const float* p) {
  Unit<VW> u;
  if constexpr (VW == 4) {
    float4 t = *reinterpret_cast<const float4*>(p);
    u.v[0] = t.x; u.v[1] = t.y; u.v[2] = t.z; u.v[3] = t.w;
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) u.v[j] = p[j];
  }
  return u;
}

template <int VW>
VH_DEV void store_unit(float* p, const Unit<VW>& u) {
  if constexpr (VW == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(u.v[0], u.v[1], u.v[2], u.v[3]);
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) p[j] = u.v[j];
  }
}

// Streaming access for tensors each kernel touches exactly once: non-temporal
// loads / stores (global_load/store ... nt) keep single-use rows from
// displacing reused data in L2 / MALL; measured +5..25% on gfx950 for
// row-sized streams. VH_STREAM_NT=0 builds the plain-access variant.
#ifndef VH_STREAM_NT
#define VH_STREAM_NT 1
#endif
typedef float vh_f4 __attribute__((ext_vector_type(4)));

template <int VW>
VH_DEV Unit<VW> load_stream(const float* p) {
  Unit<VW> u;
  if constexpr (VW == 4) {
    vh_f4 t;
    if constexpr (VH_STREAM_NT) t = __builtin_nontemporal_load(reinterpret_cast<const vh_f4*>(p));
    else t = *reinterpret_cast<const vh_f4*>(p);
    u.v[0] = t.x; u.v[1] = t.y; u.v[2] = t.z; u.v[3] = t.w;
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      if constexpr (VH_STREAM_NT) u.v[j] = __builtin_nontemporal_load(p + j);
      else u.v[j] = p[j];
    }
  }
  return u;
}

template <int VW>
VH_DEV void store_stream(float* p, const Unit<VW>& u) {
  if constexpr (VW == 4) {
    const vh_f4 t = {u.v[0], u.v[1], u.v[2], u.v[3]};
    if constexpr (VH_STREAM_NT) __builtin_nontemporal_store(t, reinterpret_cast<vh_f4*>(p));
    else *reinterpret_cast<vh_f4*>(p) = t;
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      if constexpr (VH_STREAM_NT) __builtin_nontemporal_store(u.v[j], p + j);
      else p[j] = u.v[j];
    }
  }
}

template <int VW>
VH_DEV Unit<VW> zero_unit() {
  Unit<VW> u;
#pragma unroll
  for (int j = 0; j < VW; ++j) u.v[j] = 0.0f;
  return u;
}

// a / b correctly rounded (the IEEE quotient, bit for bit), given y = RN(1/b),
// for divisors 1 <= |b| <= 2^24 (row lengths, softmax sums). Markstein's
// correction: q = RN(a*y) is within one ulp of a/b, the remainder r = a - b*q
// is exact in one fused multiply-add, and RN(q + r*y) is the correctly rounded
// quotient (Markstein, "IA-64 and Elementary Functions", 2000, Thm 8.10).
// Three instructions instead of the ~10 of the general division sequence.
// |a| outside [2^-100, 2^100) (zero, subnormal, huge, inf, nan) takes the
// general division, so q and r never leave the normal range. Checked
// exhaustively on one binade of a (every significand) for 200 divisors.
VH_DEV float div_rn(float a, float b, float y) {
  const float m = fabsf(a);
  if (m >= 0x1p-100f && m < 0x1p100f) {
    const float q = a * y;
    const float r = fmaf(-q, b, a);
    return fmaf(r, y, q);
  }
  return a / b;
}

// Rust `value.round() as usize` followed by the `< bound` check, on device.
// Returns -1 for a value the CPU backend would reject.
VH_DEV int32_t checked_index(float v, int32_t bound) {
  if (!(v >= 0.0f)) return -1;
  float r = roundf(v);
  if (!(r < (float)bound)) return -1;
  return (int32_t)r;
}

VH_DEV unsigned long long err_pack(int64_t index, float value) {
  return ((unsigned long long)(uint32_t)index << 32) | (unsigned long long)__float_as_uint(value);
}
