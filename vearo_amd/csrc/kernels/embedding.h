// embedding.h -- embedding gather forward and sort-by-token segmented-sum backward
// for gfx950.
//
// Forward (vearo-backend-cpu embedding, crates/vearo-backend-cpu/src/lib.rs:860-918):
// out[i, :] = W[round(ids[i]), :], a bit-exact copy; one wave per token, 128-bit
// loads/stores when D % 4 == 0. ids are f32 as in the reference API.
//
// Backward (lib.rs:920-980): dW = zeros[V, D]; dW[tok_i] += dy[i] for i ascending.
// Atomic-free on the floats, deterministic, and bit-exact with the CPU's order:
//   1. emb_tokens : validate/round ids, integer histogram of tokens
//   2. scan       : exclusive prefix sum -> CSR offsets [V+1]
//   3. emb_place  : drop each position into its token's segment
//   4. emb_sort_big: sort the positions of every segment longer than 64
//                   ascending (workgroup bitonic network in LDS)
//   5. emb_segsum : one wave per vocabulary row: sort a short segment in
//                   registers, sum its dy rows in ascending position order (the
//                   same f32 order as the CPU loop), or write zeros
// so dW is written exactly once (dense, 4*V*D bytes) and dy read once.
// Integer atomics in steps 1 and 3 only count; the float sums never use atomics.
#pragma once
#include "common.h"

// One wave per token, 4 waves per 256-thread workgroup.
template <int VW>
VH_DEV void emb_fwd_impl(const EmbFwdArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= a.n) return;
  const float tv = a.ids[i];
  const int32_t t = checked_index(tv, a.V);
  const int U = a.D / VW;
  float* o = a.out + i * a.D;
  if (t < 0) {
    if (lane == 0) {
      atomicMin(&a.err->token, err_pack(i, tv));
      a.err->token_bound = (unsigned)a.V;
    }
    for (int u = lane; u < U; u += 64) store_stream<VW>(o + u * VW, zero_unit<VW>());
    return;
  }
  const float* w = a.W + (int64_t)t * a.D;
  for (int u = lane; u < U; u += 64) store_stream<VW>(o + u * VW, load_unit<VW>(w + u * VW));
}

VH_DEV void emb_tokens_impl(const EmbTokArgs& a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const float tv = a.ids[i];
  const int32_t t = checked_index(tv, a.V);
  a.tok[i] = t;
  if (t < 0) {
    atomicMin(&a.err->token, err_pack(i, tv));
    a.err->token_bound = (unsigned)a.V;
  } else {
    atomicAdd(&a.counts[t], 1);
  }
}

// Single-workgroup exclusive scan of n int32 (1024 threads, contiguous chunk per
// thread), total stored at data[n].
VH_DEV void scan_impl(const ScanArgs& a) {
  // Also lists the entries whose count exceeds 64 (long embedding segments).
  __shared__ int32_t part[1024];
  const int t = threadIdx.x;
  const int chunk = (a.n + 1023) / 1024;
  const int s0 = t * chunk;
  int s1 = s0 + chunk;
  if (s1 > a.n) s1 = a.n;
  int32_t local = 0;
  for (int i = s0; i < s1; ++i) local += a.data[i];
  part[t] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 1024 partials.
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int32_t run = t > 0 ? part[t - 1] : 0;
  for (int i = s0; i < s1; ++i) {
    const int32_t c = a.data[i];
    a.data[i] = run;
    run += c;
    if (a.big && c > 64) a.big[atomicAdd(a.nbig, 1)] = i;
  }
  if (t == 1023) a.data[a.n] = part[1023];
}

VH_DEV void emb_place_impl(const EmbPlaceArgs& a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const int32_t t = a.tok[i];
  if (t < 0) return;
  const int32_t slot = a.offsets[t] + atomicAdd(&a.cursor[t], 1);
  a.pos[slot] = (int32_t)i;
}

// Bitonic sort of one value per lane across the wave (ascending by lane).
VH_DEV int32_t wave_bitonic_sort(int32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int32_t o = __shfl_xor(v, j, 64);
      const bool up = (lane & k) == 0;
      const bool lower = (lane & j) == 0;
      const int32_t lo = v < o ? v : o;
      const int32_t hi = v < o ? o : v;
      v = (lower == up) ? lo : hi;
    }
  }
  return v;
}

// Step 4 (segments longer than 64 only; shorter ones are sorted in registers by
// emb_segsum). The scan kernel lists the long segments; a fixed grid of
// workgroups walks that list, each sorting one segment at a time with a bitonic
// network over a padded power-of-two buffer: LDS when it fits, else a private
// slice [2*s0, 2*s0 + P) of the global staging buffer (P < 2m, so slices of
// different segments never overlap and stay inside its 2n entries).
#define EMB_SORT_LDS 8192

VH_DEV void emb_sort_big_impl(const EmbSortArgs& a) {
  __shared__ int32_t buf[EMB_SORT_LDS];
  const int32_t nbig = *a.nbig;
  for (int32_t idx = blockIdx.x; idx < nbig; idx += gridDim.x) {
    const int32_t v = a.big[idx];
    const int32_t s0 = a.offsets[v];
    const int32_t m = a.offsets[v + 1] - s0;
    int32_t* seg = a.pos + s0;
    int P = 128;
    while (P < m) P <<= 1;
    int32_t* b = (P <= EMB_SORT_LDS) ? buf : a.gbuf + 2 * (int64_t)s0;
    for (int i = threadIdx.x; i < P; i += blockDim.x) b[i] = i < m ? seg[i] : 0x7FFFFFFF;
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = threadIdx.x; i < P; i += blockDim.x) {
          const int l = i ^ j;
          if (l > i) {
            const int32_t x = b[i], y = b[l];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              b[i] = y;
              b[l] = x;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int i = threadIdx.x; i < m; i += blockDim.x) seg[i] = b[i];
    __syncthreads();
  }
}

// Step 5. One wave per vocabulary row, 4 waves per workgroup. Segments of up to
// 64 positions are sorted here in registers; longer ones arrive sorted.
template <int VW>
VH_DEV void emb_segsum_impl(const EmbSegArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= a.V) return;
  const int32_t s0 = a.offsets[v];
  const int32_t m = a.offsets[v + 1] - s0;
  const int D = a.D;
  const int U = D / VW;
  float* o = a.dW + v * D;
  int32_t sorted = 0x7FFFFFFF;
  if (m <= 64) {
    sorted = lane < m ? a.pos[s0 + lane] : 0x7FFFFFFF;
    sorted = wave_bitonic_sort(sorted);
  }
  for (int u0 = 0; u0 < U; u0 += 64 * 4) {
    // Up to 4 units per lane per pass keep 4 independent loads in flight.
    Unit<VW> acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = zero_unit<VW>();
    for (int32_t k = 0; k < m; ++k) {
      const int32_t p = m <= 64 ? __shfl(sorted, k, 64) : a.pos[s0 + k];
      const float* src = a.dy + (int64_t)p * D;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int u = u0 + lane + q * 64;
        if (u < U) {
          const Unit<VW> d = load_stream<VW>(src + u * VW);
#pragma unroll
          for (int j = 0; j < VW; ++j) acc[q].v[j] += d.v[j];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int u = u0 + lane + q * 64;
      if (u < U) store_stream<VW>(o + u * VW, acc[q]);
    }
  }
}
