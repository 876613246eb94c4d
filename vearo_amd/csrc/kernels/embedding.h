// embedding.h -- embedding gather forward and deterministic scatter-add backward
// for gfx950.
//
// Forward (vearo-backend-cpu embedding, crates/vearo-backend-cpu/src/lib.rs:860-918):
// out[i, :] = W[round(ids[i]), :], a bit-exact copy; one wave per token, 128-bit
// loads/stores when D % 4 == 0. ids are f32 as in the reference API.
//
// Backward (lib.rs:920-980): dW = zeros[V, D]; dW[tok_i] += dy[i] for i ascending.
// No float atomics; dW is written exactly once (dense, 4*V*D bytes), dy read once.
//   1. emb_tokens : validate/round ids; integer histogram of tokens, with the
//                   duplicates inside each wave merged first (one atomic per
//                   distinct token per wave, so hot tokens do not serialise)
//   2. emb_alloc  : rows with more than EMB_LIGHT (16) hits become "heavy": an
//                   entry and one task per 32 hits (ranked in position order),
//                   claimed with one atomic per wave
//   3. emb_place  : light positions drop into their row's 16 fixed slots; heavy
//                   hits are counted per block of positions (512 or more)
//   4. emb_rows   : the leading workgroups run heavy tasks while the rest stream
//                   the vocabulary rows, one wave per row: zeros for an unused
//                   row; for a light row, its <= 16 positions sorted in registers
//                   and the dy rows added in ascending position order from 0.0 --
//                   the CPU loop's exact f32 order, so those rows are bit-exact.
//                   A heavy task gathers the positions of its 32 ranks (visiting
//                   only blocks that hold them) and sums their rows in order into
//                   a partial row, as one wave per 64-unit column slice (one unit
//                   per lane, 16 rows in flight).
//   5. emb_heavy_final: one wave per (heavy row, column slice) adds the row's
//                   partials: each group of 8 in task order, then the group sums
//                   in group order, into dW (a fixed grouping of the same sum:
//                   deterministic, within f32 rounding of the CPU's order). A
//                   kernel of its own: an in-kernel completion tree needs
//                   device-scope fences, and on this GPU each one writes back
//                   and invalidates an XCD's whole L2 (measured: they made the
//                   Zipf case 1.8x slower once the tasks were split in slices).
#pragma once
#include "common.h"

#define EMB_LIGHT 16
#define EMB_CHUNK_HITS 32
#define EMB_GROUP 8
#define EMB_Q 3  // units per lane per pass: 3 x 64 x 4 floats covers D = 768

// acc[q] += rows[r][q] for the first `cnt` of 4 rows, in row order; the loads of
// all rows are issued before any add so a wave pays one memory latency per
// batch of 4 rows instead of one per row. NT selects streaming loads (dy, read
// once) over plain ones (partial rows, just written by other waves).
template <int VW, bool NT>
VH_DEV void emb_add_rows(Unit<VW> (&acc)[EMB_Q], const float* const (&src)[4], int cnt, int u0, int lane, int U) {
  Unit<VW> d[4][EMB_Q];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int q = 0; q < EMB_Q; ++q) {
      const int u = u0 + lane + q * 64;
      if (r < cnt && u < U)
        d[r][q] = NT ? load_stream<VW>(src[r] + u * VW) : load_unit<VW>(src[r] + u * VW);
      else
        d[r][q] = zero_unit<VW>();
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (r < cnt) {
#pragma unroll
      for (int q = 0; q < EMB_Q; ++q) {
#pragma unroll
        for (int j = 0; j < VW; ++j) acc[q].v[j] += d[r][q].v[j];
      }
    }
  }
}

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

// Bitonic sort of one value per lane within each group of KMAX lanes
// (ascending by lane; KMAX = 64 sorts the whole wave).
template <int KMAX>
VH_DEV int32_t wave_bitonic_sort(int32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= KMAX; k <<= 1) {
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

// Step 1. 256-thread workgroups over positions.
VH_DEV void emb_tokens_impl(const EmbTokArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int32_t t = -1;
  if (i < a.n) {
    const float tv = a.ids[i];
    t = checked_index(tv, a.V);
    a.tok[i] = t;
    if (t < 0) {
      atomicMin(&a.err->token, err_pack(i, tv));
      a.err->token_bound = (unsigned)a.V;
    }
  }
  // Merge duplicates within the wave: sort the 64 tokens, one atomic per run.
  const int32_t s = wave_bitonic_sort<64>(t < 0 ? INT32_MAX : t);
  const int32_t prev = __shfl(s, (lane + 63) & 63, 64);
  const bool boundary = lane == 0 || prev != s;
  const unsigned long long heads = __ballot(boundary);
  if (boundary && s != INT32_MAX) {
    const unsigned long long above = lane == 63 ? 0ull : heads & (~0ull << (lane + 1));
    const int next = above ? __builtin_ctzll(above) : 64;
    atomicAdd(&a.counts[s], next - lane);
  }
}

// Step 2. One thread per vocabulary row. Rows with more than EMB_LIGHT hits are
// registered as heavy: an entry, a run of ceil(hits/32) tasks and a zeroed
// per-block hit-count row. Entries and tasks are
// claimed with one atomic per wave (a wave prefix sum, then one atomicAdd of the
// totals); their order varies run to run but no row's result depends on it.
VH_DEV void emb_alloc_impl(const EmbAllocArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t c = v < a.V ? a.counts[v] : 0;
  const bool heavy = c > EMB_LIGHT;
  const int32_t nch = heavy ? (c + EMB_CHUNK_HITS - 1) / EMB_CHUNK_HITS : 0;
  // Low 32 bits: heavy rows; high 32 bits: tasks.
  const int64_t mine = heavy ? (((int64_t)nch << 32) | 1) : 0;
  int64_t inc = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t u = __shfl_up(inc, off, 64);
    if (lane >= off) inc += u;
  }
  int32_t hbase = 0, tbase = 0;
  if (lane == 63 && inc != 0) {
    hbase = atomicAdd(&a.ctr[0], (int32_t)(inc & 0xffffffff));
    tbase = atomicAdd(&a.ctr[1], (int32_t)(inc >> 32));
  }
  hbase = __shfl(hbase, 63, 64);
  tbase = __shfl(tbase, 63, 64);
  if (v >= a.V) return;
  int32_t h = -1;
  if (heavy) {
    const int64_t ex = inc - mine;
    h = hbase + (int32_t)(ex & 0xffffffff);
    const int32_t tb = tbase + (int32_t)(ex >> 32);
    a.heavy[4 * h + 0] = (int32_t)v;
    a.heavy[4 * h + 1] = tb;
    a.heavy[4 * h + 2] = nch;
    a.heavy[4 * h + 3] = c;
    for (int32_t k = 0; k < nch; ++k) a.taskmap[tb + k] = h;
    for (int32_t b = 0; b < a.nblk; ++b) a.blkcnt[(int64_t)h * a.nblk + b] = 0;
  }
  a.heavy_index[v] = h;
}

// Step 3. One thread per position: light positions go to their row's slots (at
// most 16 atomics per row); heavy hits are counted per 2^blk_shift-position block, with
// one atomic per (heavy token, wave) after merging the wave's duplicates.
VH_DEV void emb_place_impl(const EmbPlaceArgs& a) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int32_t h = -1;
  if (i < a.n) {
    const int32_t t = a.tok[i];
    if (t >= 0) {
      h = a.heavy_index[t];
      if (h < 0) a.pos[(int64_t)t * EMB_LIGHT + atomicAdd(&a.cursor[t], 1)] = (int32_t)i;
    }
  }
  const int32_t s = wave_bitonic_sort<64>(h < 0 ? INT32_MAX : h);
  const int32_t prev = __shfl(s, (lane + 63) & 63, 64);
  const bool boundary = lane == 0 || prev != s;
  const unsigned long long heads = __ballot(boundary);
  if (boundary && s != INT32_MAX) {
    const unsigned long long above = lane == 63 ? 0ull : heads & (~0ull << (lane + 1));
    const int next = above ? __builtin_ctzll(above) : 64;
    // The wave's 64 positions share one block (blocks hold >= 64 positions).
    const int64_t blk = (i - lane) >> a.blk_shift;
    atomicAdd(&a.blkcnt[(int64_t)s * a.nblk + blk], next - lane);
  }
}

// Index of the n-th (0-based) set bit of m; requires n < popcount(m).
VH_DEV int nth_set_bit(unsigned long long m, int n) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const int c = __popcll(m & ((1ull << w) - 1));
    if (n >= c) {
      n -= c;
      m >>= w;
      pos += w;
    }
  }
  return pos;
}

#define EMB_BATCH 16  // rows in flight per lane in a heavy task's slice

// acc += rows[r] at unit u (one unit per lane) for the first `cnt` of R rows, in
// row order; all R loads are issued before any add. NT as in emb_add_rows.
template <int VW, bool NT, int R>
VH_DEV void emb_add_slice(Unit<VW>& acc, const float* const (&src)[R], int cnt, int u, int U) {
  Unit<VW> d[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < cnt && u < U)
      d[r] = NT ? load_stream<VW>(src[r] + u * VW) : load_unit<VW>(src[r] + u * VW);
    else
      d[r] = zero_unit<VW>();
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < cnt) {
#pragma unroll
      for (int j = 0; j < VW; ++j) acc.v[j] += d[r].v[j];
    }
  }
}

// dst at unit u = sum over c < cnt of rows base + c * stride at unit u, added
// in c order from 0.0.
template <int VW>
VH_DEV void emb_sum_slice(const float* base, int64_t stride, int cnt, float* dst, bool stream_out, int u, int U) {
  Unit<VW> acc = zero_unit<VW>();
  for (int c = 0; c < cnt; c += EMB_BATCH) {
    const float* src[EMB_BATCH];
#pragma unroll
    for (int r = 0; r < EMB_BATCH; ++r) src[r] = base + (int64_t)(c + r < cnt ? c + r : c) * stride;
    emb_add_slice<VW, false, EMB_BATCH>(acc, src, cnt - c < EMB_BATCH ? cnt - c : EMB_BATCH, u, U);
  }
  if (u < U) {
    if (stream_out)
      store_stream<VW>(dst + u * VW, acc);
    else
      store_unit<VW>(dst + u * VW, acc);
  }
}

// Heavy work item = (task k, column slice sl): task k covers the hits of rank
// [32c, 32c+32) of its token (ranks in position order). Lane j first gathers
// the position of the j-th of them, visiting only blocks whose hit count
// overlaps the rank window; then the dy rows are summed in position order into
// the slice's columns of partial[k], lane l owning unit 64 sl + l.
template <int VW>
VH_DEV void emb_heavy_task(const EmbSegArgs& a, int64_t item, int lane) {
  const int U = a.D / VW;
  const int64_t k = item / a.slices;
  const int sl = (int)(item % a.slices);
  const int u = sl * 64 + lane;
  const int32_t h = a.taskmap[k];
  const int32_t tok = a.heavy[4 * h + 0], tb = a.heavy[4 * h + 1], nch = a.heavy[4 * h + 2];
  const int32_t m = a.heavy[4 * h + 3];
  const int32_t c = (int32_t)(k - tb);
  const int32_t r0 = c * EMB_CHUNK_HITS;
  const int32_t r1 = min(r0 + EMB_CHUNK_HITS, m);
  const int32_t* cnt = a.blkcnt + (int64_t)h * a.nblk;
  int32_t rr = 0;      // hits in the blocks before the current 64-block chunk
  int32_t got = 0;     // positions gathered so far (wave-uniform)
  int32_t mypos = 0;   // lane j < got: the j-th gathered position
  for (int32_t b0 = 0; b0 < a.nblk && rr < r1; b0 += 64) {
    const int32_t cb = b0 + lane < a.nblk ? cnt[b0 + lane] : 0;
    int32_t inc = cb;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t u = __shfl_up(inc, off, 64);
      if (lane >= off) inc += u;
    }
    const int32_t before = rr + inc - cb;  // hits before this lane's block
    unsigned long long want = __ballot(cb > 0 && before < r1 && before + cb > r0);
    while (want) {
      const int l = __builtin_ctzll(want);
      want &= want - 1;
      int32_t br = __shfl(before, l, 64);  // rank of the block's first hit
      const int64_t p_end = min(((int64_t)(b0 + l) + 1) << a.blk_shift, a.n);
      for (int64_t pb = (int64_t)(b0 + l) << a.blk_shift; pb < p_end && br < r1; pb += 512) {
        int32_t tk[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const int64_t p = pb + g * 64 + lane;
          tk[g] = p < p_end ? a.tok[p] : -1;
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const unsigned long long mask = __ballot(tk[g] == tok);
          const int hits = __popcll(mask);
          // This group's ranks are [br, br + hits); take those in [r0, r1).
          const int lo = max(r0 - br, 0);
          const int hi = min(r1 - br, hits);
          if (hi > lo) {
            if (lane >= got && lane < got + (hi - lo))
              mypos = (int32_t)(pb + g * 64 + nth_set_bit(mask, lane - got + lo));
            got += hi - lo;
          }
          br += hits;
        }
      }
    }
    rr += __shfl(inc, 63, 64);
  }
  float* part = a.partial + k * (int64_t)a.D;
  Unit<VW> acc = zero_unit<VW>();
  for (int j = 0; j < got; j += EMB_BATCH) {  // ascending positions, 16 rows per batch
    const float* src[EMB_BATCH];
#pragma unroll
    for (int r = 0; r < EMB_BATCH; ++r) src[r] = a.dy + (int64_t)__shfl(mypos, j + r < got ? j + r : j, 64) * a.D;
    emb_add_slice<VW, true, EMB_BATCH>(acc, src, got - j < EMB_BATCH ? got - j : EMB_BATCH, u, U);
  }
  if (u < U) store_unit<VW>(part + u * VW, acc);
}

// Step 4. Blocks [0, heavy_blocks): heavy work items (task, column slice), one
// per wave, strided over the device-side task count times the slices;
// dispatched first, so they overlap the row stream.
// Blocks beyond: one wave per vocabulary row (zeros, or a light row's bit-exact
// sequential sum; heavy rows are left to their tasks).
template <int VW>
VH_DEV void emb_rows_impl(const EmbSegArgs& a) {
  const int lane = threadIdx.x & 63;
  const int U = a.D / VW;
  if ((int)blockIdx.x >= a.heavy_blocks) {
    const int64_t v = ((int64_t)blockIdx.x - a.heavy_blocks) * 4 + (threadIdx.x >> 6);
    if (v >= a.V) return;
    const int32_t m = a.counts[v];
    if (m > EMB_LIGHT) return;
    float* o = a.dW + v * a.D;
    int32_t sorted = INT32_MAX;
    if (m > 0) sorted = lane < m ? a.pos[v * EMB_LIGHT + lane] : INT32_MAX;
    if (m > 1) sorted = wave_bitonic_sort<EMB_LIGHT>(sorted);
    for (int u0 = 0; u0 < U; u0 += 64 * EMB_Q) {
      Unit<VW> acc[EMB_Q];
#pragma unroll
      for (int q = 0; q < EMB_Q; ++q) acc[q] = zero_unit<VW>();
      for (int32_t k = 0; k < m; k += 4) {  // ascending positions, 4 rows per batch
        const float* src[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) src[r] = a.dy + (int64_t)__shfl(sorted, k + r < m ? k + r : k, 64) * a.D;
        emb_add_rows<VW, true>(acc, src, m - k < 4 ? m - k : 4, u0, lane, U);
      }
#pragma unroll
      for (int q = 0; q < EMB_Q; ++q) {
        const int u = u0 + lane + q * 64;
        if (u < U) store_stream<VW>(o + u * VW, acc[q]);
      }
    }
    return;
  }
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nworkers = (int64_t)a.heavy_blocks * 4;
  const int64_t nitems = (int64_t)a.ctr[1] * a.slices;
  for (int64_t k = wid; k < nitems; k += nworkers) emb_heavy_task<VW>(a, k, lane);
}

// Step 5. Work item w = (heavy entry h, column slice sl), one wave at a time,
// strided over the device-side count of heavy entries: dW[tok] at the slice's
// units = sum over groups (in order, from 0.0) of the group's partials summed
// in task order from 0.0; a row with one group takes that group's sum as it
// is. Four groups' partials are loaded at once.
#define EMB_FINAL_GROUPS 4
template <int VW>
VH_DEV void emb_heavy_final_impl(const EmbFinalArgs& a) {
  const int lane = threadIdx.x & 63;
  const int U = a.D / VW;
  const int64_t nitems = (int64_t)a.ctr[0] * a.slices;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); w < nitems; w += nwaves) {
    const int64_t h = w / a.slices;
    const int u = (int)(w % a.slices) * 64 + lane;
    const int32_t tok = a.heavy[4 * h + 0], tb = a.heavy[4 * h + 1], nch = a.heavy[4 * h + 2];
    const int32_t ngrp = (nch + EMB_GROUP - 1) / EMB_GROUP;
    Unit<VW> total = zero_unit<VW>();
    for (int32_t g0 = 0; g0 < ngrp; g0 += EMB_FINAL_GROUPS) {
      Unit<VW> d[EMB_FINAL_GROUPS][EMB_GROUP];
#pragma unroll
      for (int q = 0; q < EMB_FINAL_GROUPS; ++q) {
        const int32_t g = g0 + q;
        const int32_t gsize = g < ngrp ? min(EMB_GROUP, nch - g * EMB_GROUP) : 0;
#pragma unroll
        for (int r = 0; r < EMB_GROUP; ++r) {
          if (r < gsize && u < U)
            d[q][r] = load_unit<VW>(a.partial + (int64_t)(tb + g * EMB_GROUP + r) * a.D + u * VW);
          else
            d[q][r] = zero_unit<VW>();
        }
      }
#pragma unroll
      for (int q = 0; q < EMB_FINAL_GROUPS; ++q) {
        const int32_t g = g0 + q;
        if (g < ngrp) {
          const int32_t gsize = min(EMB_GROUP, nch - g * EMB_GROUP);
          Unit<VW> gs = zero_unit<VW>();
#pragma unroll
          for (int r = 0; r < EMB_GROUP; ++r) {
            if (r < gsize) {
#pragma unroll
              for (int j = 0; j < VW; ++j) gs.v[j] += d[q][r].v[j];
            }
          }
          if (ngrp == 1) {
            total = gs;
          } else {
#pragma unroll
            for (int j = 0; j < VW; ++j) total.v[j] += gs.v[j];
          }
        }
      }
    }
    if (u < U) store_stream<VW>(a.dW + (int64_t)tok * a.D + u * VW, total);
  }
}
