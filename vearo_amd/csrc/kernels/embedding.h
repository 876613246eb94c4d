// embedding.h -- embedding gather forward and deterministic scatter-add backward
// for gfx950.
//
// Forward (vearo-backend-cpu embedding, crates/vearo-backend-cpu/src/lib.rs:860-918):
// out[i, :] = W[round(ids[i]), :], a bit-exact copy; one wave per token, 128-bit
// loads/stores when D % 4 == 0. ids are f32 as in the reference API.
//
// Backward (lib.rs:920-980): dW = zeros[V, D]; dW[tok_i] += dy[i] for i ascending.
// No float atomics; dy is read once. A token with at most EMB_LIGHT (16) hits is
// "light": its row is the sum of its dy rows in ascending position order from
// 0.0 -- the CPU loop's exact f32 order, so the row is bit-exact. A "heavy"
// token's hits are cut, in position order, into tasks of EMB_CHUNK_HITS (32);
// each task's dy rows are summed in order into a partial row, and the row is
// the sum, in order from 0.0, of the sums of groups of EMB_GROUP (8) tasks in
// task order (a fixed grouping: deterministic, within f32 rounding of the CPU's
// single chain; one chain of the Zipf top id's 2292 rows would alone outlast
// the whole backward).
//
// Sorted path (n <= 16384, V <= 65534 -- every BASELINE config), two launches:
//   1. emb_sort : workgroups 0..15 each own the tokens t % 16 == k: each reads
//                 all n ids, keeps its range's keys (t / 16 << 14 | position),
//                 sorts them by token in LDS (a stable LSD radix sort, two 6-bit
//                 passes; ranks among equal digits from wave ballots, no
//                 atomics), cuts the sorted keys into one segment per token and
//                 numbers the heavy tokens and their tasks with prefix sums
//                 (segment records, heavy entries, task map). The other
//                 workgroups write dW's zeros meanwhile (154 MB at GPT-2 size,
//                 long enough to hide the sorts).
//   2. emb_sum  : one wave per (heavy task, 64-unit column slice) first, then
//                 one wave per segment. A light segment's wave adds its dy rows
//                 and writes the row. A heavy task's wave writes its partial
//                 and counts itself done; the wave that finishes a group adds
//                 the group's partials, and the wave that finishes a row's last
//                 group adds the group sums into dW -- with device-coherent
//                 stores and loads and a wait for the stores before each count,
//                 so no launch boundary or whole-L2 fence is needed between
//                 them. The heavy waves start first, so those combines run
//                 under the light segments' stream.
// General path (larger n or V), five launches and integer atomics on counters:
//   1. emb_tokens : validate/round ids; integer histogram of tokens, with the
//                   duplicates inside each wave merged first (one atomic per
//                   distinct token per wave, so hot tokens do not serialise)
//   2. emb_alloc  : heavy rows get an entry and their tasks (ranked in
//                   position order), claimed with one atomic per wave
//   3. emb_place  : light positions drop into their row's 16 fixed slots; heavy
//                   hits are counted per block of positions (512 or more)
//   4. emb_rows   : the leading workgroups run heavy tasks while the rest stream
//                   the vocabulary rows, one wave per row: zeros for an unused
//                   row; for a light row, its <= 16 positions sorted in registers
//                   and the dy rows added in ascending position order from 0.0.
//                   A heavy task gathers the positions of its 32 ranks (visiting
//                   only blocks that hold them) and sums their rows in order into
//                   a partial row, as one wave per 64-unit column slice.
//   5. emb_heavy_final: one wave per (heavy row, column slice) adds the row's
//                   partials with the grouping above.
// The two paths give the same bits: the same light-row order, the same 32-hit
// tasks and the same final grouping.
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

// ------------------------------------------------------------- sorted path --
#define EMB_SORT_N 16384   // keys a range workgroup holds (n <= this)
#define EMB_CNT_STRIDE 17  // words per digit row of the [digit][wave] counts (odd: no bank conflicts)
#define EMB_LT_BITS 6      // bits per pass over the 12-bit range-local token

// Inclusive prefix sum over the 64 lanes of a wave (DPP row shifts within
// rows of 16, then the row_bcast steps across rows; lanes a step does not
// write keep 0 to add).
VH_DEV uint32_t wave_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

// Exclusive prefix over the 16 waves of the workgroup of one wave-uniform
// value per wave: returns the sum over lower waves, *total the sum over all.
// Every thread must call (two barriers).
VH_DEV uint32_t waves_excl_scan(uint32_t v, uint32_t* wsum, uint32_t* total) {
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) wsum[w] = v;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t t = wsum[i];
    before += i < w ? t : 0u;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before;
}

// Count of the lanes below this one in mask m.
VH_DEV uint32_t lanes_below(unsigned long long m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Launch 1 of the sorted path, 1024-thread workgroups. Workgroup k <
// EMB_RANGES owns the tokens t with t % EMB_RANGES == k (so a distribution's
// hot tokens spread over the workgroups): it reads every id, keeps its
// positions in position order, sorts them by t / EMB_RANGES (a stable LSD
// radix sort of two 6-bit passes; each key's rank among the earlier keys of
// its wave with the same digit comes from six wave ballots -- a lane keeps a
// ballot where its bit is 1 and its complement where it is 0 -- no atomics)
// into its own spos region, then cuts them into one segment per token and
// numbers the heavy tokens (> EMB_LIGHT hits) and their 32-hit tasks, in token
// order, with prefix sums. The other workgroups write dW's zeros (154 MB at
// GPT-2 size, long enough to hide the sorts); launch 2 rewrites the rows with
// hits. (Zeroing only the rows no id names, from a row bitmap each filler
// builds from all ids, was measured: 2.5 us faster on uniform ids, 2-4 us
// slower on Zipf ids, whose hot ids share bitmap words and serialise the
// atomics that set them.)
VH_DEV void emb_sort_impl(const EmbSortArgs& a) {
  if ((int)blockIdx.x >= EMB_RANGES) {
    // Four stores per iteration (one grid stride apart), then the rest.
    const int64_t stride = (int64_t)(gridDim.x - EMB_RANGES) * blockDim.x;
    int64_t u = (int64_t)(blockIdx.x - EMB_RANGES) * blockDim.x + threadIdx.x;
    if (a.vec) {
      for (; u + 3 * stride < a.fill_n; u += 4 * stride) {
#pragma unroll
        for (int j = 0; j < 4; ++j) store_stream<4>(a.dW + (u + j * stride) * 4, zero_unit<4>());
      }
      for (; u < a.fill_n; u += stride) store_stream<4>(a.dW + u * 4, zero_unit<4>());
    } else {
      for (; u + 3 * stride < a.fill_n; u += 4 * stride) {
#pragma unroll
        for (int j = 0; j < 4; ++j) store_stream<1>(a.dW + u + j * stride, zero_unit<1>());
      }
      for (; u < a.fill_n; u += stride) store_stream<1>(a.dW + u, zero_unit<1>());
    }
    return;
  }
  __shared__ uint32_t kb[2][EMB_SORT_N];
  __shared__ uint32_t cnt[2][64 * EMB_CNT_STRIDE];
  __shared__ uint32_t wsum[2][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int tid = threadIdx.x;
  const int rk = blockIdx.x;
  for (int e = tid; e < 2 * 64 * EMB_CNT_STRIDE; e += 1024) (&cnt[0][0])[e] = 0;
  // Launch 2 counts finished groups per (heavy entry, slice) and finished
  // tasks per (group, slice) from zero.
  {
    int32_t* c = a.ctr + (size_t)rk * (a.hmax + a.tmax) * a.slices;
    for (int e = tid; e < (a.hmax + a.tmax) * a.slices; e += 1024) c[e] = 0;
  }

  // 1. Lane l of wave w holds position w*1024 + r*64 + l in slot r. Range 0
  // reports invalid ids. Each wave keeps its range's keys (local token << 14
  // | position) in position order in its own LDS region kb[0][1024 w ...).
  uint32_t mw = 0;  // keys in this wave's region
  {
    float tv[16];  // all 16 loads in flight before the checks
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = w * 1024 + r * 64 + lane;
      tv[r] = i < a.n ? a.ids[i] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = w * 1024 + r * 64 + lane;
      const int32_t t = i < a.n ? checked_index(tv[r], a.V) : -1;
      if (rk == 0 && i < a.n && t < 0) {
        atomicMin(&a.err->token, err_pack(i, tv[r]));  // the panic report, not the sum
        a.err->token_bound = (unsigned)a.V;
      }
      const bool in = t >= 0 && (t % EMB_RANGES) == rk;
      const unsigned long long mk = __ballot(in);
      if (in) kb[0][w * 1024 + mw + lanes_below(mk)] = ((uint32_t)(t / EMB_RANGES) << 14) | (uint32_t)i;
      mw += (uint32_t)__popcll(mk);
    }
  }
  uint32_t m;
  (void)waves_excl_scan(mw, wsum[0], &m);
  // 2. Stable LSD sort by the local token. Pass 0 reads the waves' regions,
  // pass 1 the dense result [0, m) in chunks of `per` per wave; either way
  // (wave, round, lane) order is the input order.
  const uint32_t per = ((m + 1023) / 1024) * 64;
  uint32_t k[16], rank[16];
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const uint32_t* src = kb[pass];
    uint32_t* dst = kb[pass ^ 1];
    uint32_t* cn = cnt[pass];
    const int shift = 14 + EMB_LT_BITS * pass;
    const uint32_t jb = pass == 0 ? (uint32_t)w * 1024 : (uint32_t)w * per;
    const uint32_t jn = pass == 0 ? mw : (m > (uint32_t)w * per ? min(per, m - (uint32_t)w * per) : 0u);
    const int rounds = (int)((jn + 63) / 64);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (r < rounds) {
        const uint32_t j = (uint32_t)(r * 64 + lane);
        const bool act = j < jn;
        k[r] = act ? src[jb + j] : 0u;
        const unsigned long long am = __ballot(act);
        uint32_t plo = (uint32_t)am, phi = (uint32_t)(am >> 32);
#pragma unroll
        for (int b = 0; b < EMB_LT_BITS; ++b) {
          const uint32_t rep = (uint32_t)__builtin_amdgcn_sbfe((int)k[r], shift + b, 1);  // 0 or ~0
          const unsigned long long bal = __ballot(rep != 0u);
          plo &= ~((uint32_t)bal ^ rep);
          phi &= ~((uint32_t)(bal >> 32) ^ rep);
        }
        if (act) {
          const unsigned long long peers = ((unsigned long long)phi << 32) | plo;
          const uint32_t lt = lanes_below(peers);
          const uint32_t at = ((k[r] >> shift) & 63u) * EMB_CNT_STRIDE + (uint32_t)w;
          const uint32_t base = cn[at];
          rank[r] = base + lt;
          if (lt == 0) cn[at] = base + (uint32_t)__popcll(peers);
        }
      }
    }
    __syncthreads();
    // Offsets: exclusive prefix over (digit, wave) in that order (64 x 16 =
    // 1024 entries, one per thread), so keys land by digit, then wave, round, lane.
    {
      const uint32_t at = (uint32_t)(tid >> 4) * EMB_CNT_STRIDE + (uint32_t)(tid & 15);
      const uint32_t c = cn[at];
      const uint32_t inc = wave_incl_scan(c);
      uint32_t all;
      const uint32_t before = waves_excl_scan(__shfl(inc, 63, 64), wsum[pass], &all);
      cn[at] = before + inc - c;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (r < rounds && (uint32_t)(r * 64 + lane) < jn)
        dst[cn[((k[r] >> shift) & 63u) * EMB_CNT_STRIDE + (uint32_t)w] + rank[r]] = k[r];
    }
    __syncthreads();
  }
  const uint32_t* sorted = kb[0];
  int32_t* sposk = a.spos + (size_t)rk * a.n;
  // m <= EMB_SORT_N = 16 x 1024: a fixed count of predicated rounds (a loop
  // bounded by m left the kernel with an unused private-memory frame).
#pragma unroll
  for (int r = 0; r < EMB_SORT_N / 1024; ++r) {
    const uint32_t j = (uint32_t)(r * 1024 + tid);
    if (j < m) sposk[j] = (int32_t)(sorted[j] & 0x3FFFu);
  }
  // 3. Segments: heads (a local token differing from the previous key's),
  // numbered by the count of heads before them.
  const uint32_t jw = (uint32_t)w * per;
  const int rounds = (int)(per / 64);
  auto head_mask = [&](int r) {
    const uint32_t j = jw + (uint32_t)(r * 64 + lane);
    const bool head = j < m && (j == 0 || (sorted[j] >> 14) != (sorted[j - 1] >> 14));
    return __ballot(head);
  };
  uint32_t nh = 0;
  for (int r = 0; r < rounds; ++r) nh += (uint32_t)__popcll(head_mask(r));
  uint32_t nseg;
  uint32_t s0 = waves_excl_scan(nh, wsum[0], &nseg);
  uint32_t* start = kb[1];  // segment s covers sorted[start[s], start[s + 1]) (the last ends at m)
  for (int r = 0; r < rounds; ++r) {
    const unsigned long long hm = head_mask(r);
    if ((hm >> lane) & 1ull) start[s0 + lanes_below(hm)] = jw + (uint32_t)(r * 64 + lane);
    s0 += (uint32_t)__popcll(hm);
  }
  __syncthreads();
  // 4. Per segment (wave w takes [w pers, (w+1) pers) in rounds of 64): hits,
  // and for heavy ones their entry and first task, numbered in token order.
  const uint32_t pers = ((nseg + 1023) / 1024) * 64;
  const int srounds = (int)(pers / 64);
  const uint32_t sw = (uint32_t)w * pers;
  auto seg_hits = [&](int r) -> uint32_t {
    const uint32_t sg = sw + (uint32_t)(r * 64 + lane);
    return sg < nseg ? (sg + 1 < nseg ? start[sg + 1] : m) - start[sg] : 0u;
  };
  auto tasks_of = [](uint32_t h) -> uint32_t {
    return h > EMB_LIGHT ? (h + EMB_CHUNK_HITS - 1) / EMB_CHUNK_HITS : 0u;
  };
  uint32_t tot_t = 0, tot_h = 0;
  for (int r = 0; r < srounds; ++r) {
    const uint32_t h = seg_hits(r);
    const unsigned long long hv = __ballot(h > EMB_LIGHT);
    if (hv) tot_t += __shfl(wave_incl_scan(tasks_of(h)), 63, 64);
    tot_h += (uint32_t)__popcll(hv);
  }
  uint32_t ntask, nheavy;
  uint32_t tb = waves_excl_scan(tot_t, wsum[0], &ntask);
  uint32_t hb = waves_excl_scan(tot_h, wsum[1], &nheavy);
  int32_t* segk = a.seg + (size_t)rk * a.n * EMB_REC;
  int32_t* heavyk = a.heavy + (size_t)rk * a.hmax * 4;
  int32_t* hstk = a.heavy_start + (size_t)rk * a.hmax;
  int32_t* tmapk = a.taskmap + (size_t)rk * a.tmax;
  for (int r = 0; r < srounds; ++r) {
    const uint32_t sg = sw + (uint32_t)(r * 64 + lane);
    const uint32_t h = seg_hits(r), nt = tasks_of(h);
    const unsigned long long hv = __ballot(h > EMB_LIGHT);
    const uint32_t tinc = hv ? wave_incl_scan(nt) : 0u;
    if (sg < nseg) {
      const uint32_t st = start[sg];
      const int32_t tok = (int32_t)(sorted[st] >> 14) * EMB_RANGES + rk;
      int32_t* rec = segk + (size_t)EMB_REC * sg;
      *reinterpret_cast<int4*>(rec) = make_int4(tok, (int32_t)st, (int32_t)h, 0);
      if (h <= EMB_LIGHT) {
        for (uint32_t q = 0; q < h; ++q) rec[4 + q] = (int32_t)(sorted[st + q] & 0x3FFFu);
      } else {
        const uint32_t e = hb + lanes_below(hv);
        const uint32_t t0 = tb + tinc - nt;
        *reinterpret_cast<int4*>(heavyk + 4 * e) = make_int4(tok, (int32_t)t0, (int32_t)nt, (int32_t)h);
        hstk[e] = (int32_t)st;
      }
    }
    // Task map: the wave writes each heavy lane's run of tasks together (one
    // lane at a time, its tasks spread over the lanes).
    for (unsigned long long rem = hv; rem; rem &= rem - 1) {
      const int l = __builtin_ctzll(rem);
      const uint32_t nl = (uint32_t)__builtin_amdgcn_readlane((int)nt, l);
      const uint32_t t0l = tb + (uint32_t)__builtin_amdgcn_readlane((int)tinc, l) - nl;
      const int32_t el = (int32_t)(hb + (uint32_t)__popcll(hv & ((1ull << l) - 1ull)));
      for (uint32_t c = (uint32_t)lane; c < nl; c += 64) tmapk[t0l + c] = el;
    }
    if (hv) tb += __shfl(tinc, 63, 64);
    hb += (uint32_t)__popcll(hv);
  }
  if (tid == 0) {
    a.counts[rk] = (int32_t)nseg;
    a.counts[EMB_RANGES + rk] = (int32_t)ntask;
    a.counts[2 * EMB_RANGES + rk] = (int32_t)nheavy;
  }
}

// The 16 ranges' counts of kind `kind` (0 segments, 1 tasks, 2 heavy
// entries): lane l < 16 gets range l's inclusive prefix; *total the sum.
VH_DEV uint32_t range_prefix(const int32_t* counts, int kind, uint32_t* total) {
  const int lane = threadIdx.x & 63;
  const uint32_t c = lane < EMB_RANGES ? (uint32_t)counts[kind * EMB_RANGES + lane] : 0u;
  const uint32_t inc = wave_incl_scan(c);
  *total = __shfl(inc, EMB_RANGES - 1, 64);
  return inc;
}
// The range holding global item x (0 <= x < total) and x's index within it.
VH_DEV int range_of(uint32_t inc, uint32_t x, uint32_t* local) {
  const int lane = threadIdx.x & 63;
  const int k = __popcll(__ballot(lane < EMB_RANGES && inc <= x));
  const uint32_t before = k > 0 ? __shfl(inc, k - 1, 64) : 0u;
  *local = x - before;
  return k;
}

// The sum, in order from 0.0, of cnt rows (at unit u) of the partial rows
// first, first + step, first + 2 step, ..., read with device-coherent loads,
// 8 rows in flight.
template <int VW>
VH_DEV Unit<VW> emb_coherent_sum(const float* partial, int64_t D, int64_t first, int64_t step, int32_t cnt, int u,
                                 int U) {
  Unit<VW> acc = zero_unit<VW>();
  for (int32_t c0 = 0; c0 < cnt; c0 += EMB_GROUP) {
    Unit<VW> d[EMB_GROUP];
#pragma unroll
    for (int r = 0; r < EMB_GROUP; ++r) {
      if (c0 + r < cnt && u < U) {
        const float* src = partial + (first + (int64_t)(c0 + r) * step) * D + u * VW;
#pragma unroll
        for (int j = 0; j < VW; ++j) d[r].v[j] = __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        d[r] = zero_unit<VW>();
      }
    }
#pragma unroll
    for (int r = 0; r < EMB_GROUP; ++r) {
      if (c0 + r < cnt) {
#pragma unroll
        for (int j = 0; j < VW; ++j) acc.v[j] += d[r].v[j];
      }
    }
  }
  return acc;
}

// Stores v at unit u of partial row `row` with device-coherent stores, then
// waits until they are done (every lane's), so a counter bumped after this
// by the wave tells another wave that the row can be read.
template <int VW>
VH_DEV void emb_coherent_store(float* partial, int64_t D, int64_t row, const Unit<VW>& v, int u, int U) {
  if (u < U) {
    float* dst = partial + row * D + u * VW;
#pragma unroll
    for (int j = 0; j < VW; ++j) __hip_atomic_store(dst + j, v.v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Bumps a device-scope counter once for the wave; returns its old value to
// every lane.
VH_DEV int32_t emb_count_done(int32_t* c) {
  int32_t old = 0;
  if ((threadIdx.x & 63) == 0) old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return old;
}

// Launch 2 of the sorted path: 256-thread workgroups, waves striding over the
// (heavy task, column slice) pairs (tasks numbered range by range), then the
// segments (light ones summed; heavy ones are skipped).
template <int VW>
VH_DEV void emb_sum_impl(const EmbSumArgs& a) {
  const int lane = threadIdx.x & 63;
  const int U = a.D / VW;
  uint32_t nseg, ntask;
  const uint32_t seg_inc = range_prefix(a.counts, 0, &nseg);
  const uint32_t task_inc = range_prefix(a.counts, 1, &ntask);
  // Heavy tasks first: the waves that start first take them, so the combine
  // of each heavy row's slices overlaps the light segments' stream.
  const int64_t nheavy_items = (int64_t)ntask * a.slices;
  const int64_t nitems = (int64_t)nseg + nheavy_items;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t it = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); it < nitems; it += nw) {
    if (it >= nheavy_items) {
      uint32_t s;
      const int k = range_of(seg_inc, (uint32_t)(it - nheavy_items), &s);
      // One load of the record: lanes 0-3 the header, 4 .. 4+hits the positions.
      const int32_t* rec = a.seg + ((size_t)k * a.n + s) * EMB_REC;
      const int32_t rv = lane < EMB_REC ? rec[lane] : 0;
      const int32_t tok = __shfl(rv, 0, 64), m = __shfl(rv, 2, 64);
      if (m > EMB_LIGHT) continue;
      const int32_t mypos = __shfl(rv, 4 + (lane < EMB_LIGHT ? lane : 0), 64);  // ascending
      float* o = a.dW + (int64_t)tok * a.D;
      for (int u0 = 0; u0 < U; u0 += 64 * EMB_Q) {
        Unit<VW> acc[EMB_Q];
#pragma unroll
        for (int q = 0; q < EMB_Q; ++q) acc[q] = zero_unit<VW>();
        for (int32_t kk = 0; kk < m; kk += 4) {
          const float* src[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) src[r] = a.dy + (int64_t)__shfl(mypos, kk + r < m ? kk + r : kk, 64) * a.D;
          emb_add_rows<VW, true>(acc, src, m - kk < 4 ? m - kk : 4, u0, lane, U);
        }
#pragma unroll
        for (int q = 0; q < EMB_Q; ++q) {
          const int u = u0 + lane + q * 64;
          if (u < U) store_stream<VW>(o + u * VW, acc[q]);
        }
      }
    } else {
      const int64_t item = it;
      const uint32_t t = (uint32_t)(item / a.slices);  // global task index
      const int u = (int)(item % a.slices) * 64 + lane;
      uint32_t lt;
      const int k = range_of(task_inc, t, &lt);
      const int32_t e = a.taskmap[(size_t)k * a.tmax + lt];
      const int4 hv = *reinterpret_cast<const int4*>(a.heavy + ((size_t)k * a.hmax + e) * 4);
      const int32_t r0 = ((int32_t)lt - hv.y) * EMB_CHUNK_HITS;
      const int32_t got = min(r0 + EMB_CHUNK_HITS, hv.w) - r0;
      const int32_t mypos = lane < got ? a.spos[(size_t)k * a.n + a.heavy_start[(size_t)k * a.hmax + e] + r0 + lane] : 0;
      Unit<VW> acc = zero_unit<VW>();
      for (int jj = 0; jj < got; jj += EMB_BATCH) {  // ascending positions, 16 rows per batch
        const float* src[EMB_BATCH];
#pragma unroll
        for (int r = 0; r < EMB_BATCH; ++r)
          src[r] = a.dy + (int64_t)__shfl(mypos, jj + r < got ? jj + r : jj, 64) * a.D;
        emb_add_slice<VW, true, EMB_BATCH>(acc, src, got - jj < EMB_BATCH ? got - jj : EMB_BATCH, u, U);
      }
      // A heavy row's slice is finished by the waves that end last, with no
      // further launch: partials go out with device-coherent stores (past this
      // XCD's L2) and each wave waits for its stores before it bumps a counter;
      // the wave that counts the last task of a group of EMB_GROUP tasks reads
      // the group's partials back with device-coherent loads and sums them in
      // task order (into the group's first partial row), and the wave that
      // counts a row's last group sums the group sums in group order into dW.
      // That is the device-scope release / acquire pair without the whole-L2
      // write-back and invalidate a fence performs, which these rows -- never
      // read by plain loads -- do not need. Same grouping, same bits as the
      // general path's final kernel.
      emb_coherent_store<VW>(a.partial, a.D, (int64_t)t, acc, u, U);
      const int sl = (int)(item % a.slices);
      const int32_t nch = hv.z, ngrp = (nch + EMB_GROUP - 1) / EMB_GROUP;
      const int32_t g = ((int32_t)lt - hv.y) / EMB_GROUP;
      const int32_t gsize = min(EMB_GROUP, nch - g * EMB_GROUP);
      int32_t* ck = a.ctr + (size_t)k * (a.hmax + a.tmax) * a.slices;
      if (emb_count_done(ck + ((size_t)a.hmax + hv.y + g * EMB_GROUP) * a.slices + sl) != gsize - 1) continue;
      const int64_t tg = (int64_t)t - ((int32_t)lt - hv.y - g * EMB_GROUP);  // the group's first task
      const Unit<VW> gs = emb_coherent_sum<VW>(a.partial, a.D, tg, 1, gsize, u, U);
      float* o = a.dW + (int64_t)hv.x * a.D + u * VW;
      if (ngrp == 1) {
        if (u < U) store_stream<VW>(o, gs);
        continue;
      }
      emb_coherent_store<VW>(a.partial, a.D, tg, gs, u, U);
      if (emb_count_done(ck + ((size_t)e * a.slices + sl)) != ngrp - 1) continue;
      const int64_t tb = (int64_t)t - ((int32_t)lt - hv.y);  // the row's first task
      const Unit<VW> gsum = emb_coherent_sum<VW>(a.partial, a.D, tb, EMB_GROUP, ngrp, u, U);
      if (u < U) store_stream<VW>(o, gsum);
    }
  }
}

