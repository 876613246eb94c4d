// gemm.h -- f32 matrix multiply on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Semantics: vearo-backend-cpu matmul (crates/vearo-backend-cpu/src/lib.rs:266-417),
// C[m, n] = sum_k A[m, k] * B[k, n] in f32 (the matrix core accumulates in f32;
// the grouping of the k sum differs from the CPU's sequential mul_add chain,
// which is within f32 rounding). The epilogue applies, in this order,
//   v = acc * alpha;  v = v + E[m, n] (optional addend);  v = C[m, n] + v (optional)
// which are exactly the separate ops the reference runs after a matmul:
// `* scale` and `+ mask` in attention (cpu:2431-2449), `+ bias` in Linear
// (nn:120-128), and gradient accumulation `existing.add(g)` (autograd:733-742).
//
// Tiling: a 256-thread workgroup computes a 128 x TN tile of C (TN = 128, or
// 64 for the attention products with N = Dk = 64); its 4 waves own 64 x TN/2
// quadrants as 2 x TN/64 matrix-core tiles of 32 x 32. K advances in
// tiles of 32, double-buffered through LDS: the global loads of tile t+1 are in
// flight while tile t is multiplied. LDS keeps each operand in the orientation
// of its HBM layout, so staging is 128-bit and bank-conflict free both ways:
// a k-contiguous operand as [row][k] (rows padded to 36 floats), read as 128-bit
// fragments; a row-contiguous one (a transposed view) as [k][row] (132 floats
// per k), read 32 bits at a time with consecutive lanes on consecutive rows.
// Lane half h (lanes 32h..32h+31) takes k in [16h, 16h+16) of the tile, step s
// pairing k = s with k = 16 + s.
// A operand layouts: k-contiguous (A[m, k] at m*lda + k) or m-contiguous
// (A[m, k] at k*lda + m, a transposed view); the same for B. Global loads are
// 128-bit when the layout allows (host-checked alignment), else 32-bit.
//
// Causal modes for attention's score blocks (the masked part is exactly 0 or
// never read, so skipping it changes no result):
//   1: skip tiles entirely above the diagonal (n > m for all elements);
//   2: only k <= m contributes (P V and dS K: row m's weights are 0 past m);
//   3: only k >= m contributes (P^T dO and dS^T Q).
#pragma once
#include "common.h"

#define GM_TM VH_GEMM_TILE_M
#define GM_TK 32
#define GM_LS (GM_TK + 4)  // [row][k] LDS row stride (floats): 16-byte aligned rows, staggered banks
#define GM_LT (GM_TM + 4)  // [k][row] LDS stride (floats)
#define GM_STAGE (GM_TM * GM_LS > GM_TK * GM_LT ? GM_TM * GM_LS : GM_TK * GM_LT)  // one 128-row operand tile
#define GM_GROUP 8         // tile rows per group in the launch order (L2 reuse of B)

typedef float vh_f32x16 __attribute__((ext_vector_type(16)));

template <bool B>
struct GmFlag {
  static constexpr bool value = B;
};

// The [NR rows x 32 k] tile (NR = 128 or 64) whose element (r, k) is at
//   KC:  base[(r0 + r) * ld + k0 + k]      !KC: base[(k0 + k) * ld + r0 + r]
// into NR/8 staging registers per thread; rows >= R or k >= K read as 0.
// VEC requires 16-byte aligned base and ld, and K (KC) or R (!KC) % 4 == 0.
// CHECK = false: the caller knows the whole tile is inside (no tests, no
// branches: the loads can be scheduled among the matrix-core products).
template <bool KC, bool VEC, int NR, bool CHECK = true>
VH_DEV void gm_load(const float* base, int64_t ld, int64_t r0, int64_t R, int64_t k0, int64_t K, int tid,
                    float (&st)[NR / 8]) {
  if constexpr (KC && VEC) {
#pragma unroll
    for (int i = 0; i < NR / 32; ++i) {
      const int r = (tid >> 3) + 32 * i, k = (tid & 7) * 4;
      vh_f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (!CHECK || (r0 + r < R && k0 + k < K)) v = *reinterpret_cast<const vh_f4*>(base + (r0 + r) * ld + k0 + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) st[4 * i + e] = v[e];
    }
  } else if constexpr (KC) {
#pragma unroll
    for (int i = 0; i < NR / 8; ++i) {
      const int r = (tid >> 5) + 8 * i, k = tid & 31;
      st[i] = (!CHECK || (r0 + r < R && k0 + k < K)) ? base[(r0 + r) * ld + k0 + k] : 0.0f;
    }
  } else if constexpr (VEC) {
    constexpr int TPR = NR / 4;  // threads per k row
#pragma unroll
    for (int i = 0; i < NR / 32; ++i) {
      const int k = tid / TPR + (256 / TPR) * i, r = (tid % TPR) * 4;
      vh_f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (!CHECK || (k0 + k < K && r0 + r < R)) v = *reinterpret_cast<const vh_f4*>(base + (k0 + k) * ld + r0 + r);
#pragma unroll
      for (int e = 0; e < 4; ++e) st[4 * i + e] = v[e];
    }
  } else {
#pragma unroll
    for (int i = 0; i < NR / 8; ++i) {
      const int k = tid / NR + (256 / NR) * i, r = tid % NR;
      st[i] = (!CHECK || (k0 + k < K && r0 + r < R)) ? base[(k0 + k) * ld + r0 + r] : 0.0f;
    }
  }
}

template <bool KC, bool VEC, int NR>
VH_DEV void gm_store_lds(float* S, int tid, const float (&st)[NR / 8]) {
  if constexpr (KC && VEC) {
#pragma unroll
    for (int i = 0; i < NR / 32; ++i) {
      const int r = (tid >> 3) + 32 * i, k = (tid & 7) * 4;
      vh_f4 v = {st[4 * i], st[4 * i + 1], st[4 * i + 2], st[4 * i + 3]};
      *reinterpret_cast<vh_f4*>(S + r * GM_LS + k) = v;
    }
  } else if constexpr (KC) {
#pragma unroll
    for (int i = 0; i < NR / 8; ++i) S[((tid >> 5) + 8 * i) * GM_LS + (tid & 31)] = st[i];
  } else if constexpr (VEC) {
    constexpr int TPR = NR / 4;
#pragma unroll
    for (int i = 0; i < NR / 32; ++i) {
      const int k = tid / TPR + (256 / TPR) * i, r = (tid % TPR) * 4;
      vh_f4 v = {st[4 * i], st[4 * i + 1], st[4 * i + 2], st[4 * i + 3]};
      *reinterpret_cast<vh_f4*>(S + k * GM_LT + r) = v;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NR / 8; ++i) S[(tid / NR + (256 / NR) * i) * GM_LT + tid % NR] = st[i];
  }
}

// Fragment of row `row` for k = k0 .. k0+3 (4 matrix-core steps).
template <bool KC>
VH_DEV vh_f4 gm_frag(const float* S, int row, int k0) {
  if constexpr (KC) {
    return *reinterpret_cast<const vh_f4*>(S + row * GM_LS + k0);
  } else {
    vh_f4 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = S[(k0 + e) * GM_LT + row];
    return f;
  }
}

// Workgroup -> C tile. Workgroups are dealt to the 8 XCDs round-robin; this
// gives each XCD a contiguous run of tile ids, and runs of GM_GROUP tile rows
// sweep the tile columns together, so an XCD's L2 sees the same B columns
// and A rows reused.
VH_DEV void gm_tile_of(int bid, int nblk, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per = nblk / 8, rem = nblk % 8;
  const int x = bid % 8, local = bid / 8;
  const int t = x * per + (x < rem ? x : rem) + local;
  const int span = GM_GROUP * tiles_n;
  const int first = (t / span) * GM_GROUP;
  const int gsize = tiles_m - first < GM_GROUP ? tiles_m - first : GM_GROUP;
  const int in = t % span;
  tm = first + in % gsize;
  tn = in / gsize;
}

// The launch's causal mode: a.causal, unless a device flag says the product is dense.
VH_DEV int gm_causal(const GemmArgs& a) { return (a.causal_flag && *a.causal_flag == 0) ? 0 : a.causal; }
// The addend: under a device flag that says causal, E is the attention's mask,
// whose allowed entries are +-0 and whose masked ones the causal form skips, so
// it is not added (as a caller passing causal = 1 drops it).
VH_DEV const float* gm_addend(const GemmArgs& a) {
  return (a.causal_flag && *a.causal_flag != 0) ? nullptr : a.E;
}

// The epilogue of one output element from its product sum v: the raw partial
// under split-K (raw), else alpha v (+ E[m, n]) (+ old = out[m, n]).
VH_DEV float gm_finish(const GemmArgs& a, const float* E, bool raw, float v, int64_t m, int64_t n, float old) {
  if (raw) return v;
  v = v * a.alpha;
  if (E) v = v + E[m * a.sem + n * a.sen];
  if (a.accumulate) v = old + v;
  return v;
}

// A wave's 64 x TN/2 quadrant of the tile at (m0, n0) straight from its
// accumulators: register r of a 32 x 32 tile holds row 8*(r/4) + 4*h + r%4,
// column li; elements outside M x N are dropped. NT: streaming (nontemporal)
// stores, which do not allocate the written lines in L2.
template <int NTW, bool NT = false>
VH_DEV void gm_store_direct(const GemmArgs& a, const vh_f32x16 (&acc)[2][NTW], float* out, int64_t ldo,
                            const float* E, bool raw, int64_t m0, int64_t n0, int wm, int wn, int li, int h) {
  if (m0 + GM_TM <= a.M && n0 + NTW * 64 <= a.N && !E && (raw || !a.accumulate)) {
    // A whole tile that reads nothing back: the stores go out back to back
    // (a conditional load of C among them makes each wait for all earlier
    // stores, as the memory counter covers both).
    const float alpha = raw ? 1.0f : a.alpha;
    float* base = out + (m0 + wm * 64 + 4 * h) * ldo + n0 + wn * (NTW * 32) + li;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float* cp = base + (mt * 32 + 8 * (r >> 2) + (r & 3)) * ldo + nt * 32;
          const float v = raw ? acc[mt][nt][r] : acc[mt][nt][r] * alpha;
          if constexpr (NT)
            __builtin_nontemporal_store(v, cp);
          else
            *cp = v;
        }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int64_t n = n0 + wn * (NTW * 32) + nt * 32 + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 64 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < a.M && n < a.N) {
          float* cp = out + m * ldo + n;
          const float v = gm_finish(a, E, raw, acc[mt][nt][r], m, n, a.accumulate && !raw ? *cp : 0.0f);
          if constexpr (NT)
            __builtin_nontemporal_store(v, cp);
          else
            *cp = v;
        }
      }
    }
  }
}

template <bool A_KC, bool A_VEC, bool B_KC, bool B_VEC, int TN>
VH_DEV void gemm_f32_impl(const GemmArgs& a) {
  static_assert(TN == 128 || TN == 64, "C tile width");
  constexpr int NTW = TN / 64;  // 32-wide n tiles per wave
  // L[0..1]: A's two k stages, L[2..3]: B's; after the k loop, the C tile.
  __shared__ __attribute__((aligned(16))) float L[4][GM_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int tm, tn;
  int64_t bat = blockIdx.y;  // batch index (both batch dims)
  const int causal = gm_causal(a);
  if (causal >= 2 && a.ksplit <= 1) {
    // The k range grows with the tile row (k <= m) or shrinks (k >= m): deal
    // the workgroups longest first across all batches, so the last ones to
    // start are short (the launch order is x fastest, then y).
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t rank = lin / gridDim.y;
    bat = lin % gridDim.y;
    const int row = (int)(rank / a.tiles_n);
    tm = causal == 2 ? a.tiles_m - 1 - row : row;
    tn = (int)(rank % a.tiles_n);
  } else {
    gm_tile_of(blockIdx.x, gridDim.x, a.tiles_m, a.tiles_n, tm, tn);
  }
  const int64_t m0 = (int64_t)tm * GM_TM, n0 = (int64_t)tn * TN;
  if (causal == 1 && n0 > m0 + GM_TM - 1) return;  // the whole tile is masked

  const bool split = a.ksplit > 1;
  const int64_t b1 = split ? 0 : bat / a.nb2, b2 = split ? 0 : bat % a.nb2;
  const float* A = a.A + b1 * a.sa1 + b2 * a.sa2;
  const float* B = a.B + b1 * a.sb1 + b2 * a.sb2;
  float* C = a.C + b1 * a.sc1 + b2 * a.sc2;

  int64_t kb = 0, ke = a.K;
  if (causal == 2) ke = m0 + GM_TM < a.K ? m0 + GM_TM : a.K;
  if (causal == 3) kb = (m0 / GM_TK) * GM_TK;
  if (split) {
    kb = (int64_t)blockIdx.y * a.kchunk;
    ke = kb + a.kchunk < a.K ? kb + a.kchunk : a.K;
  }

  vh_f32x16 acc[2][NTW];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[i][j] = vh_f32x16{};

  const int wm = w >> 1, wn = w & 1, li = lane & 31, h = lane >> 5;
  float sa[GM_TM / 8], sb[TN / 8];
  int s = 0;
  if (kb < ke) {
    gm_load<A_KC, A_VEC, GM_TM>(A, a.lda, m0, a.M, kb, a.K, tid, sa);
    gm_load<B_KC, B_VEC, TN>(B, a.ldb, n0, a.N, kb, a.K, tid, sb);
    gm_store_lds<A_KC, A_VEC, GM_TM>(L[0], tid, sa);
    gm_store_lds<B_KC, B_VEC, TN>(L[2], tid, sb);
    __syncthreads();
  }
  // Per k tile: the next tile's global loads go out; then all of this tile's
  // fragments are read from LDS at once (the products wait only on the reads
  // they use, which return in order); the next tile is written to the other
  // LDS buffer (free since the last barrier) between the last group's
  // products. On the last tile that write goes to a buffer nothing reads again
  // (the loop body stays one block, so the order below holds).
  // A tile entirely inside A, B and K (all but the edge tiles) runs a copy of
  // the loop without bounds tests or branches around its loads; on the last
  // k tile they fetch that tile again rather than branch.
  constexpr int RD = 4 * ((A_KC ? 2 : 8) + NTW * (B_KC ? 1 : 4));              // LDS reads per tile
  constexpr int WR = (A_VEC ? GM_TM / 32 : GM_TM / 8) + (B_VEC ? TN / 32 : TN / 8);  // LDS writes per tile
  constexpr int VM = (A_VEC ? GM_TM / 32 : GM_TM / 8) + (B_VEC ? TN / 32 : TN / 8);  // global loads per tile
  constexpr int MF = 8 * NTW;                                                   // products per 4-k group
  // One k step on the k tile staged in stage sc: the loads of k tile kl go
  // out into (la, lb), this tile's products run, and (wa, wb) -- the k tile
  // that follows this one -- are staged into the other LDS buffers.
  auto kstep = [&](auto unchecked, int sc, float (&la)[GM_TM / 8], float (&lb)[TN / 8],
                   const float (&wa)[GM_TM / 8], const float (&wb)[TN / 8], int64_t kl, bool load) {
    constexpr bool CHECK = !decltype(unchecked)::value;
    if constexpr (CHECK) {
      if (load) {
        gm_load<A_KC, A_VEC, GM_TM>(A, a.lda, m0, a.M, kl, a.K, tid, la);
        gm_load<B_KC, B_VEC, TN>(B, a.ldb, n0, a.N, kl, a.K, tid, lb);
      }
    } else {
      gm_load<A_KC, A_VEC, GM_TM, false>(A, a.lda, m0, a.M, kl, a.K, tid, la);
      gm_load<B_KC, B_VEC, TN, false>(B, a.ldb, n0, a.N, kl, a.K, tid, lb);
    }
    vh_f4 fa[4][2], fb[4][NTW];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kc = h * 16 + 4 * q;
      fa[q][0] = gm_frag<A_KC>(L[sc], wm * 64 + li, kc);
      fa[q][1] = gm_frag<A_KC>(L[sc], wm * 64 + 32 + li, kc);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) fb[q][nt] = gm_frag<B_KC>(L[2 + sc], wn * (TN / 2) + nt * 32 + li, kc);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          acc[0][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q][0][e], fb[q][nt][e], acc[0][nt], 0, 0, 0);
          acc[1][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q][1][e], fb[q][nt][e], acc[1][nt], 0, 0, 0);
        }
      }
    }
    gm_store_lds<A_KC, A_VEC, GM_TM>(L[sc ^ 1], tid, wa);
    gm_store_lds<B_KC, B_VEC, TN>(L[2 + (sc ^ 1)], tid, wb);
    if constexpr (!CHECK) __builtin_amdgcn_sched_group_barrier(0x020, VM, 0);  // the loads
    __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);                        // all fragment reads
    __builtin_amdgcn_sched_group_barrier(0x008, 3 * MF, 0);                    // groups 0-2
#pragma unroll
    for (int i = 0; i < MF; ++i) {  // group 3 with the writes
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, (WR + MF - 1) / MF, 0);
    }
    __syncthreads();
  };
  // 128 x 128 tiles: the next k tile's loads are in flight during one step
  // (1.7 us of products). 128 x 64 tiles have half the products per step, less
  // than the load latency under load, so with 128-bit loads (registers to
  // spare) theirs run two steps ahead through a second register set: step 0
  // of a pair computes stage 0, loads k tile k0+64 into (sa, sb) and stages
  // (sa2, sb2) = k0+32; step 1 the reverse. Unchecked loads past the range
  // fetch the last k tile again.
  constexpr bool DEEP = TN == 64 && A_VEC && B_VEC;
  auto main_loop = [&](auto unchecked) {
    constexpr bool CHECK = !decltype(unchecked)::value;
    auto kn = [&](int64_t k) { return CHECK || k < ke ? k : ke - GM_TK; };
    if constexpr (!DEEP) {
      for (int64_t k0 = kb; k0 < ke; k0 += GM_TK) {
        kstep(unchecked, s, sa, sb, sa, sb, kn(k0 + GM_TK), k0 + GM_TK < ke);
        s ^= 1;
      }
    } else {
      float sa2[GM_TM / 8] = {}, sb2[TN / 8] = {};
      if (kb < ke) {
        if constexpr (CHECK) {
          if (kb + GM_TK < ke) {
            gm_load<A_KC, A_VEC, GM_TM>(A, a.lda, m0, a.M, kb + GM_TK, a.K, tid, sa2);
            gm_load<B_KC, B_VEC, TN>(B, a.ldb, n0, a.N, kb + GM_TK, a.K, tid, sb2);
          }
        } else {
          gm_load<A_KC, A_VEC, GM_TM, false>(A, a.lda, m0, a.M, kn(kb + GM_TK), a.K, tid, sa2);
          gm_load<B_KC, B_VEC, TN, false>(B, a.ldb, n0, a.N, kn(kb + GM_TK), a.K, tid, sb2);
        }
      }
      for (int64_t k0 = kb; k0 < ke; k0 += 2 * GM_TK) {
        kstep(unchecked, 0, sa, sb, sa2, sb2, kn(k0 + 2 * GM_TK), k0 + 2 * GM_TK < ke);
        if (k0 + GM_TK >= ke) break;
        kstep(unchecked, 1, sa2, sb2, sa, sb, kn(k0 + 3 * GM_TK), k0 + 3 * GM_TK < ke);
      }
    }
  };
  const bool inside = m0 + GM_TM <= a.M && n0 + TN <= a.N && (ke - kb) % GM_TK == 0 && ke <= a.K;
  if (inside)
    main_loop(GmFlag<true>{});
  else
    main_loop(GmFlag<false>{});

  // Epilogue. Straight from the accumulators, one wave store covers two
  // 128-byte row pieces; a tile wholly inside C with 16-byte aligned rows goes
  // through LDS instead (the k loop's last barrier has freed it), so that each
  // store writes 16 bytes and a half-wave a whole 512-byte row.
  float* out = split ? a.ws + (int64_t)blockIdx.y * a.M * a.N : C;
  const int64_t ldo = split ? a.N : a.ldc;
  const float* E0 = gm_addend(a);
  const float* E = !split && E0 ? E0 + b1 * a.se1 + b2 * a.se2 : nullptr;
  const bool whole = m0 + GM_TM <= a.M && n0 + TN <= a.N && (ldo & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (whole) {
    constexpr int CS = TN + 8;  // row stride (floats): rows 4 apart are 32 banks apart
    static_assert(GM_TM * CS <= 4 * GM_STAGE, "C tile fits the operand LDS");
    float* Cs = &L[0][0];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          Cs[(wm * 64 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) * CS + wn * (TN / 2) + nt * 32 + li] =
              acc[mt][nt][r];
    __syncthreads();
    constexpr int Q = TN / 4;      // 16-byte pieces per row
    constexpr int RP = 256 / Q;    // rows per pass
    const int c = (tid % Q) * 4, r0 = tid / Q;
#pragma unroll 4
    for (int i = 0; i < GM_TM / RP; ++i) {
      const int row = r0 + RP * i;
      const int64_t m = m0 + row, n = n0 + c;
      vh_f4 v = *reinterpret_cast<const vh_f4*>(Cs + row * CS + c);
      vh_f4* op = reinterpret_cast<vh_f4*>(out + m * ldo + n);
      if (!split) {
        const vh_f4 old = a.accumulate ? *op : vh_f4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gm_finish(a, E, false, v[e], m, n + e, old[e]);
      }
      *op = v;
    }
    return;
  }
  gm_store_direct<NTW>(a, acc, out, ldo, E, split, m0, n0, wm, wn, li, h);
}

// Persistent form for batched products with a short k range (attention's
// scores q k^T and dP = dO v^T: K = Dk = 64, 2 k tiles per C tile). Launched
// as one workgroup per resident slot (a multiple of 8), each walks a list of
// C tiles as one continuous k loop: the last k step of a tile loads the
// first k tile of the next one, so its global loads are in flight under the
// current tile's products and epilogue instead of exposed at the start of a
// short-lived workgroup. Work items are the live tiles of every batch, batch
// major (causal 1: the tiles with tn <= tm, which with tiles_n >= tiles_m are
// T (T + 1) / 2 for T = tiles_m); XCD x (= workgroup id % 8, the hardware's
// round-robin) takes the x-th contiguous eighth of the items, so one XCD works
// on one or two batches at a time and its L2 holds their operands. Tile width
// 128; no split, causal 0 or 1 only (the host guarantees both).
template <bool A_KC, bool A_VEC, bool B_KC, bool B_VEC>
VH_DEV void gemm_f32_persist(const GemmArgs& a) {
  constexpr int TN = 128, NTW = 2;
  __shared__ __attribute__((aligned(16))) float L[4][GM_STAGE];  // A stages 0-1, B stages 2-3
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1, li = lane & 31, h = lane >> 5;
  const int causal = gm_causal(a);
  const float* E0 = gm_addend(a);
  const int64_t live = causal == 1 ? (int64_t)a.tiles_m * (a.tiles_m + 1) / 2 : (int64_t)a.tiles_m * a.tiles_n;
  const int64_t total = live * a.nbat;
  const int nloc = (int)(gridDim.x / 8), x = (int)(blockIdx.x % 8);
  const int64_t per = (total + 7) / 8;
  const int64_t end = (x + 1) * per < total ? (x + 1) * per : total;
  int64_t item = x * per + (int64_t)(blockIdx.x / 8);
  if (item >= end) return;

  struct Tile {
    const float* A;
    const float* B;
    float* C;
    const float* E;
    int64_t m0, n0;
    bool inside;  // the whole tile and its k range are inside A, B and C
  };
  auto decode = [&](int64_t it, Tile& t) {
    const int64_t bat = it / live;
    const int64_t u = it % live;
    int64_t tm, tn;
    if (causal == 1) {  // u = tm (tm + 1) / 2 + tn, tn <= tm
      tm = (int64_t)((sqrtf(8.0f * (float)u + 1.0f) - 1.0f) * 0.5f);
      while (tm * (tm + 1) / 2 > u) --tm;
      while ((tm + 1) * (tm + 2) / 2 <= u) ++tm;
      tn = u - tm * (tm + 1) / 2;
    } else {
      tm = u / a.tiles_n;
      tn = u % a.tiles_n;
    }
    const int64_t b1 = bat / a.nb2, b2 = bat % a.nb2;
    t.A = a.A + b1 * a.sa1 + b2 * a.sa2;
    t.B = a.B + b1 * a.sb1 + b2 * a.sb2;
    t.C = a.C + b1 * a.sc1 + b2 * a.sc2;
    t.E = E0 ? E0 + b1 * a.se1 + b2 * a.se2 : nullptr;
    t.m0 = tm * GM_TM;
    t.n0 = tn * TN;
    t.inside = t.m0 + GM_TM <= a.M && t.n0 + TN <= a.N && a.K % GM_TK == 0;
  };

  Tile cur, nxt;
  decode(item, cur);
  float sa[GM_TM / 8], sb[TN / 8];
  gm_load<A_KC, A_VEC, GM_TM>(cur.A, a.lda, cur.m0, a.M, 0, a.K, tid, sa);
  gm_load<B_KC, B_VEC, TN>(cur.B, a.ldb, cur.n0, a.N, 0, a.K, tid, sb);
  gm_store_lds<A_KC, A_VEC, GM_TM>(L[0], tid, sa);
  gm_store_lds<B_KC, B_VEC, TN>(L[2], tid, sb);
  __syncthreads();
  int s = 0;

  constexpr int RD = 4 * ((A_KC ? 2 : 8) + NTW * (B_KC ? 1 : 4));
  constexpr int WR = (A_VEC ? GM_TM / 32 : GM_TM / 8) + (B_VEC ? TN / 32 : TN / 8);
  constexpr int VM = WR;
  constexpr int MF = 8 * NTW;
  for (;;) {
    const int64_t nit = item + nloc;
    const bool has_next = nit < end;
    if (has_next)
      decode(nit, nxt);
    else
      nxt = cur;
    vh_f32x16 acc[2][NTW];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NTW; ++j) acc[i][j] = vh_f32x16{};
    // One k step: the next stage (this tile's next k tile, else the next
    // tile's first, else this one's last again) is loaded, this stage is
    // multiplied, and the loaded one is staged into the other LDS buffer.
    auto k_loop = [&](auto unchecked) {
      constexpr bool CHECK = !decltype(unchecked)::value;
      for (int64_t k0 = 0; k0 < a.K; k0 += GM_TK) {
        const bool more = k0 + GM_TK < a.K;
        const float* An = more ? cur.A : nxt.A;
        const float* Bn = more ? cur.B : nxt.B;
        const int64_t mn = more ? cur.m0 : nxt.m0, nn = more ? cur.n0 : nxt.n0;
        const int64_t kn = more ? k0 + GM_TK : (has_next ? 0 : k0);
        if constexpr (CHECK) {
          if (more || has_next) {
            gm_load<A_KC, A_VEC, GM_TM>(An, a.lda, mn, a.M, kn, a.K, tid, sa);
            gm_load<B_KC, B_VEC, TN>(Bn, a.ldb, nn, a.N, kn, a.K, tid, sb);
          }
        } else {
          gm_load<A_KC, A_VEC, GM_TM, false>(An, a.lda, mn, a.M, kn, a.K, tid, sa);
          gm_load<B_KC, B_VEC, TN, false>(Bn, a.ldb, nn, a.N, kn, a.K, tid, sb);
        }
        vh_f4 fa[4][2], fb[4][NTW];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int kc = h * 16 + 4 * q;
          fa[q][0] = gm_frag<A_KC>(L[s], wm * 64 + li, kc);
          fa[q][1] = gm_frag<A_KC>(L[s], wm * 64 + 32 + li, kc);
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) fb[q][nt] = gm_frag<B_KC>(L[2 + s], wn * (TN / 2) + nt * 32 + li, kc);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
              acc[0][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q][0][e], fb[q][nt][e], acc[0][nt], 0, 0, 0);
              acc[1][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q][1][e], fb[q][nt][e], acc[1][nt], 0, 0, 0);
            }
          }
        }
        gm_store_lds<A_KC, A_VEC, GM_TM>(L[s ^ 1], tid, sa);
        gm_store_lds<B_KC, B_VEC, TN>(L[2 + (s ^ 1)], tid, sb);
        if constexpr (!CHECK) __builtin_amdgcn_sched_group_barrier(0x020, VM, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 3 * MF, 0);
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, (WR + MF - 1) / MF, 0);
        }
        __syncthreads();
        s ^= 1;
      }
    };
    if (cur.inside && nxt.inside)
      k_loop(GmFlag<true>{});
    else
      k_loop(GmFlag<false>{});
    // Streaming stores: with normal ones the write of a score-sized output
    // runs at ~1.8 TB/s here, with these at ~2.8 TB/s (measured).
    gm_store_direct<NTW, true>(a, acc, cur.C, a.ldc, cur.E, false, cur.m0, cur.n0, wm, wn, li, h);
    if (!has_next) break;
    item = nit;
    cur = nxt;
  }
}

// C[m, n] = epilogue(sum over y of ws[y][m][n], y ascending): the split-K
// partials in a fixed order, so the result does not depend on timing.
VH_DEV void gemm_reduce_impl(const GemmReduceArgs& a) {
  const int64_t total = a.M * a.N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t m = i / a.N, n = i % a.N;
    float s = a.ws[i];
    for (int y = 1; y < a.ksplit; ++y) s += a.ws[(int64_t)y * total + i];
    float v = s * a.alpha;
    if (a.E) v = v + a.E[m * a.sem + n * a.sen];
    float* cp = a.C + m * a.ldc + n;
    if (a.accumulate) v = *cp + v;
    *cp = v;
  }
}
