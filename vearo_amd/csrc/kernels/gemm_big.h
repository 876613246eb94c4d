// gemm_big.h -- f32 matrix multiply for the large dense products (the lm_head
// and Linear layers of the GPT block step) on the gfx950 matrix cores.
//
// Same semantics and epilogue as gemm.h (C = alpha A B (+ E) (+ C), each
// operand k-contiguous or row-contiguous), for unbatched, non-causal products
// whose operands allow 128-bit loads and 32-bit tile offsets, and whose
// k-contiguous operands have K % 32 == 0 (the host checks; it runs a ragged
// k tail as a second, accumulating product, and everything else on gemm.h).
//
// One 512-thread workgroup per CU, persistent: the grid is the CU count G
// and each workgroup walks a list of (C tile, k range) segments as one
// continuous stream of k tiles, so the loads of its next segment overlap the
// current one's products.
//   * Whole-tile rounds: while at least G tiles remain, workgroup g takes one
//     whole tile per round. Round r covers tiles [rG, rG + G); XCD x (=
//     g mod 8, the hardware's round-robin) takes G/8 consecutive ones, which
//     the tile order maps to a block of tile rows x tile columns, so the
//     XCD's L2 serves each A and B panel to several workgroups.
//   * Last round (stream-K): the rem = tiles mod G tiles left over have rem *
//     nk k tiles in all; workgroup g takes the contiguous run [g W / G,
//     (g + 1) W / G) of them (tile-major), so every CU stays busy to the end.
//     A run that covers a whole tile stores it directly; a partial piece goes
//     to a workspace slot, and gemm_big_fix sums a split tile's pieces in k
//     order (fixed, so results do not depend on timing) and applies the
//     epilogue.
//
// Tile: 256 x BN (BN = 192 or 256). NW = 8 waves, two per SIMD, own 64 x BN/2
// blocks (a 4 x 2 grid) as 2 x BN/64 matrix-core tiles of 32 x 32
// (v_mfma_f32_32x32x2_f32). At two waves per SIMD each wave has 256 registers
// of the unified register file; the compiler keeps the accumulators in
// ordinary VGPRs beside the fragments and addresses (the code object reports
// 256 VGPRs and no accumulation registers). While one wave of a SIMD waits on
// LDS or the barrier, the other's products keep the matrix core busy. (NW = 4, one wave per SIMD owning 128 x BN/2,
// measured on MI355X at [16384 x 768] x [768 x 50260] and the lm_head
// gradients: 0.87-0.88 of the f32 matrix peak against 0.90-0.93 for NW = 8,
// which also fits its registers without spilling and needs no software
// prefetch of far-apart k-contiguous rows.)
//
// K advances in tiles of 32 through two LDS stages and one set of staging
// registers: the k step on k tile p first writes tile p + 1 (loaded during
// the previous step) from the registers to the free stage, then reloads the
// registers with tile p + 2, then multiplies tile p -- so each load has a
// whole step to arrive, and the barrier ending the step waits only for LDS.
// Loads are buffer loads whose record count is the bytes from the tile
// origin to the operand's last element, so reads past the operand return
// zero without touching memory; rows past M (columns past N) of a tile read
// zeros or the next k row's values, which reach only outputs that are never
// stored, and k past K (row-contiguous operands only, see above) reads zeros.
// The k loop has no bounds tests. Products of step (q, e) (q, e = 0..3) take
// k = 8q + 4h + e from lane half h.
// LDS layouts:
//   k-contiguous: [row][32 k] as 128-byte rows whose eight 16-byte k slots are
//     XOR-permuted by swz(r) = (r & 7) ^ ((r >> 3) & 1), so that 128-bit
//     accesses of 16 consecutive rows at one k (fragment reads) or of two rows
//     (the staging writes) hit distinct bank groups;
//   row-contiguous: [k][row], padded to NR + 8 floats so the two lane halves'
//     32-bit fragment reads (4 k apart) sit 32 banks apart.
#pragma once
#include <type_traits>

#include "common.h"
#include "gemm.h"

#define GB_TM VH_GEMMB_TM
#define GB_TK 32
#define GB_GROUP 8             // tile rows per group in the tile order
#define GB_RSRC_W3 0x00020000  // buffer resource word 3: 32-bit data, raw (no swizzle, no stride)

template <bool KC, int NR, int NT = 256>
struct GbOp {
  static constexpr int LT = NR + 8;                           // [k][row] stride (floats)
  static constexpr int STAGE = KC ? NR * GB_TK : GB_TK * LT;  // floats per LDS stage
  static constexpr int PER = NR * 8 / NT;                     // 128-bit pieces per thread per k tile
};

VH_DEV int gb_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Piece i of thread tid in an [NR rows x 32 k] tile: row r, k offset k; 4
// consecutive k (k-contiguous) or rows (row-contiguous) per piece, so eight
// (or NR / 4) threads cover one 128-byte row (or k row) of the operand.
template <bool KC, int NR, int NT = 256>
VH_DEV void gb_piece(int tid, int i, int& r, int& k) {
  const int f = tid + NT * i;
  r = KC ? f >> 3 : (f % (NR / 4)) * 4;
  k = KC ? (f & 7) * 4 : f / (NR / 4);
}
// The piece's byte offset from the tile origin in the operand.
template <bool KC, int NR, int NT = 256>
VH_DEV uint32_t gb_goff(int64_t ld, int tid, int i) {
  int r, k;
  gb_piece<KC, NR, NT>(tid, i, r, k);
  return (uint32_t)((KC ? r * ld + k : k * ld + r) * 4);
}
// The piece's float index in an LDS stage.
template <bool KC, int NR, int NT = 256>
VH_DEV int gb_loff(int tid, int i) {
  int r, k;
  gb_piece<KC, NR, NT>(tid, i, r, k);
  return KC ? r * GB_TK + (((k >> 2) ^ gb_swz(r)) << 2) : k * GbOp<KC, NR>::LT + r;
}

// Buffer resource for the tile whose origin is `org`, covering `bytes` bytes
// (clamped to 32 bits: the host guarantees a tile's reads fit below that).
// The record count: bytes clamped to [0, 2^32 - 1], from the two 32-bit halves
// (scalar compares only; a 64-bit compare needs a vector register, whose
// write the compiler fences with a wait for every outstanding load).
VH_DEV __amdgpu_buffer_rsrc_t gb_rsrc(const float* org, int64_t bytes) {
  const uint64_t u = (uint64_t)bytes;
  const uint32_t hi = (uint32_t)(u >> 32), lo = (uint32_t)u;
  const uint32_t nrec = (hi & 0x80000000u) ? 0u : (hi ? 0xFFFFFFFFu : lo);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(org), (short)0, (int)nrec, GB_RSRC_W3);
}

// Tile order index u -> (tm, tn): groups of GB_GROUP tile rows swept column
// by column, so consecutive indices form a block of rows x columns.
VH_DEV void gb_tile_of(int u, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int span = GB_GROUP * tiles_n;
  const int grp = u / span;
  const int first = grp * GB_GROUP;
  const int gsize = tiles_m - first < GB_GROUP ? tiles_m - first : GB_GROUP;
  const int in = u - grp * span;
  tn = in / gsize;
  tm = first + (in - tn * gsize);
}

// The work split shared by the kernel and the fix-up: G workgroups, `full`
// whole-tile rounds, then W = rem * nk k tiles split evenly (the host keeps
// tile and k tile counts, and W, below 2^31).
struct GbSplit {
  int tiles, nk, full, rem, W, G;
  VH_DEV GbSplit(const GemmArgs& a, int G_) : G(G_) {
    tiles = a.tiles_m * a.tiles_n * (int)a.nbat;  // tiles of all batches (the host keeps it < 2^31)
    nk = (int)((a.K + GB_TK - 1) / GB_TK);
    full = tiles / G;
    rem = tiles - full * G;
    W = rem * nk;
  }
  VH_DEV int begin(int g) const { return (int)((int64_t)W * g / G); }
  VH_DEV int end(int g) const { return (int)((int64_t)W * (g + 1) / G); }
};

// One segment of a workgroup's list: C tile (m0, n0) of one batch, k tiles
// [kt0, kt1), and that batch's element offsets into A, B, C and E.
struct GbSeg {
  int m0, n0, kt0, kt1;
  int slot;  // -1: store C; else the workspace slot this partial piece goes to
  int64_t ao, bo, co, eo;
};

// Tile u of the whole list -> batch (tile-major within a batch), its (tm, tn)
// and the batch's offsets (batch = outer * nb2 + inner, each with its stride).
VH_DEV void gb_locate(const GemmArgs& a, int u, int& tm, int& tn, GbSeg& s) {
  const int tpb = a.tiles_m * a.tiles_n;
  const int bat = u / tpb;
  gb_tile_of(u - bat * tpb, a.tiles_m, a.tiles_n, tm, tn);
  const int b1 = bat / a.nb2, b2 = bat - b1 * a.nb2;
  s.ao = b1 * a.sa1 + b2 * a.sa2;
  s.bo = b1 * a.sb1 + b2 * a.sb2;
  s.co = b1 * a.sc1 + b2 * a.sc2;
  s.eo = b1 * a.se1 + b2 * a.se2;
}
#define GB_SLOTS VH_GEMMB_SLOTS  // workspace slots per workgroup: stream-K first / last piece

// Operands need only 4-byte alignment: a 128-bit buffer load at a 4-byte-aligned
// offset returns the four floats there, and the record-count check applies to
// each of its dwords on its own (a load straddling the record's end returns
// the in-range dwords and zeros; measured on MI355X), so a leading dimension
// like 50257 floats or a base one float into an allocation takes the same
// loads as an aligned operand.
template <bool A_KC, bool B_KC, int BN, int NW = 8>
VH_DEV void gemm_big_impl(const GemmArgs& a) {
  static_assert(BN == 256 || BN == 192, "tile width");
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  constexpr int NT = 64 * NW;          // threads
  constexpr int WR = GB_TM / (NW / 2);  // rows of a wave's block (the waves form NW/2 x 2)
  constexpr int WM = WR / 32;           // 32-row matrix-core tiles per wave
  constexpr int NB = BN / 64;           // 32-wide n tiles per wave
  using OA = GbOp<A_KC, GB_TM, NT>;
  using OB = GbOp<B_KC, BN, NT>;
  // Two stages, each A's k tile then B's.
  constexpr int STG = OA::STAGE + OB::STAGE;
  __shared__ __attribute__((aligned(1024))) float L[2 * STG];
  float* const LA0 = L;
  float* const LB0 = L + OA::STAGE;
  float* const LA1 = L + STG;
  float* const LB1 = L + STG + OA::STAGE;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1, li = lane & 31, h = lane >> 5;
  const int G = (int)gridDim.x, g = (int)blockIdx.x;
  const GbSplit sp(a, G);

  // This workgroup's segments: `full` whole tiles, then the pieces of its
  // stream-K run [sb, se) cut at tile boundaries.
  if (sp.nk == 0) return;
  const int sb = sp.begin(g), se = sp.end(g);
  const int t0 = sb / sp.nk;
  const int npieces = se > sb ? (se - 1) / sp.nk - t0 + 1 : 0;
  const int ndp = sp.full;  // whole-tile-round segments
  const int nseg = ndp + npieces;
  if (nseg == 0) return;
  const int local = (g % 8) * (G / 8) + g / 8;  // XCD-major position in a round
  auto seg_of = [&](int j) {
    GbSeg s;
    int u, kt0 = 0, kt1 = sp.nk;
    s.slot = -1;
    if (j < ndp) {
      u = j * G + local;
    } else {
      const int p = j - ndp, t = t0 + p;
      u = sp.full * G + t;
      const int lo = t * sp.nk;
      kt0 = (sb > lo ? sb : lo) - lo;
      kt1 = (se < lo + sp.nk ? se : lo + sp.nk) - lo;
      if (kt0 != 0 || kt1 != sp.nk) s.slot = p == 0 ? 0 : 1;
    }
    int tm, tn;
    gb_locate(a, u, tm, tn, s);
    s.m0 = tm * GB_TM;
    s.n0 = tn * BN;
    s.kt0 = kt0;
    s.kt1 = kt1;
    return s;
  };

  uint32_t goa[OA::PER], gob[OB::PER];
#pragma unroll
  for (int i = 0; i < OA::PER; ++i) goa[i] = gb_goff<A_KC, GB_TM, NT>(a.lda, tid, i);
#pragma unroll
  for (int i = 0; i < OB::PER; ++i) gob[i] = gb_goff<B_KC, BN, NT>(a.ldb, tid, i);
  // Buffer resources of k tile kt of the tile at rows m0 (A) / columns n0 (B):
  // origin and the bytes from there to the operand's last element; a
  // resource of no bytes where the k tile stream has ended (reads give 0).
  // (Per batch: the bound is that batch's last element, so k past K reads 0.)
  auto rsrc_a = [&](const GbSeg& sg, int64_t kt, bool valid) -> __amdgpu_buffer_rsrc_t {
    const int64_t k0 = kt * GB_TK, m0 = sg.m0;
    if (!valid) return gb_rsrc(a.A, 0);
    const float* A = a.A + sg.ao;
    if constexpr (A_KC)
      return gb_rsrc(A + m0 * a.lda + k0, ((a.M - 1 - m0) * a.lda + a.K - k0) * 4);
    else
      return gb_rsrc(A + k0 * a.lda + m0, ((a.K - 1 - k0) * a.lda + a.M - m0) * 4);
  };
  auto rsrc_b = [&](const GbSeg& sg, int64_t kt, bool valid) -> __amdgpu_buffer_rsrc_t {
    const int64_t k0 = kt * GB_TK, n0 = sg.n0;
    if (!valid) return gb_rsrc(a.B, 0);
    const float* B = a.B + sg.bo;
    if constexpr (B_KC)
      return gb_rsrc(B + n0 * a.ldb + k0, ((a.N - 1 - n0) * a.ldb + a.K - k0) * 4);
    else
      return gb_rsrc(B + k0 * a.ldb + n0, ((a.K - 1 - k0) * a.ldb + a.N - n0) * 4);
  };
  // Staging registers: one k tile's pieces of A and B.
  vh_f4 ga[OA::PER], gb[OB::PER];
  auto piece = [](__amdgpu_buffer_rsrc_t r, uint32_t off) -> vh_f4 {
    return __builtin_bit_cast(vh_f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  };
  auto gload = [&](__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb) {
#pragma unroll
    for (int i = 0; i < OA::PER; ++i) ga[i] = piece(ra, goa[i]);
#pragma unroll
    for (int i = 0; i < OB::PER; ++i) gb[i] = piece(rb, gob[i]);
  };
  auto swrite = [&](float* SA, float* SB) {
#pragma unroll
    for (int i = 0; i < OA::PER; ++i) *reinterpret_cast<vh_f4*>(SA + gb_loff<A_KC, GB_TM, NT>(tid, i)) = ga[i];
#pragma unroll
    for (int i = 0; i < OB::PER; ++i) *reinterpret_cast<vh_f4*>(SB + gb_loff<B_KC, BN, NT>(tid, i)) = gb[i];
  };
  // Barrier for LDS only: the staging loads in flight are not waited for.
  auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // The load cursor walks the same k tile stream two tiles ahead of the
  // products: segment lj, k tile lkt (lv false past the end).
  int lj = 0;
  GbSeg lseg = seg_of(0);
  int lkt = lseg.kt0;
  bool lv = true;
  auto advance = [&]() {
    if (!lv) return;
    if (++lkt == lseg.kt1) {
      if (++lj < nseg) {
        lseg = seg_of(lj);
        lkt = lseg.kt0;
      } else {
        lv = false;
      }
    }
  };
  GbSeg cur = lseg;
  gload(rsrc_a(lseg, lkt, true), rsrc_b(lseg, lkt, true));
  swrite(LA0, LB0);
  advance();
  gload(rsrc_a(lseg, lkt, lv), rsrc_b(lseg, lkt, lv));
  lds_barrier();
  vh_f32x16 acc[WM][NB];

  // Fragment reads. k-contiguous: row base + the swizzled slot of k4 = 2q + h
  // (rows differ by multiples of 32, so swz depends on li only); row-
  // contiguous: four 32-bit reads 4 h .. 4 h + 3 k rows into the quarter.
  const int x = h ^ gb_swz(li);
  vh_f4 fa[2][WM], fb[2][NB];
  // Fragment f of quarter q into register set `set`: f < WM is A's row group
  // f, else B's column group f - WM.
  auto read_f = [&](const float* SA, const float* SB, int q, int set, int f) {
    if (f < WM) {
      const int row = wm * WR + 32 * f + li;
      if constexpr (A_KC) {
        fa[set][f] = *reinterpret_cast<const vh_f4*>(SA + row * GB_TK + (((2 * q) ^ x) << 2));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) fa[set][f][e] = SA[(8 * q + 4 * h + e) * OA::LT + row];
      }
    } else {
      const int jj = f - WM;
      const int row = wn * (BN / 2) + 32 * jj + li;
      if constexpr (B_KC) {
        fb[set][jj] = *reinterpret_cast<const vh_f4*>(SB + row * GB_TK + (((2 * q) ^ x) << 2));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) fb[set][jj][e] = SB[(8 * q + 4 * h + e) * OB::LT + row];
      }
    }
  };
  constexpr int NF = WM + NB;  // fragments per quarter
  // Reads in the order the products first need them: B's group 0, A's
  // groups, then B's other groups (the products run B group-major).
  auto read_q = [&](const float* SA, const float* SB, int q, int set) {
    read_f(SA, SB, q, set, WM);
#pragma unroll
    for (int f = 0; f < WM; ++f) read_f(SA, SB, q, set, f);
#pragma unroll
    for (int f = WM + 1; f < NF; ++f) read_f(SA, SB, q, set, f);
  };
  auto mfma_q = [&](int set, int e0, int e1) {
#pragma unroll
    for (int e = e0; e < e1; ++e)
#pragma unroll
      for (int jj = 0; jj < NB; ++jj)
#pragma unroll
        for (int i = 0; i < WM; ++i)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[set][i][e], fb[set][jj][e], acc[i][jj], 0, 0, 0);
  };
  read_q(LA0, LB0, 0, 0);

  // One k step on the stage (SA, SB), in two scheduling regions split by the
  // barrier:
  //   A: the staged k tile is written to the other stage (NA, NBp) and the
  //      staging registers reloaded with the one after, interleaved with the
  //      first products of quarter 0; then quarter 1's reads spread among the
  //      rest of quarter 0, quarters 1-2 likewise with the reads of 2-3, and
  //      half of quarter 3;
  //   B: after the barrier, quarter 0 of the other stage is read during the
  //      second half of quarter 3, so the next step starts on fragments
  //      already in registers.
  constexpr int VM = OA::PER + OB::PER;                  // LDS writes per step
  constexpr int VL = OA::PER + OB::PER;                  // load instructions per step
  constexpr int SP = VM + VL;                            // quarter-0 products that carry the staging
  constexpr int MQ = 4 * WM * NB;                        // products per quarter
  constexpr int RA = A_KC ? 1 : 4, RB = B_KC ? 1 : 4;    // LDS read instructions per fragment
  static_assert(SP <= MQ, "staging fits in quarter 0");
  auto kstep = [&](__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, const float* SA, const float* SB,
                   float* NA, float* NBp) {
    swrite(NA, NBp);
    gload(ra, rb);
    read_q(SA, SB, 1, 1);
    mfma_q(0, 0, 4);
    read_q(SA, SB, 2, 0);
    mfma_q(1, 0, 4);
    read_q(SA, SB, 3, 1);
    mfma_q(0, 0, 4);
    mfma_q(1, 0, 2);
#pragma unroll
    for (int i = 0; i < VM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    // Quarter 0: after the staging, quarter 1's reads over the products
    // left; quarters 1-2: the next quarter's reads one per RP products from
    // the start, so the last arrives well before the quarter ends.
    constexpr int RP = (MQ / 2) / NF;
    __builtin_amdgcn_sched_group_barrier(0x008, (MQ - SP) % NF, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
#pragma unroll
    for (int f = 0; f < WM; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x008, (MQ - SP) / NF, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
    }
#pragma unroll
    for (int f = WM + 1; f < NF; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x008, (MQ - SP) / NF, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, (MQ - SP) / NF, 0);
#pragma unroll
    for (int q = 1; q < 3; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, RP, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
#pragma unroll
      for (int f = 0; f < WM; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, RP, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
      }
#pragma unroll
      for (int f = WM + 1; f < NF; ++f) {
        __builtin_amdgcn_sched_group_barrier(0x008, RP, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, MQ - NF * RP, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MQ / 2, 0);
    lds_barrier();
    read_q(NA, NBp, 0, 0);
    mfma_q(1, 2, 4);
    __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, MQ / 2 / NF, 0);
#pragma unroll
    for (int f = 0; f < WM; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, MQ / 2 / NF, 0);
    }
#pragma unroll
    for (int f = WM + 1; f < NF; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x100, RB, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, MQ / 2 / NF, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, (MQ / 2) % NF, 0);
  };

  int s = 0;
  // The current segment's epilogue straight from the accumulators: register
  // r of a 32 x 32 tile holds row 8 (r / 4) + 4 h + r % 4, column li. A
  // partial piece goes raw to its workspace slot, a whole tile to C as
  // alpha v (+ E) (+ C) inside M x N. The row stride and this lane's row and
  // column are opaque here, so that the compiler forms the per-element
  // offsets where they are used instead of keeping them in registers across
  // the whole segment loop.
  auto epilogue = [&]() {
    const bool raw = cur.slot >= 0;
    int64_t ldo = raw ? BN : a.ldc;
    int lrow = wm * WR + 4 * h, lcol = wn * (BN / 2) + li;
    asm volatile("" : "+s"(ldo), "+v"(lrow), "+v"(lcol));
    const int64_t slot_elems = (int64_t)GB_TM * BN;
    if (raw) {
      float* base = a.ws + ((int64_t)g * GB_SLOTS + cur.slot) * slot_elems + lrow * BN + lcol;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float* row = base + (32 * i + 8 * (r >> 2) + (r & 3)) * BN;
#pragma unroll
          for (int jj = 0; jj < NB; ++jj) row[32 * jj] = acc[i][jj][r];
        }
      return;
    }
    const bool inner = cur.m0 + GB_TM <= a.M && cur.n0 + BN <= a.N;
    float* const Cb = a.C + cur.co;
    const float* const Eb = a.E ? a.E + cur.eo : nullptr;
    if (inner && !a.E && !a.accumulate) {
      float* base = Cb + (cur.m0 + lrow) * ldo + cur.n0 + lcol;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float* row = base + (32 * i + 8 * (r >> 2) + (r & 3)) * ldo;
#pragma unroll
          for (int jj = 0; jj < NB; ++jj) row[32 * jj] = acc[i][jj][r] * a.alpha;
        }
      return;
    }
    if (inner && (!Eb || a.sem == 0)) {
      // Whole tile inside C with at most a per-column addend (a bias, E
      // stride 0 along m, read once per column): v = alpha acc (+ bias)
      // (+ old C), in gm_finish's order, no bounds tests. The stores may
      // alias the old-C reads as far as the compiler knows, so it keeps
      // each read behind the stores before it: the reads go out 8 rows x
      // NB columns at a time, ahead of their stores, so a wave waits on
      // memory 2 WM times, not once per element.
      float* base = Cb + (cur.m0 + lrow) * ldo + cur.n0 + lcol;
      float eb[NB];
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) eb[jj] = Eb ? Eb[(cur.n0 + lcol + 32 * jj) * a.sen] : 0.0f;
      auto tile = [&](auto has_bias, auto acc_c) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int r0 = 0; r0 < 16; r0 += 8) {
            float old[8][NB];
            if constexpr (decltype(acc_c)::value) {
#pragma unroll
              for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int jj = 0; jj < NB; ++jj)
                  old[r][jj] = base[(32 * i + 8 * ((r0 + r) >> 2) + ((r0 + r) & 3)) * ldo + 32 * jj];
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              float* row = base + (32 * i + 8 * ((r0 + r) >> 2) + ((r0 + r) & 3)) * ldo;
#pragma unroll
              for (int jj = 0; jj < NB; ++jj) {
                float v = acc[i][jj][r0 + r] * a.alpha;
                if constexpr (decltype(has_bias)::value) v = v + eb[jj];
                if constexpr (decltype(acc_c)::value) v = old[r][jj] + v;
                row[32 * jj] = v;
              }
            }
          }
      };
      using T = std::true_type;
      using F = std::false_type;
      if (Eb) {
        if (a.accumulate) tile(T{}, T{}); else tile(T{}, F{});
      } else {
        tile(F{}, T{});  // accumulate (the plain store returned above)
      }
      return;
    }
    if (inner) {
      // Whole tile inside C with a full addend E[m, n]: v = alpha acc + E
      // (+ old C), in gm_finish's order, without bounds tests.
      float* base = Cb + (cur.m0 + lrow) * ldo + cur.n0 + lcol;
      const float* E = Eb;
      const bool ecol = E && a.sem == 0;
      float eb[NB];
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) eb[jj] = ecol ? E[(cur.n0 + lcol + 32 * jj) * a.sen] : 0.0f;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = 32 * i + 8 * (r >> 2) + (r & 3);
          float* row = base + rl * ldo;
#pragma unroll
          for (int jj = 0; jj < NB; ++jj) {
            float v = acc[i][jj][r] * a.alpha;
            if (ecol)
              v = v + eb[jj];
            else if (E)
              v = v + E[(cur.m0 + lrow + rl) * a.sem + (cur.n0 + lcol + 32 * jj) * a.sen];
            if (a.accumulate) v = row[32 * jj] + v;
            row[32 * jj] = v;
          }
        }
      return;
    }
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) {
        const int64_t n = cur.n0 + lcol + 32 * jj;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = 32 * i + 8 * (r >> 2) + (r & 3);
          const int64_t m = cur.m0 + lrow + rl;
          if (m < a.M && n < a.N) {
            float* cp = Cb + m * ldo + n;
            *cp = gm_finish(a, Eb, false, acc[i][jj][r], m, n, a.accumulate ? *cp : 0.0f);
          }
        }
      }
  };
  // Segments in order; per segment, one k step per k tile on alternating
  // stages (the staged tile -- the next in the stream -- goes to LDS and the
  // one after it is loaded), then the epilogue.
  for (int j = 0;;) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) acc[i][jj] = vh_f32x16{};
    for (int kt = cur.kt0; kt < cur.kt1; ++kt) {
      advance();
      kstep(rsrc_a(lseg, lkt, lv), rsrc_b(lseg, lkt, lv), s ? LA1 : LA0, s ? LB1 : LB0, s ? LA0 : LA1,
            s ? LB0 : LB1);
      s ^= 1;
    }
    epilogue();
    if (++j == nseg) break;
    cur = seg_of(j);
  }
}

// Finishes the tiles of the stream-K round that were split between
// workgroups: C = epilogue(sum of the pieces in k order). Workgroup
// (blockIdx.x) takes 16 rows of split tile blockIdx.x / (256 / 16).
template <int BN>
VH_DEV void gemm_big_fix_impl(const GemmArgs& a) {
  const int G = a.ksplit;  // the main kernel's grid
  const GbSplit sp(a, G);
  const int t = (int)(blockIdx.x / (GB_TM / 16));
  const int rows0 = (int)(blockIdx.x % (GB_TM / 16)) * 16;
  if (t >= sp.rem) return;
  // Workgroups whose runs meet tile t: [glo, ghi].
  const int lo = t * sp.nk, hi = lo + sp.nk;
  int glo = 0, ghi = G - 1;
  {
    int l = 0, r = G - 1;  // first g with end(g) > lo
    while (l < r) {
      const int m = (l + r) / 2;
      if (sp.end(m) > lo) r = m; else l = m + 1;
    }
    glo = l;
    l = 0;
    r = G - 1;  // last g with begin(g) < hi
    while (l < r) {
      const int m = (l + r + 1) / 2;
      if (sp.begin(m) < hi) l = m; else r = m - 1;
    }
    ghi = l;
  }
  if (glo == ghi) return;  // one workgroup covered the whole tile and stored it
  int tm, tn;
  GbSeg sg;
  gb_locate(a, sp.full * G + t, tm, tn, sg);
  float* const Cb = a.C + sg.co;
  const float* const Eb = a.E ? a.E + sg.eo : nullptr;
  const int64_t m0 = (int64_t)tm * GB_TM, n0 = (int64_t)tn * BN;
  constexpr int Q = BN / 4;  // 128-bit pieces per row
  for (int f = threadIdx.x; f < 16 * Q; f += 256) {
    const int rl = rows0 + f / Q, cl = (f % Q) * 4;
    vh_f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    // The pieces of workgroups glo..ghi, four at a time: the four loads go
    // out together, then the pieces are added in workgroup order. Indices
    // past ghi are clamped to ghi and not added; with fewer k tiles than
    // workgroups (W < G) some runs are empty and wrote no piece: their slots
    // (in bounds, holding an earlier call's data) are read but not added.
    for (int g0 = glo; g0 <= ghi; g0 += 4) {
      vh_f4 p[4];
      bool used[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int gg = g0 + j <= ghi ? g0 + j : ghi;
        const int b = sp.begin(gg);
        used[j] = g0 + j <= ghi && b != sp.end(gg);
        const int slot = b / sp.nk == t ? 0 : 1;
        p[j] = *reinterpret_cast<const vh_f4*>(a.ws + ((int64_t)gg * GB_SLOTS + slot) * GB_TM * BN + rl * BN + cl);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (used[j]) v += p[j];
    }
    const int64_t m = m0 + rl;
    if (m >= a.M) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t n = n0 + cl + e;
      if (n < a.N) {
        float* cp = Cb + m * a.ldc + n;
        *cp = gm_finish(a, Eb, false, v[e], m, n, a.accumulate ? *cp : 0.0f);
      }
    }
  }
}
