// vh_kargs.h -- kernel argument blocks shared by the host runtime and the gfx950
// code object. Every kernel takes exactly one of these structs by value, so the
// host (hipModuleLaunchKernel with a one-element kernelParams array) and the
// device always agree on the parameter layout.
#pragma once
#include <stdint.h>

#define VH_MAX_RANK 8

// Device-side error record (one per device, zeroed at init). Kernels that meet an
// input the CPU backend would panic on fold (index << 32 | value bits) into the
// record with an atomic min, so the host reports the FIRST offending element in
// row-major order, as the CPU's sequential loop does.
struct VhErrRecord {
  unsigned long long token;   // embedding fwd/bwd: bad token id
  unsigned long long target;  // cross-entropy fwd/bwd: bad target class
  unsigned int token_bound;   // vocabulary size of the failing embedding launch
  unsigned int target_bound;  // vocabulary size of the failing cross-entropy launch
};
#define VH_ERR_NONE 0xFFFFFFFFFFFFFFFFull

struct LnFwdArgs {
  const float* x;
  const float* w;
  const float* b;
  float* y;
  int64_t rows;
  int32_t C;
  float eps;
};

struct LnBwdArgs {
  const float* x;
  const float* w;
  const float* dy;
  float* dx;
  float* part;  // [nblocks][2][C] per-block dgamma / dbeta partials
  int64_t rows;  // rows are dealt grid-stride to the gridDim.x * teams-per-block teams
  int32_t C;
  float eps;
};

// LayerNorm backward over rows too long for the register kernels
// (kernels/rowwide.h): per-row statistics, then column tiles over row blocks.
struct LnWideArgs {
  const float* x;
  const float* w;
  const float* dy;
  float* dx;
  float* stats;  // [rows][4]: mean, inv_std, sum(dy*w), sum(dy*w*xhat)
  float* part;   // [row blocks][2][C] dgamma / dbeta partials
  int64_t rows;
  int64_t rpb;   // rows per row block
  int32_t C;
  float eps;
};

// Column reduction of [P][2][C] partials into dw[C], db[C] (fixed order).
// Column reduce launch shape: VH_COLR_COLS columns per workgroup, 16 partial
// ranges per column, so VH_COLR_COLS * 16 threads.
#define VH_COLR_COLS 16
struct ColReduceArgs {
  const float* part;
  float* out0;  // component 0 (dgamma / dbias)
  float* out1;  // component 1 (dbeta); unused when ncomp == 1
  int32_t P;
  int32_t C;
  int32_t ncomp;
};

// Per-workgroup column sums of a [rows, C] block of rows (first stage of a
// fixed-order row sum; the second stage is the column reduce above).
struct ColPartialArgs {
  const float* x;
  float* part;  // [G][C]
  int64_t rows;
  int64_t rpb;  // rows per workgroup
  int32_t C;
};

struct SoftmaxArgs {
  const float* x;   // fwd: scores; bwd: y (or x when input_is_x)
  const float* dy;  // bwd only
  float* y;         // fwd: probabilities; bwd: dx
  int64_t rows;
  int32_t T;        // row length
  int32_t causal;   // 1: row r keeps columns [0, r % T], the rest are known masked
  int32_t input_is_x;
  int32_t attn;     // 1: fused-attention numerics (p = e * (1/(sum + 1e-9)), fma sum of dy*y)
  int32_t ztile;    // causal, > 0: a row's masked zeros are written only up to the end of
                    // its ztile-row tile (what the causal products read); 0: the whole row
  const int32_t* causal_flag;  // non-null: the causal form applies only when *causal_flag is 1,
                               // else the rows are dense (decided on the device: vh_attn_decide)
};

// C tile of one GEMM workgroup (host and device agree on the grid).
#define VH_GEMM_TILE_M 128
#define VH_GEMM_TILE_N 128
// The persistent kernel for large dense products (kernels/gemm_big.h): C tile
// rows x columns, and the workspace slots per workgroup of its stream-K round.
#define VH_GEMMB_TM 256
#define VH_GEMMB_TN 192       // the default tile width (and the smallest N it takes)
#define VH_GEMMB_TN_WIDE 256  // the tile width for long k loops over a row-contiguous B
#define VH_GEMMB_WIDE_K 8192  // K (whole k tiles) from which the wide tile is used
#define VH_GEMMB_SLOTS 2

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  const float* E;  // optional addend E[m, n] (null = none)
  int64_t M, N, K;
  int64_t lda;  // A's non-unit stride: along m (k-contiguous A) or along k (m-contiguous A)
  int64_t ldb;  // B's non-unit stride: along n (k-contiguous B) or along k (n-contiguous B)
  int64_t ldc;  // C row stride; C's column stride is 1
  int64_t sa1, sa2, sb1, sb2, sc1, sc2, se1, se2;  // strides of the two batch dims
  int64_t sem, sen;                                // E strides along m and n
  int32_t nb2;                                     // size of the inner batch dim
  int32_t tiles_m, tiles_n;
  int32_t accumulate;  // 1: C = C + result
  int32_t causal;      // 0 none; 1 skip tiles above the diagonal; 2 k <= m; 3 k >= m
  float alpha;
  // Split K (unbatched only): workgroup row y takes k in [y*kchunk, (y+1)*kchunk)
  // and stores its raw partial to ws[y][M][N]; vh_gemm_reduce finishes.
  int32_t ksplit;
  int64_t kchunk;
  float* ws;
  int64_t nbat;  // persistent form (vh_gemmp_*): batches in the launch (grid y is 1)
  const int32_t* causal_flag;  // non-null: `causal` applies only when *causal_flag is 1, else dense
};

// Fixed-order sum of the split-K partials plus the GEMM epilogue.
struct GemmReduceArgs {
  const float* ws;  // [ksplit][M][N]
  float* C;
  const float* E;
  int64_t M, N, ldc, sem, sen;
  int32_t ksplit;
  int32_t accumulate;
  float alpha;
};

struct AdamArgs {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  float beta1, beta2, omb1, omb2;  // omb = 1 - beta, rounded to f32 as the reference does
  float bc1, bc2;                  // 1 - beta^t
  float lr, lrwd, eps;             // lrwd = lr * weight_decay (f32)
};

// Several parameter tensors in one launch: tensor s takes blocks
// [blk0, blk0 + its units / 256 rounded up), units of 4 floats (vec) or 1.
#define VH_ADAMW_MULTI_MAX 32
struct AdamSeg {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  int32_t blk0;
  int32_t vec;
};
struct AdamMultiArgs {
  AdamArgs h;  // the hyper-parameters (p, g, m, v, n unused)
  int32_t count;
  int32_t pad;
  AdamSeg seg[VH_ADAMW_MULTI_MAX];
};

struct EltArgs {
  const float* x;
  const float* bias;  // [C] or null
  const float* dy;
  float* y;
  int64_t n;
  int32_t C;          // bias period (row length) when bias != null
};

struct GeluBiasBwdArgs {
  const float* x;
  const float* bias;
  const float* dy;
  float* dx;
  float* part;  // [nblocks][C] dbias partials
  int64_t rows;
  int64_t rows_per_block;
  int32_t C;
};

struct EmbFwdArgs {
  const float* ids;
  const float* W;
  float* out;
  VhErrRecord* err;
  int64_t n;
  int32_t V;
  int32_t D;
};

// Embedding backward: sort-by-token CSR build + segmented gather-sum.
struct EmbTokArgs {
  const float* ids;
  int32_t* tok;      // [n] validated token ids (-1 on error)
  int32_t* counts;   // [V] hits per vocabulary row (zeroed by the host)
  VhErrRecord* err;
  int64_t n;
  int32_t V;
};

struct EmbAllocArgs {
  const int32_t* counts;  // [V] hits per vocabulary row
  int32_t* heavy_index;   // [V] heavy entry or -1
  int32_t* heavy;         // [4 * max] token, first task, task count, hits
  int32_t* taskmap;       // [tasks] heavy entry of each task
  int32_t* blkcnt;        // [max][nblk] heavy hits per position block
  int32_t* ctr;           // [2]: heavy entries, tasks (zeroed by the host)
  int32_t V;
  int32_t nblk;
};

struct EmbPlaceArgs {
  const int32_t* tok;
  const int32_t* heavy_index;
  int32_t* cursor;  // [V] zeroed
  int32_t* pos;     // [V][16] light positions per vocabulary row (unordered)
  int32_t* blkcnt;
  int64_t n;
  int32_t nblk;
  int32_t blk_shift;  // positions per block = 1 << blk_shift (>= 64)
};

struct EmbSegArgs {
  const int32_t* counts;
  const int32_t* pos;
  const int32_t* tok;
  const int32_t* heavy;
  const int32_t* taskmap;
  const int32_t* blkcnt;
  const int32_t* ctr;
  float* partial;  // [tasks][D] heavy partial rows
  const float* dy;
  float* dW;
  int64_t n;
  int32_t V;
  int32_t D;
  int32_t nblk;
  int32_t blk_shift;
  int32_t heavy_blocks;  // leading workgroups that run heavy tasks
  int32_t slices;        // column slices per heavy task (64 units of VW floats each)
};

// Embedding backward, sorted path (n <= 16384, V <= 65534). Launch 1:
// workgroup k < EMB_RANGES sorts the keys of the tokens t % EMB_RANGES == k
// and writes that range's lists (below); the others write dW's zeros. Launch 2
// walks the lists (light segment sums; heavy partial rows, the last task of a
// heavy row's column slice adding them into dW), each wave taking the 16
// ranges' counts and their prefix sums itself.
#define EMB_RANGES 16
#define EMB_SORT_MAXV 65534  // vocabulary bound of the sorted path (t / EMB_RANGES < 4096)
#define EMB_REC 20  // ints per segment record: token, start, hits, 0, then a light token's positions
struct EmbSortArgs {
  const float* ids;
  float* dW;             // zeroed by workgroups EMB_RANGES.. (fill_n units of 4 floats if vec, else 1)
  int32_t* spos;         // [EMB_RANGES][n]: each range's positions sorted by token, ascending within a token
  int32_t* seg;          // [EMB_RANGES][n][20]: token, start in the range's spos, hits, 0, then the positions
                         // of a light token (<= 16 hits) -- one record per token
  int32_t* heavy;        // [EMB_RANGES][hmax][4]: token, range-local first task, task count, hits
  int32_t* heavy_start;  // [EMB_RANGES][hmax]: start in the range's spos of each heavy token's hits
  int32_t* taskmap;      // [EMB_RANGES][tmax]: range-local heavy entry of each task
  int32_t* counts;       // [3][EMB_RANGES]: segments, tasks, heavy entries of each range
  int32_t* ctr;          // [EMB_RANGES][hmax + tmax][slices]: launch 2's counters (groups finished per
                         // heavy entry and slice, then tasks finished per group and slice), zeroed here
  VhErrRecord* err;
  int64_t fill_n;
  int32_t n;
  int32_t V;
  int32_t hmax;
  int32_t tmax;
  int32_t vec;
  int32_t slices;        // column slices per heavy row (64 units each)
};

struct EmbSumArgs {
  const int32_t* spos;
  const int32_t* seg;
  const int32_t* heavy;
  const int32_t* heavy_start;
  const int32_t* taskmap;
  const int32_t* counts;
  int32_t* ctr;    // [EMB_RANGES][hmax + tmax][slices]: groups finished per (heavy entry, slice), then
                   // tasks finished per (group's first task, slice); zero at launch
  float* partial;  // [tasks][D], tasks numbered range by range
  const float* dy;
  float* dW;
  int32_t n;
  int32_t hmax;
  int32_t tmax;
  int32_t D;
  int32_t slices;  // column slices per heavy task / heavy row (64 units of VW floats each)
};

// Heavy rows' final sums: one wave per (heavy entry, column slice).
struct EmbFinalArgs {
  const int32_t* heavy;   // [4 * max] token, first task, task count, hits
  const int32_t* ctr;     // [0]: heavy entries
  const float* partial;   // [tasks][D]
  float* dW;
  int32_t D;
  int32_t slices;
};

struct XentArgs {
  const float* logits;
  const float* targets;
  const float* grad_out;  // bwd: device scalar
  float* out;             // fwd: per-row losses [B]; bwd and fused: dlogits [B, V]
  float* row_loss;        // fused forward+backward: per-row losses [B]
  VhErrRecord* err;
  int64_t B;
  int64_t ld;             // row stride of logits and dlogits (>= V)
  int32_t V;
  float* stats;           // fwd: NULL or per-row (max, sum-exp) out [B, 2]; bwd_rs: in
};

struct XentReduceArgs {
  const float* row_loss;  // [B]
  float* loss;            // [1]
  int64_t B;
};

struct StridedLayout {
  int32_t rank;
  int32_t pad;
  int64_t dims[VH_MAX_RANK];
  int64_t strides[VH_MAX_RANK];
};

struct BinaryArgs {
  const float* l;
  const float* r;
  float* out;
  StridedLayout ol;  // output dims, contiguous strides
  StridedLayout ll;  // lhs strides aligned to the output rank (0 for broadcast dims)
  StridedLayout rl;  // rhs strides aligned to the output rank
  int64_t n;
  int32_t op;        // 0 add, 1 sub, 2 mul, 3 div
  int32_t contiguous;
  int64_t bn;        // row-broadcast form: the vector's length (a product of the output's trailing
                     // dims, or 1); column-broadcast form: output elements per vector element
  int32_t vec_lhs;   // broadcast forms: 1 when the vector is the left operand
};

struct ReduceArgs {
  const float* x;
  float* out;
  StridedLayout ol;  // outer (kept) dims with input strides, dim removed
  int64_t n_out;
  int64_t red_len;
  int64_t red_stride;
  int32_t mean;
};

struct CopyArgs {
  const float* src;
  float* dst;
  StridedLayout sl;  // dims + source strides
  int64_t n;
};

// dst[b][r][c] = src[b0 * sb0 + b1 * sb1 + r + c * sc] for a view whose last
// dim is strided and whose second-to-last has unit stride (a transpose), with
// up to two leading dims flattened into b = b0 * nb1 + b1.
struct TransposeArgs {
  const float* src;
  float* dst;
  int64_t R, C, sc;
  int64_t nb1, sb0, sb1;
};

struct FillArgs {
  float* p;
  int64_t n;
  float value;
};

// Diagnostic: y[i] = expf / logf / tanhf (x[i]) (fn = VH_MATH_EXP / LOG / TANH).
struct MathProbeArgs {
  const float* x;
  float* y;
  int64_t n;
  int32_t fn;
};

// Device-to-device copy of n4 16-byte units (both pointers 16-byte aligned).
struct StreamCopyArgs {
  const float* src;
  float* dst;
  int64_t n4;
};

// Whether an additive attention mask may be replaced by the causal kernels
// (vh_attention_mask_is_causal): segment 0 is the mask over its own dims
// (right-aligned to 4, the last two [S, S]), segments 1-4 are q, k, v and the
// output gradient ([B, H, S, Dk], unit last stride; rows = 0 for an absent one).
struct AttnProbeArgs {
  const float* t[5];
  int32_t d0[5], d1[5], d2[5], d3[5];     // dims
  int64_t s0[5], s1[5], s2[5], s3[5];     // strides (elements)
  uint32_t* words;  // 64 slots of 8: [0] mask pattern failures, [1] 0x7f800000 - min |masked| bits, [2..5] max |x| bits of q, k, v, g
  int32_t Y;        // grid y per segment: the largest leading (b, h) count
};

// The probe's verdict from its 64 slots (vh_attn_decide, one wave): *flag = 1
// when the causal kernels give the dense masked form's bits, else 0.
struct AttnDecideArgs {
  const uint32_t* words;
  int32_t* flag;
  double scale;  // the attention's 1/sqrt(Dk) as f32, widened
  int32_t Dk;
  int32_t has_g;  // the backward's output gradient was probed (segment 4)
};
