/*
 * vearo_cpu_gpt.c -- CPU oracle, part 2: matmul, fused attention, AdamW and the
 * SimpleGPT training step of config[4] (token+position embedding, one pre-LN
 * transformer block, final layernorm, lm_head, cross-entropy, autograd
 * backward, AdamW).
 *
 * TEST INFRASTRUCTURE. Nothing in the product links, loads or calls this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Numerics follow the Rust sources cited per function (paths as in
 * vearo_cpu_ref.h, plus nn: crates/vearo-nn/src/lib.rs, tensor:
 * crates/vearo-core/src/tensor.rs, optim: crates/vearo-optim/src/lib.rs).
 * `mul_add` in Rust is a fused multiply-add with one rounding; it is fmaf()
 * here (or the equivalent AVX2 vfmadd, which rounds identically). Loops are
 * blocked and threaded for speed, but every output element is produced by the
 * same chain of operations in the same order as the reference's loops, so the
 * results are bit-identical to a straight restatement: blocking only reorders
 * work across independent elements, never within one element's chain.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "vearo_cpu_ref.h"

/* ------------------------------------------------------------ threading -- */

static int g_threads;

void vo_set_threads(int n) { g_threads = n; }

static int nthreads(void) {
  if (g_threads > 0) return g_threads;
  const char* e = getenv("VO_THREADS");
  if (!e || !*e) e = getenv("OMP_NUM_THREADS");
  if (e && atoi(e) > 0) return atoi(e);
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

typedef void (*task_fn)(void* ctx, int64_t begin, int64_t end);
typedef struct {
  task_fn fn;
  void* ctx;
  int64_t begin, end;
} chunk_t;

static void* run_chunk(void* p) {
  chunk_t* c = (chunk_t*)p;
  c->fn(c->ctx, c->begin, c->end);
  return NULL;
}

/* Runs fn over [0, n) split into contiguous ranges, one per thread. Which
 * thread computes an item never changes its value (items are independent). */
static void parallel_for(int64_t n, task_fn fn, void* ctx) {
  int64_t t = nthreads();
  if (t > n) t = n;
  if (t <= 1) {
    if (n > 0) fn(ctx, 0, n);
    return;
  }
  pthread_t* th = (pthread_t*)calloc((size_t)t, sizeof(pthread_t));
  chunk_t* c = (chunk_t*)calloc((size_t)t, sizeof(chunk_t));
  int* started = (int*)calloc((size_t)t, sizeof(int));
  int64_t per = (n + t - 1) / t;
  for (int64_t i = 0; i < t; ++i) {
    c[i].fn = fn;
    c[i].ctx = ctx;
    c[i].begin = i * per;
    c[i].end = (i + 1) * per < n ? (i + 1) * per : n;
    if (c[i].begin >= c[i].end) continue;
    if (pthread_create(&th[i], NULL, run_chunk, &c[i]) == 0)
      started[i] = 1;
    else
      run_chunk(&c[i]);
  }
  for (int64_t i = 0; i < t; ++i)
    if (started[i]) pthread_join(th[i], NULL);
  free(th);
  free(c);
  free(started);
}

static int have_fma(void) {
  static int cached = -1;
  if (cached < 0) {
    __builtin_cpu_init();
    cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  }
  return cached;
}

/* -------------------------------------------------------------- matmul -- */

/* cpu:384-393 (the portable branch; the 4x8 AVX2 block at cpu:318-370 runs
 * the same per-element chain): for each output row, row[n] starts at 0.0 and
 * for k ascending row[n] = lhs[m,k].mul_add(rhs[k,n], row[n]). Below, C is
 * zeroed by the caller and the k loop runs in ascending chunks, so each C
 * element sees exactly that chain. */
#define MM_KC 256
#define MM_MB 96
#define MM_NB 256

__attribute__((target("avx2,fma"))) static void mk_6x16(const float* A, int64_t lda, const float* B,
                                                      int64_t ldb, float* C, int64_t ldc, int64_t k0,
                                                      int64_t k1) {
  __m256 c[6][2];
  for (int r = 0; r < 6; ++r) {
    c[r][0] = _mm256_loadu_ps(C + r * ldc);
    c[r][1] = _mm256_loadu_ps(C + r * ldc + 8);
  }
  for (int64_t k = k0; k < k1; ++k) {
    const __m256 b0 = _mm256_loadu_ps(B + k * ldb);
    const __m256 b1 = _mm256_loadu_ps(B + k * ldb + 8);
    for (int r = 0; r < 6; ++r) {
      const __m256 a = _mm256_broadcast_ss(A + r * lda + k);
      c[r][0] = _mm256_fmadd_ps(a, b0, c[r][0]);
      c[r][1] = _mm256_fmadd_ps(a, b1, c[r][1]);
    }
  }
  for (int r = 0; r < 6; ++r) {
    _mm256_storeu_ps(C + r * ldc, c[r][0]);
    _mm256_storeu_ps(C + r * ldc + 8, c[r][1]);
  }
}

static void mk_any(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                   int64_t rows, int64_t cols, int64_t k0, int64_t k1) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = k0; k < k1; ++k) {
      const float a = A[r * lda + k];
      for (int64_t j = 0; j < cols; ++j) C[r * ldc + j] = fmaf(a, B[k * ldb + j], C[r * ldc + j]);
    }
}

/* C[M,N] += A[M,K] B[K,N] (all row-major with leading dims), C pre-zeroed. */
static void mm_tile(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                    int64_t M, int64_t N, int64_t K) {
  const int fast = have_fma();
  for (int64_t k0 = 0; k0 < K; k0 += MM_KC) {
    const int64_t k1 = k0 + MM_KC < K ? k0 + MM_KC : K;
    for (int64_t j = 0; j < N; j += 16) {
      const int64_t cols = N - j < 16 ? N - j : 16;
      for (int64_t i = 0; i < M; i += 6) {
        const int64_t rows = M - i < 6 ? M - i : 6;
        if (fast && rows == 6 && cols == 16)
          mk_6x16(A + i * lda, lda, B + j, ldb, C + i * ldc + j, ldc, k0, k1);
        else
          mk_any(A + i * lda, lda, B + j, ldb, C + i * ldc + j, ldc, rows, cols, k0, k1);
      }
    }
  }
}

typedef struct {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, K, mt, nt;
  const int64_t* aoff;
  const int64_t* boff;
} mm_ctx;

static void mm_task(void* p, int64_t begin, int64_t end) {
  const mm_ctx* c = (const mm_ctx*)p;
  const int64_t per_batch = c->mt * c->nt;
  for (int64_t t = begin; t < end; ++t) {
    const int64_t b = t / per_batch, r = t % per_batch;
    const int64_t i0 = (r / c->nt) * MM_MB, j0 = (r % c->nt) * MM_NB;
    const int64_t rows = c->M - i0 < MM_MB ? c->M - i0 : MM_MB;
    const int64_t cols = c->N - j0 < MM_NB ? c->N - j0 : MM_NB;
    float* Cb = c->C + b * c->M * c->N + i0 * c->N + j0;
    for (int64_t i = 0; i < rows; ++i) memset(Cb + i * c->N, 0, (size_t)cols * sizeof(float));
    mm_tile(c->A + c->aoff[b] + i0 * c->K, c->K, c->B + c->boff[b] + j0, c->N, Cb, c->N, rows, cols, c->K);
  }
}

/* Batched matmul over broadcast batch dims of contiguous operands
 * (cpu:266-417; both operands are made contiguous there first). */
static void matmul_batched(const float* A, const float* B, float* C, int64_t nbatch, const int64_t* aoff,
                           const int64_t* boff, int64_t M, int64_t N, int64_t K) {
  if (M == 0 || N == 0 || nbatch == 0) return;
  mm_ctx c = {A, B, C, M, N, K, (M + MM_MB - 1) / MM_MB, (N + MM_NB - 1) / MM_NB, aoff, boff};
  parallel_for(nbatch * c.mt * c.nt, mm_task, &c);
}

/* 2-D C[M,N] = A[M,K] B[K,N]. */
static void matmul2(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  const int64_t z = 0;
  matmul_batched(A, B, C, 1, &z, &z, M, N, K);
}

int vo_matmul(const float* lhs, const vo_layout* ll, const float* rhs, const vo_layout* rl, float* out,
              char* err, size_t errlen) {
  if (ll->rank < 2 || rl->rank < 2) {
    if (err && errlen) snprintf(err, errlen, "Matmul requires rank >= 2");
    return VO_PANIC;
  }
  const int64_t M = ll->dims[ll->rank - 2], K = ll->dims[ll->rank - 1];
  const int64_t K2 = rl->dims[rl->rank - 2], N = rl->dims[rl->rank - 1];
  if (K != K2) {
    if (err && errlen) snprintf(err, errlen, "Incompatible dimensions for matmul");
    return VO_PANIC;
  }
  const int lb = ll->rank - 2, rb = rl->rank - 2;
  const int ob = lb > rb ? lb : rb;
  int64_t odims[VO_MAX_RANK];
  for (int i = 0; i < ob; ++i) {
    const int li = i - (ob - lb), ri = i - (ob - rb);
    const int64_t a = li >= 0 ? ll->dims[li] : 1, b = ri >= 0 ? rl->dims[ri] : 1;
    if (a != b && a != 1 && b != 1) {
      if (err && errlen) snprintf(err, errlen, "Batch shapes are not broadcastable");
      return VO_PANIC;
    }
    odims[i] = a > b ? a : b;
  }
  int64_t nbatch = 1;
  for (int i = 0; i < ob; ++i) nbatch *= odims[i];
  int64_t* aoff = (int64_t*)calloc((size_t)(nbatch ? nbatch : 1), sizeof(int64_t));
  int64_t* boff = (int64_t*)calloc((size_t)(nbatch ? nbatch : 1), sizeof(int64_t));
  for (int64_t bi = 0; bi < nbatch; ++bi) {
    int64_t rem = bi, ao = 0, bo = 0, as = M * K, bs = K * N;
    for (int i = ob - 1; i >= 0; --i) {
      const int64_t c = rem % odims[i];
      rem /= odims[i];
      const int li = i - (ob - lb), ri = i - (ob - rb);
      if (li >= 0) {
        if (ll->dims[li] != 1) ao += c * as;
        as *= ll->dims[li];
      }
      if (ri >= 0) {
        if (rl->dims[ri] != 1) bo += c * bs;
        bs *= rl->dims[ri];
      }
    }
    aoff[bi] = ao;
    boff[bi] = bo;
  }
  matmul_batched(lhs, rhs, out, nbatch, aoff, boff, M, N, K);
  free(aoff);
  free(boff);
  return VO_OK;
}

/* ------------------------------------------------------ fused attention -- */

/* Mask right-aligned to rank 4 (cpu:2395-2404): dims[4] with leading ones. */
typedef struct {
  const float* q;
  const float* k;
  const float* v;
  const float* go;
  const float* mask;
  int64_t mdims[4];
  float *out, *dq, *dk, *dv;
  int64_t H, S, Dk;
} att_ctx;

static inline float mask_at(const att_ctx* c, int64_t b, int64_t h, int64_t i, int64_t j) {
  const int64_t* m = c->mdims;
  const int64_t mb = m[0] == 1 ? 0 : b, mh = m[1] == 1 ? 0 : h, ms = m[2] == 1 ? 0 : i,
                mc = m[3] == 1 ? 0 : j;
  return c->mask[mb * (m[1] * m[2] * m[3]) + mh * (m[2] * m[3]) + ms * m[3] + mc];
}

/* Row i of head (b, h): scores[j] = softmax weights p_ij exactly as
 * cpu:2420-2458 (dot by mul_add over d, *scale, +mask, max with strict >,
 * exp and sequential sum, inv_sum = 1/(sum + 1e-9), p = e * inv_sum).
 * kT is K of this head transposed to [Dk][S] so the j loop vectorises; each
 * dot still runs d ascending. */
__attribute__((target_clones("fma", "default"))) static void att_probs(
    const att_ctx* c, int64_t b, int64_t h, int64_t i, const float* qrow, const float* kT, float* scores) {
  const int64_t S = c->S, Dk = c->Dk;
  const float scale = 1.0f / sqrtf((float)Dk);
  for (int64_t j = 0; j < S; ++j) scores[j] = 0.0f;
  for (int64_t d = 0; d < Dk; ++d) {
    const float qd = qrow[d];
    const float* kr = kT + d * S;
    for (int64_t j = 0; j < S; ++j) scores[j] = fmaf(qd, kr[j], scores[j]);
  }
  float mx = -INFINITY;
  for (int64_t j = 0; j < S; ++j) {
    float dot = scores[j] * scale;
    if (c->mask) dot += mask_at(c, b, h, i, j);
    scores[j] = dot;
    if (dot > mx) mx = dot;
  }
  float sum = 0.0f;
  for (int64_t j = 0; j < S; ++j) {
    scores[j] = expf(scores[j] - mx);
    sum += scores[j];
  }
  const float inv = 1.0f / (sum + 1e-9f);
  for (int64_t j = 0; j < S; ++j) scores[j] *= inv;
}

static void transpose_head(const float* src, int64_t S, int64_t Dk, float* dst) {
  for (int64_t j = 0; j < S; ++j)
    for (int64_t d = 0; d < Dk; ++d) dst[d * S + j] = src[j * Dk + d];
}

/* out[i][d] = sum_j p_ij.mul_add(v[j][d], .) for j ascending (cpu:2460-2468). */
__attribute__((target_clones("fma", "default"))) static void att_out_row(const float* p,
                                                                                const float* V, int64_t S,
                                                                                int64_t Dk, float* out) {
  for (int64_t d = 0; d < Dk; ++d) out[d] = 0.0f;
  for (int64_t j = 0; j < S; ++j) {
    const float pj = p[j];
    const float* vr = V + j * Dk;
    for (int64_t d = 0; d < Dk; ++d) out[d] = fmaf(pj, vr[d], out[d]);
  }
}

static void att_fwd_task(void* p, int64_t begin, int64_t end) {
  const att_ctx* c = (const att_ctx*)p;
  const int64_t S = c->S, Dk = c->Dk;
  float* kT = (float*)malloc((size_t)(S * Dk) * sizeof(float));
  float* scores = (float*)malloc((size_t)S * sizeof(float));
  for (int64_t bh = begin; bh < end; ++bh) {
    const int64_t b = bh / c->H, h = bh % c->H, off = bh * S * Dk;
    transpose_head(c->k + off, S, Dk, kT);
    for (int64_t i = 0; i < S; ++i) {
      att_probs(c, b, h, i, c->q + off + i * Dk, kT, scores);
      att_out_row(scores, c->v + off, S, Dk, c->out + off + i * Dk);
    }
  }
  free(kT);
  free(scores);
}

/* Backward for row i (cpu:2571-2613): dp_j = sum_d go[d].mul_add(v[j][d]);
 * s = sum_j dp_j.mul_add(p_j); ds_j = p_j * (dp_j - s);
 * dq[i][d] = (sum_j ds_j.mul_add(k[j][d])) * scale;
 * dv[j][d] = p_j.mul_add(go[d], dv[j][d]); dk[j][d] = (ds_j*scale).mul_add(q[d], dk[j][d]). */
__attribute__((target_clones("fma", "default"))) static void att_bwd_row(
    const float* p, const float* gorow, const float* qrow, const float* vT, const float* K, int64_t S,
    int64_t Dk, float scale, float* dp, float* dqrow, float* dK, float* dV) {
  for (int64_t j = 0; j < S; ++j) dp[j] = 0.0f;
  for (int64_t d = 0; d < Dk; ++d) {
    const float g = gorow[d];
    const float* vr = vT + d * S;
    for (int64_t j = 0; j < S; ++j) dp[j] = fmaf(g, vr[j], dp[j]);
  }
  float s = 0.0f;
  for (int64_t j = 0; j < S; ++j) s = fmaf(dp[j], p[j], s);
  for (int64_t j = 0; j < S; ++j) dp[j] = p[j] * (dp[j] - s); /* ds_j */
  for (int64_t d = 0; d < Dk; ++d) dqrow[d] = 0.0f;
  for (int64_t j = 0; j < S; ++j) {
    const float dsj = dp[j];
    const float* kr = K + j * Dk;
    for (int64_t d = 0; d < Dk; ++d) dqrow[d] = fmaf(dsj, kr[d], dqrow[d]);
  }
  for (int64_t d = 0; d < Dk; ++d) dqrow[d] *= scale;
  for (int64_t j = 0; j < S; ++j) {
    const float pj = p[j];
    float* dvr = dV + j * Dk;
    for (int64_t d = 0; d < Dk; ++d) dvr[d] = fmaf(pj, gorow[d], dvr[d]);
  }
  for (int64_t j = 0; j < S; ++j) {
    const float dsj = dp[j] * scale;
    float* dkr = dK + j * Dk;
    for (int64_t d = 0; d < Dk; ++d) dkr[d] = fmaf(dsj, qrow[d], dkr[d]);
  }
}

static void att_bwd_task(void* p, int64_t begin, int64_t end) {
  const att_ctx* c = (const att_ctx*)p;
  const int64_t S = c->S, Dk = c->Dk;
  const float scale = 1.0f / sqrtf((float)Dk);
  float* kT = (float*)malloc((size_t)(S * Dk) * sizeof(float));
  float* vT = (float*)malloc((size_t)(S * Dk) * sizeof(float));
  float* scores = (float*)malloc((size_t)S * sizeof(float));
  float* dp = (float*)malloc((size_t)S * sizeof(float));
  for (int64_t bh = begin; bh < end; ++bh) {
    const int64_t b = bh / c->H, h = bh % c->H, off = bh * S * Dk;
    transpose_head(c->k + off, S, Dk, kT);
    transpose_head(c->v + off, S, Dk, vT);
    for (int64_t x = 0; x < S * Dk; ++x) {
      c->dk[off + x] = 0.0f;
      c->dv[off + x] = 0.0f;
    }
    for (int64_t i = 0; i < S; ++i) {
      att_probs(c, b, h, i, c->q + off + i * Dk, kT, scores);
      att_bwd_row(scores, c->go + off + i * Dk, c->q + off + i * Dk, vT, c->k + off, S, Dk, scale, dp,
                  c->dq + off + i * Dk, c->dk + off, c->dv + off);
    }
  }
  free(kT);
  free(vT);
  free(scores);
  free(dp);
}

static void att_setup(att_ctx* c, const float* q, const float* k, const float* v, int64_t H, int64_t S,
                      int64_t Dk, const float* mask, const vo_layout* ml) {
  memset(c, 0, sizeof(*c));
  c->q = q;
  c->k = k;
  c->v = v;
  c->H = H;
  c->S = S;
  c->Dk = Dk;
  c->mask = mask;
  for (int i = 0; i < 4; ++i) c->mdims[i] = 1;
  if (mask && ml)
    for (int i = 0; i < ml->rank && i < 4; ++i) c->mdims[4 - ml->rank + i] = ml->dims[i];
}

int vo_fused_attention(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t S,
                       int64_t Dk, const float* mask, const vo_layout* ml, float* out) {
  att_ctx c;
  att_setup(&c, q, k, v, H, S, Dk, mask, ml);
  c.out = out;
  parallel_for(B * H, att_fwd_task, &c);
  return VO_OK;
}

int vo_fused_attention_backward(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                                int64_t S, int64_t Dk, const float* mask, const vo_layout* ml,
                                const float* go, float* dq, float* dk, float* dv) {
  att_ctx c;
  att_setup(&c, q, k, v, H, S, Dk, mask, ml);
  c.go = go;
  c.dq = dq;
  c.dk = dk;
  c.dv = dv;
  parallel_for(B * H, att_bwd_task, &c);
  return VO_OK;
}

/* ---------------------------------------------------- unfused attention -- */

static float* falloc(int64_t n);

/* [N][R][C] -> [N][C][R] (a transposed view made contiguous, as the CPU
 * matmul does with every operand, cpu:307-308). */
static void transpose_last2(const float* src, int64_t N, int64_t R, int64_t C, float* dst) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t r = 0; r < R; ++r)
      for (int64_t c = 0; c < C; ++c) dst[(n * C + c) * R + r] = src[(n * R + r) * C + c];
}

static void lay4(vo_layout* l, int64_t a, int64_t b, int64_t c, int64_t d) {
  const int64_t dims[4] = {a, b, c, d};
  vo_contiguous_layout(l, 4, dims);
}

/* The intermediates of the unfused path (nn:603-613): scores after the mask
 * (the Softmax node's saved input) and the probabilities. */
static int unfused_scores(const float* q, const float* k, int64_t B, int64_t H, int64_t S, int64_t Dk,
                          const float* mask, const vo_layout* ml, float* scores, float* probs, char* err,
                          size_t errlen) {
  const int64_t N = B * H;
  vo_layout lq, lkT, ls, lsc;
  lay4(&lq, B, H, S, Dk);
  lay4(&lkT, B, H, Dk, S);
  lay4(&ls, B, H, S, S);
  const int64_t one = 1;
  vo_contiguous_layout(&lsc, 1, &one);
  /* scale = Tensor::from_f32(&[1.0 / (d_k as f32).sqrt()], [1]) */
  const float scale = 1.0f / sqrtf((float)Dk);
  float* kT = falloc(N * Dk * S);
  float* raw = falloc(N * S * S);
  transpose_last2(k, N, S, Dk, kT); /* k.transpose(2, 3) */
  int rc = vo_matmul(q, &lq, kT, &lkT, raw, err, errlen);
  free(kT);
  if (rc == VO_OK) rc = vo_binary(2, raw, &ls, &scale, &lsc, mask ? raw : scores, &ls, err, errlen); /* .mul(&scale) */
  if (rc == VO_OK && mask) rc = vo_binary(0, raw, &ls, mask, ml, scores, &ls, err, errlen);         /* .add(m) */
  free(raw);
  if (rc == VO_OK) rc = vo_softmax(scores, &ls, 3, probs, err, errlen); /* .softmax(3) */
  return rc;
}

int vo_attention_unfused(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t S,
                         int64_t Dk, const float* mask, const vo_layout* ml, float* out, char* err, size_t errlen) {
  const int64_t N = B * H;
  vo_layout ls, lv;
  lay4(&ls, B, H, S, S);
  lay4(&lv, B, H, S, Dk);
  float* scores = falloc(N * S * S);
  float* probs = falloc(N * S * S);
  int rc = unfused_scores(q, k, B, H, S, Dk, mask, ml, scores, probs, err, errlen);
  free(scores);
  if (rc == VO_OK) rc = vo_matmul(probs, &ls, v, &lv, out, err, errlen); /* probs.matmul(&v) */
  free(probs);
  return rc;
}

/* The tape of the unfused path walked back (autograd:429-760): the Matmul arm
 * of probs.matmul(v) (autograd:503-515: go.matmul(v^T), probs^T.matmul(go)),
 * the Softmax arm on the saved scores (547-553), the Add arm (the mask's
 * share is dropped: the mask needs no gradient), the Mul arm (go.mul(scale)),
 * the Matmul arm of q.matmul(k^T) and the Transpose arm back to k's layout. */
int vo_attention_unfused_backward(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                                  int64_t S, int64_t Dk, const float* mask, const vo_layout* ml, const float* go,
                                  float* dq, float* dk, float* dv, char* err, size_t errlen) {
  const int64_t N = B * H;
  vo_layout ls, lv, lvT, lkT, lsc;
  lay4(&ls, B, H, S, S);
  lay4(&lv, B, H, S, Dk);
  lay4(&lvT, B, H, Dk, S);
  lay4(&lkT, B, H, Dk, S);
  const int64_t one = 1;
  vo_contiguous_layout(&lsc, 1, &one);
  const float scale = 1.0f / sqrtf((float)Dk);
  float* scores = falloc(N * S * S);
  float* probs = falloc(N * S * S);
  float *tmp = NULL, *g = NULL, *gs = NULL;
  int rc = unfused_scores(q, k, B, H, S, Dk, mask, ml, scores, probs, err, errlen);
  if (rc != VO_OK) goto out;
  /* probs.matmul(v): d probs = go.matmul(v^T), dv = probs^T.matmul(go).
   * tmp holds [S, S] or [Dk, S] blocks: v^T, probs^T, then (as gs) the
   * scores' gradient and k_t's. */
  tmp = falloc(N * S * (S > Dk ? S : Dk));
  g = falloc(N * S * S);
  transpose_last2(v, N, S, Dk, tmp);
  rc = vo_matmul(go, &lv, tmp, &lvT, g, err, errlen);
  if (rc != VO_OK) goto out;
  transpose_last2(probs, N, S, S, tmp);
  rc = vo_matmul(tmp, &ls, go, &lv, dv, err, errlen);
  if (rc != VO_OK) goto out;
  free(probs);
  probs = NULL;
  /* Softmax arm on the saved input, then the Add arm (identity for scores). */
  gs = tmp;
  tmp = NULL;
  rc = vo_softmax_backward_composite(scores, g, &ls, 3, gs, err, errlen);
  if (rc != VO_OK) goto out;
  /* Mul arm: d raw = d scores .mul(scale) */
  rc = vo_binary(2, gs, &ls, &scale, &lsc, g, &ls, err, errlen);
  if (rc != VO_OK) goto out;
  /* q.matmul(k_t): dq = g.matmul(k_t^T = k), d k_t = q^T.matmul(g) */
  rc = vo_matmul(g, &ls, k, &lv, dq, err, errlen);
  if (rc != VO_OK) goto out;
  tmp = falloc(N * Dk * S);
  transpose_last2(q, N, S, Dk, tmp);
  rc = vo_matmul(tmp, &lkT, g, &ls, gs, err, errlen); /* [B, H, Dk, S] into gs's storage */
  if (rc != VO_OK) goto out;
  transpose_last2(gs, N, Dk, S, dk); /* Transpose arm: back to [B, H, S, Dk] */
out:
  free(scores);
  free(probs);
  free(tmp);
  free(g);
  free(gs);
  return rc;
}

/* ---------------------------------------------------------------- AdamW -- */

/* f32::powi(t) lowers to compiler-rt's __powisf2: binary exponentiation. */
static float powi_f32(float a, int b) {
  const int recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

/* tensor:967-986 (CPU branch), one parameter tensor. */
void vo_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, int t, float lr, float beta1,
                   float beta2, float eps, float wd) {
  const float bc1 = 1.0f - powi_f32(beta1, t);
  const float bc2 = 1.0f - powi_f32(beta2, t);
  for (int64_t i = 0; i < n; ++i) {
    const float gi = g[i];
    m[i] = beta1 * m[i] + (1.0f - beta1) * gi;
    v[i] = beta2 * v[i] + (1.0f - beta2) * gi * gi;
    const float m_hat = m[i] / bc1;
    const float v_hat = v[i] / bc2;
    p[i] -= lr * wd * p[i];
    p[i] -= lr * m_hat / (sqrtf(v_hat) + eps);
  }
}

/* ------------------------------------------------------- SimpleGPT step -- */

void vo_gpt_param_numel(const vo_gpt_config* c, int64_t* n) {
  const int64_t D = c->D, F = c->F;
  const int64_t sz[VO_GPT_NPARAMS] = {c->V * D, c->P * D, D, D, D * D, D, D * D, D, D * D, D, D * D, D,
                                      D,        D,        F * D, F, D * F, D, D, D, c->V * D};
  for (int i = 0; i < VO_GPT_NPARAMS; ++i) n[i] = sz[i];
}

static float* falloc(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

static void transpose2(const float* src, int64_t R, int64_t C, float* dst) {
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) dst[c * R + r] = src[r * C + c];
}

/* Linear::forward (nn:120-128): out = x.matmul(W^T) (+ bias, a broadcast add
 * after the matmul, cpu:160-202). x is [R, Din] (rank 3 inputs give the same
 * rows: each output row depends only on its input row). */
static void linear_fwd(const float* x, int64_t R, int64_t Din, const float* W, int64_t Dout, const float* bias,
                       float* out) {
  float* Wt = falloc(Din * Dout);
  transpose2(W, Dout, Din, Wt);
  matmul2(x, Wt, out, R, Dout, Din);
  free(Wt);
  if (bias)
    for (int64_t r = 0; r < R; ++r)
      for (int64_t c = 0; c < Dout; ++c) out[r * Dout + c] = out[r * Dout + c] + bias[c];
}

/* Backward of Linear through the unchanged autograd: the Add arm
 * (autograd:460-469) gives db = reduce_to(dy, [Dout]) (sequential over rows,
 * autograd:316-361); the Matmul arm (autograd:502-519) gives
 * dx = dy.matmul(W) and dW^T = x^T.matmul(dy), the latter batched over the
 * leading dim of a rank-3 x ([Bt, Din, S] x [Bt, S, Dout]) and reduce_to'd
 * over it in batch order; the Transpose arm hands dW = (dW^T)^T to the
 * weight. Bt = 1 for the rank-2 lm_head input. */
static void linear_bwd(const float* x, int64_t Bt, int64_t S, int64_t Din, const float* W, int64_t Dout,
                       const float* dy, float* dx, float* dW, float* db) {
  const int64_t R = Bt * S;
  if (db) {
    for (int64_t c = 0; c < Dout; ++c) db[c] = 0.0f;
    for (int64_t r = 0; r < R; ++r)
      for (int64_t c = 0; c < Dout; ++c) db[c] += dy[r * Dout + c];
  }
  if (dx) matmul2(dy, W, dx, R, Din, Dout);
  float* xT = falloc(R * Din);
  for (int64_t b = 0; b < Bt; ++b) transpose2(x + b * S * Din, S, Din, xT + b * S * Din);
  float* gT = falloc(Bt * Din * Dout);
  int64_t* aoff = (int64_t*)calloc((size_t)Bt, sizeof(int64_t));
  int64_t* boff = (int64_t*)calloc((size_t)Bt, sizeof(int64_t));
  for (int64_t b = 0; b < Bt; ++b) {
    aoff[b] = b * Din * S;
    boff[b] = b * S * Dout;
  }
  matmul_batched(xT, dy, gT, Bt, aoff, boff, Din, Dout, S);
  /* reduce_to over the batch dim: out starts at 0.0, batches added in order. */
  float* red = gT;
  if (Bt > 1) {
    red = falloc(Din * Dout);
    for (int64_t b = 0; b < Bt; ++b)
      for (int64_t e = 0; e < Din * Dout; ++e) red[e] += gT[b * Din * Dout + e];
  }
  transpose2(red, Din, Dout, dW);
  if (red != gT) free(red);
  free(gT);
  free(xT);
  free(aoff);
  free(boff);
}

static void add_into(float* dst, const float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = a[i] + b[i];
}

/* [B, S, H, Dk] (a reshape of [B, S, D]) -> [B, H, S, Dk] contiguous, i.e.
 * reshape + transpose(1, 2) + contiguous (nn:585-588, cpu fused_attention's
 * q.contiguous()); `back` does the inverse (nn:601). */
static void heads_split(const float* src, int64_t B, int64_t S, int64_t H, int64_t Dk, float* dst, int back) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t s = 0; s < S; ++s)
      for (int64_t h = 0; h < H; ++h)
        for (int64_t d = 0; d < Dk; ++d) {
          const int64_t a = ((b * S + s) * H + h) * Dk + d, t = ((b * H + h) * S + s) * Dk + d;
          if (back)
            dst[a] = src[t];
          else
            dst[t] = src[a];
        }
}

#define TRY(x)              \
  do {                      \
    int rc_ = (x);          \
    if (rc_) goto done;     \
  } while (0)

int vo_gpt_step(const vo_gpt_config* cfg, const float* const* P, const float* ids, const float* targets,
                float* loss, float* const* G, char* err, size_t errlen) {
  return vo_gpt_step_ex(cfg, P, ids, targets, 0, loss, G, err, errlen);
}

int vo_gpt_step_ex(const vo_gpt_config* cfg, const float* const* P, const float* ids, const float* targets,
                   int unfused, float* loss, float* const* G, char* err, size_t errlen) {
  const int64_t B = cfg->B, S = cfg->S, D = cfg->D, H = cfg->H, F = cfg->F, V = cfg->V;
  const int64_t R = B * S, Dk = D / H;
  const float eps = 1e-5f;
  int rc = VO_OK;
  vo_layout lid, lrd, lrv, ld, lwte, lwpe, lmask, ltg;
  const int64_t d_bs[2] = {B, S}, d_rd[2] = {R, D}, d_rf[2] = {R, F}, d_rv[2] = {R, V}, d_d[1] = {D},
                d_wte[2] = {V, D}, d_wpe[2] = {cfg->P, D}, d_m[2] = {S, S}, d_r[1] = {R};
  vo_contiguous_layout(&lid, 2, d_bs);
  vo_contiguous_layout(&lrd, 2, d_rd);
  vo_contiguous_layout(&lrv, 2, d_rv);
  vo_contiguous_layout(&ld, 1, d_d);
  vo_contiguous_layout(&lwte, 2, d_wte);
  vo_contiguous_layout(&lwpe, 2, d_wpe);
  vo_contiguous_layout(&lmask, 2, d_m);
  vo_contiguous_layout(&ltg, 1, d_r);

  /* Forward (nn:745-791 and nn:666-675). */
  float *pos = falloc(R), *tok = falloc(R * D), *pe = falloc(R * D), *h0 = falloc(R * D), *ln1 = falloc(R * D);
  float *q = falloc(R * D), *k = falloc(R * D), *v = falloc(R * D), *qh = falloc(R * D), *kh = falloc(R * D);
  float *vh = falloc(R * D), *atth = falloc(R * D), *att = falloc(R * D), *o = falloc(R * D), *h1 = falloc(R * D);
  float *ln2 = falloc(R * D), *f1 = falloc(R * F), *g = falloc(R * F), *f2 = falloc(R * D), *h2 = falloc(R * D);
  float *lnf = falloc(R * D), *logits = falloc(R * V), *mask = falloc(S * S);
  float *dlogits = NULL, *d1 = NULL, *d2 = NULL, *dh1 = NULL, *dh0 = NULL, *dF = NULL, *dF2 = NULL;
  float *dqh = NULL, *dkh = NULL, *dvh = NULL, *dq = NULL, *dk = NULL, *dv = NULL, *datth = NULL, *tmp = NULL;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t s = 0; s < S; ++s) pos[b * S + s] = (float)s;
  for (int64_t i = 0; i < S; ++i)
    for (int64_t j = 0; j < S; ++j) mask[i * S + j] = j > i ? -1e9f : 0.0f;

  TRY(rc = vo_embedding(ids, &lid, P[VO_P_WTE], &lwte, tok, err, errlen));
  TRY(rc = vo_embedding(pos, &lid, P[VO_P_WPE], &lwpe, pe, err, errlen));
  add_into(h0, tok, pe, R * D);
  TRY(rc = vo_layernorm(h0, &lrd, P[VO_P_LN1_W], &ld, P[VO_P_LN1_B], &ld, eps, ln1, err, errlen));
  linear_fwd(ln1, R, D, P[VO_P_Q_W], D, P[VO_P_Q_B], q);
  linear_fwd(ln1, R, D, P[VO_P_K_W], D, P[VO_P_K_B], k);
  linear_fwd(ln1, R, D, P[VO_P_V_W], D, P[VO_P_V_B], v);
  heads_split(q, B, S, H, Dk, qh, 0);
  heads_split(k, B, S, H, Dk, kh, 0);
  heads_split(v, B, S, H, Dk, vh, 0);
  if (unfused)
    TRY(rc = vo_attention_unfused(qh, kh, vh, B, H, S, Dk, mask, &lmask, atth, err, errlen));
  else
    vo_fused_attention(qh, kh, vh, B, H, S, Dk, mask, &lmask, atth);
  heads_split(atth, B, S, H, Dk, att, 1);
  linear_fwd(att, R, D, P[VO_P_O_W], D, P[VO_P_O_B], o);
  add_into(h1, h0, o, R * D);
  TRY(rc = vo_layernorm(h1, &lrd, P[VO_P_LN2_W], &ld, P[VO_P_LN2_B], &ld, eps, ln2, err, errlen));
  linear_fwd(ln2, R, D, P[VO_P_FC1_W], F, P[VO_P_FC1_B], f1);
  {
    vo_layout lg;
    vo_contiguous_layout(&lg, 2, d_rf);
    vo_gelu(f1, &lg, g);
  }
  linear_fwd(g, R, F, P[VO_P_FC2_W], D, P[VO_P_FC2_B], f2);
  add_into(h2, h1, f2, R * D);
  TRY(rc = vo_layernorm(h2, &lrd, P[VO_P_LNF_W], &ld, P[VO_P_LNF_B], &ld, eps, lnf, err, errlen));
  linear_fwd(lnf, R, D, P[VO_P_LM_W], V, NULL, logits);
  TRY(rc = vo_cross_entropy(logits, &lrv, targets, &ltg, loss, err, errlen));
  if (!G) goto done;

  /* Backward in reverse tape order (autograd:429-760). */
  {
    const float one = 1.0f;
    dlogits = falloc(R * V);
    TRY(rc = vo_cross_entropy_backward(logits, &lrv, targets, &ltg, &one, 1, dlogits, err, errlen));
  }
  free(logits);
  logits = NULL;
  d1 = falloc(R * D);
  linear_bwd(lnf, 1, R, D, P[VO_P_LM_W], V, dlogits, d1, G[VO_P_LM_W], NULL);
  free(dlogits);
  dlogits = NULL;
  dh1 = falloc(R * D); /* grad of h2 first */
  TRY(rc = vo_layernorm_backward(h2, &lrd, P[VO_P_LNF_W], &ld, &ld, d1, &lrd, eps, dh1, G[VO_P_LNF_W],
                                 G[VO_P_LNF_B], err, errlen));
  /* h2 = h1 + f2: h1's grad starts as dh2 (clone), f2's grad is dh2. */
  dF = falloc(R * F);
  dF2 = falloc(R * F);
  linear_bwd(g, B, S, F, P[VO_P_FC2_W], D, dh1, dF, G[VO_P_FC2_W], G[VO_P_FC2_B]);
  vo_gelu_grad_mask(f1, R * F, dF2);
  for (int64_t i = 0; i < R * F; ++i) dF[i] = dF[i] * dF2[i];
  d2 = falloc(R * D);
  linear_bwd(ln2, B, S, D, P[VO_P_FC1_W], F, dF, d2, G[VO_P_FC1_W], G[VO_P_FC1_B]);
  tmp = falloc(R * D);
  TRY(rc = vo_layernorm_backward(h1, &lrd, P[VO_P_LN2_W], &ld, &ld, d2, &lrd, eps, tmp, G[VO_P_LN2_W],
                                 G[VO_P_LN2_B], err, errlen));
  for (int64_t i = 0; i < R * D; ++i) dh1[i] = dh1[i] + tmp[i];
  /* h1 = h0 + o: h0's grad starts as dh1, o's grad is dh1. */
  linear_bwd(att, B, S, D, P[VO_P_O_W], D, dh1, d2, G[VO_P_O_W], G[VO_P_O_B]);
  datth = falloc(R * D);
  heads_split(d2, B, S, H, Dk, datth, 0);
  dqh = falloc(R * D);
  dkh = falloc(R * D);
  dvh = falloc(R * D);
  if (unfused)
    TRY(rc = vo_attention_unfused_backward(qh, kh, vh, B, H, S, Dk, mask, &lmask, datth, dqh, dkh, dvh, err,
                                           errlen));
  else
    vo_fused_attention_backward(qh, kh, vh, B, H, S, Dk, mask, &lmask, datth, dqh, dkh, dvh);
  dq = falloc(R * D);
  dk = falloc(R * D);
  dv = falloc(R * D);
  heads_split(dqh, B, S, H, Dk, dq, 1);
  heads_split(dkh, B, S, H, Dk, dk, 1);
  heads_split(dvh, B, S, H, Dk, dv, 1);
  /* v, then k, then q (reverse tape order); ln1's grad accumulates by add. */
  dh0 = falloc(R * D);
  linear_bwd(ln1, B, S, D, P[VO_P_V_W], D, dv, d1, G[VO_P_V_W], G[VO_P_V_B]);
  linear_bwd(ln1, B, S, D, P[VO_P_K_W], D, dk, tmp, G[VO_P_K_W], G[VO_P_K_B]);
  for (int64_t i = 0; i < R * D; ++i) d1[i] = d1[i] + tmp[i];
  linear_bwd(ln1, B, S, D, P[VO_P_Q_W], D, dq, tmp, G[VO_P_Q_W], G[VO_P_Q_B]);
  for (int64_t i = 0; i < R * D; ++i) d1[i] = d1[i] + tmp[i];
  TRY(rc = vo_layernorm_backward(h0, &lrd, P[VO_P_LN1_W], &ld, &ld, d1, &lrd, eps, tmp, G[VO_P_LN1_W],
                                 G[VO_P_LN1_B], err, errlen));
  for (int64_t i = 0; i < R * D; ++i) dh0[i] = dh1[i] + tmp[i];
  /* h0 = tok + pe: both grads are dh0; the position embedding was recorded
   * after the token embedding, so its arm runs first (values independent). */
  {
    vo_layout lgo;
    const int64_t d_go[3] = {B, S, D};
    vo_contiguous_layout(&lgo, 3, d_go);
    TRY(rc = vo_embedding_backward(pos, &lid, &lwpe, dh0, &lgo, G[VO_P_WPE], err, errlen));
    TRY(rc = vo_embedding_backward(ids, &lid, &lwte, dh0, &lgo, G[VO_P_WTE], err, errlen));
  }

done:
  free(pos); free(tok); free(pe); free(h0); free(ln1); free(q); free(k); free(v); free(qh); free(kh);
  free(vh); free(atth); free(att); free(o); free(h1); free(ln2); free(f1); free(g); free(f2); free(h2);
  free(lnf); free(logits); free(mask); free(dlogits); free(d1); free(d2); free(dh1); free(dh0); free(dF);
  free(dF2); free(dqh); free(dkh); free(dvh); free(dq); free(dk); free(dv); free(datth); free(tmp);
  return rc;
}
