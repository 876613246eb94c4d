/*
 * vearo_hip.h -- C ABI of libvearo_hip.so, the MI355X (gfx950) backend for
 * vearo's fused layer kernels.
 *
 * This is the drop-in boundary: the entry points a `vearo-backend-hip` crate
 * binds with `extern "C"` to fill vearo's BackendOps table
 * (reference: crates/vearo-core/src/tensor.rs:1108-1175) and its storage hooks
 * (tensor.rs:1321-1363). All arguments are plain pointers, sizes and flags:
 *   - tensors are f32 device pointers (vh_alloc or any HIP device allocation);
 *     hot-path entries take contiguous row-major buffers; strided inputs go
 *     through vh_strided_copy first (the device replacement for the host
 *     round-trip in Tensor::contiguous, tensor.rs:345-486);
 *   - ids and targets are f32, as in the reference API (cpu lib.rs:892-899);
 *   - `stream` is a hipStream_t passed as void*; NULL selects the runtime's own
 *     stream (vh_stream()). Launches are asynchronous on that stream.
 * Every entry returns 0 on success or a VH_ERR_* code; vh_last_error() gives a
 * thread-local message. Nothing throws across the ABI. Zero-sized work returns
 * 0 without launching (the reference returns empty outputs, cpu lib.rs:669-672).
 *
 * Data the CPU backend would panic on (negative / out-of-range token ids and
 * targets, cpu lib.rs:893-905, 1015-1027) is caught on the device: the kernel
 * records the first offending element and vh_sync() / vh_check_device_error()
 * return VH_ERR_DEVICE_PANIC with the CPU backend's panic text.
 *
 * "cpu" below is crates/vearo-backend-cpu/src/lib.rs, "cuda" is
 * crates/vearo-backend-cuda/src/lib.rs, "autograd" is crates/vearo-autograd/src/lib.rs.
 */
#ifndef VEARO_HIP_H
#define VEARO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VH_OK 0
#define VH_ERR_INVALID 1       /* bad argument: shape, size, null pointer      */
#define VH_ERR_HIP 2           /* HIP runtime error                           */
#define VH_ERR_NOT_INIT 3      /* vh_init has not run                         */
#define VH_ERR_DEVICE_PANIC 4  /* a kernel met data the CPU backend panics on */
#define VH_ERR_UNSUPPORTED 5   /* size outside the implemented range          */
#define VH_ERR_OOM 6           /* device allocation failed                    */
#define VH_ERR_IO 7            /* a file could not be opened, read or written */

#define VH_MAX_RANK 8

/* dims + element strides, as vearo-core's Shape pair (shape.rs:8-12, rank <= 8). */
typedef struct {
  int32_t rank;
  int32_t pad_;
  int64_t dims[VH_MAX_RANK];
  int64_t strides[VH_MAX_RANK];
} vh_layout;

typedef struct {
  size_t live_bytes;    /* handed out and not yet freed                  */
  size_t cached_bytes;  /* held in the arena's free lists                */
  size_t peak_bytes;    /* high-water mark of live_bytes                 */
  size_t hip_bytes;     /* total obtained from hipMalloc                 */
} vh_mem_stats;

/* ------------------------------------------------------------- runtime -- */

/* Device init: select the GPU, create the stream, load the embedded gfx950
 * code object with hipModuleLoadData, zero the device error record.
 * Replaces cuda init (load_ptx + CudaDevice::new, cuda:165-242). Idempotent. */
int vh_init(int device);
/* Release the stream, module and every cached allocation. */
int vh_shutdown(void);
/* Thread-local text of the last failure (empty string if none). */
const char* vh_last_error(void);
/* The runtime's stream as a hipStream_t. */
void* vh_stream(void);
/* Number of compute units of the current device. */
int vh_device_cu_count(void);
/* Wait for the stream, then check the device error record. Replaces the
 * implicit sync of cuda's read hook (cuda:124-132). */
int vh_sync(void);
/* Check (and clear) the device error record; syncs the stream first. */
int vh_check_device_error(void);

/* -------------------------------------------------------------- memory -- */

/* Arena allocation over hipMalloc (size classes, cached free lists, 256-byte
 * alignment). zero != 0 fills with 0.0f on the stream, as the CUDA slot arena
 * zero-fills on reuse (cuda:41-112) and Tensor::zeros_on relies on
 * (tensor.rs:88-117). Replaces the alloc hook of register_cuda_hooks. */
int vh_alloc(size_t bytes, int zero, void** out);
/* Return a block to the arena (stream-ordered reuse). Replaces refcount_dec's
 * slot release (cuda:134-163). */
int vh_free(void* ptr);
/* Synchronous copies, ordered after the stream's queued work. Replace the
 * write (cuda:114-122) and read (cuda:124-132) hooks. */
int vh_h2d(void* dst, const void* src, size_t bytes);
int vh_d2h(void* dst, const void* src, size_t bytes);
/* Asynchronous device-to-device copy on `stream` (the regions must not
 * overlap). 16-byte aligned copies run the library's streaming copy kernel. */
int vh_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* out[i] = value for i < n (a fill kernel, never hipMemset). */
int vh_fill_f32(float* out, float value, int64_t n, void* stream);
/* Diagnostic, with no counterpart in the reference: y[i] = expf, logf or
 * tanhf of x[i] (which = VH_MATH_EXP / LOG / TANH), evaluated by the same
 * device functions the kernels call (softmax's and cross-entropy's exp,
 * cross-entropy's log, GELU's tanh), for tests that bound their rounding
 * against correctly rounded values and the C library's. */
#define VH_MATH_EXP 0
#define VH_MATH_LOG 1
#define VH_MATH_TANH 2
int vh_math_probe(int32_t which, const float* x, float* y, int64_t n, void* stream);
int vh_mem_stats_get(vh_mem_stats* out);
/* hipFree every cached (free) block. */
int vh_empty_cache(void);

/* ---------------------------------------------------- hot path: layernorm -- */

/* y = layernorm over the last dim C of x[rows, C] with weight w[C], bias b[C].
 * Replaces BackendOps.layernorm (tensor.rs:1133; cpu:665-740; cuda:1205-1261). */
int vh_layernorm_fwd(const float* x, const float* w, const float* b, float* y,
                     int64_t rows, int64_t C, float eps, void* stream);
/* dx[rows, C], dw[C], db[C] from x, w and upstream dy (bias enters only through
 * its shape in the reference). Deterministic, atomic-free dw/db.
 * Replaces BackendOps.layernorm_backward (tensor.rs:1135; cpu:742-858;
 * cuda:1263-1353). scratch may be NULL (the runtime uses its arena); otherwise
 * it must hold vh_layernorm_bwd_scratch_bytes(rows, C) bytes. */
int vh_layernorm_bwd(const float* x, const float* w, const float* dy, float* dx,
                     float* dw, float* db, int64_t rows, int64_t C, float eps,
                     void* scratch, size_t scratch_bytes, void* stream);
size_t vh_layernorm_bwd_scratch_bytes(int64_t rows, int64_t C);

/* Size of the device-resident scratch each GPU holds for the allocation-free
 * entry points (a file-scope device array, one copy per GPU for the life of
 * the process). */
#define VH_NOALLOC_SCRATCH_BYTES (4u << 20)

/* vh_layernorm_bwd with its dgamma/dbeta partials in the device-resident
 * scratch: no hipMalloc, no hipFree and no allocating library call, for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid it). No counterpart in the reference; the same
 * kernels and results as vh_layernorm_bwd. Returns VH_ERR_UNSUPPORTED when
 * vh_layernorm_bwd_scratch_bytes(rows, C) exceeds VH_NOALLOC_SCRATCH_BYTES
 * (e.g. [16384, 768] needs 1.5 MiB; C above 1024 with many rows does not fit).
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (different streams, or threads) race. */
int vh_layernorm_bwd_noalloc(const float* x, const float* w, const float* dy, float* dx,
                             float* dw, float* db, int64_t rows, int64_t C, float eps,
                             void* stream);

/* -------------------------------------------------------- hot path: gelu -- */

/* y = gelu(x) elementwise, tanh form. Replaces BackendOps.gelu (tensor.rs:1129;
 * cpu:456-497; cuda unary_op + gelu_forward, cuda:1108-1140). */
int vh_gelu_fwd(const float* x, float* y, int64_t n, void* stream);
/* y[r, c] = gelu(x[r, c] + bias[c]): the Linear bias add (nn lib.rs:120-128 ->
 * BackendOps.add, cpu:160-202) fused with BackendOps.gelu. */
int vh_gelu_bias_fwd(const float* x, const float* bias, float* y, int64_t rows,
                     int64_t C, void* stream);
/* dx = dy * gelu'(x): the autograd Gelu arm (autograd:542-546) -- host-side
 * gelu_grad_mask (autograd:383-403) then BackendOps.mul -- as one kernel. */
int vh_gelu_grad_mul(const float* x, const float* dy, float* dx, int64_t n,
                     void* stream);
/* dx = dy * gelu'(x + bias) and dbias = column sums of dx: the Gelu arm plus the
 * Add arm's host reduce_to for the bias (autograd:460-469, 316-361), fused.
 * scratch: NULL or vh_gelu_bias_bwd_scratch_bytes(rows, C) bytes. */
int vh_gelu_bias_bwd(const float* x, const float* bias, const float* dy, float* dx,
                     float* dbias, int64_t rows, int64_t C, void* scratch,
                     size_t scratch_bytes, void* stream);
size_t vh_gelu_bias_bwd_scratch_bytes(int64_t rows, int64_t C);

/* ----------------------------------------------------- hot path: softmax -- */

/* y = softmax over rows of length T of x[rows, T]. causal != 0 declares the
 * rows to be T x T score blocks whose entries j > (row % T) are masked (-inf or
 * a large negative additive mask): they are not read and y there is 0, which
 * is the reference's exact result for such inputs. Replaces BackendOps.softmax
 * (tensor.rs:1131; cpu:499-563; cuda:1142-1203) on the last dim. */
int vh_softmax_fwd(const float* x, float* y, int64_t rows, int64_t T, int causal,
                   void* stream);
/* dx = y * (dy - sum(dy * y)) per row: the autograd Softmax arm
 * (autograd:547-553: softmax, mul, sum, sub, mul) as one kernel. input_is_x != 0
 * means `in` is the saved input x (y is recomputed in registers, as the arm
 * does); otherwise `in` is y. */
int vh_softmax_bwd(const float* in, const float* dy, float* dx, int64_t rows,
                   int64_t T, int input_is_x, int causal, void* stream);

/* --------------------------------------------------- hot path: embedding -- */

/* out[i, :] = W[round(ids[i]), :] for i < n; W is [V, D]. Bit-exact copy.
 * Replaces BackendOps.embedding (tensor.rs:1137; cpu:860-918; cuda:1355-1410). */
int vh_embedding_fwd(const float* ids, const float* W, float* out, int64_t n,
                     int64_t V, int64_t D, void* stream);
/* dW[V, D] = dense scatter-add of dy[n, D] by token, written in full (rows no
 * token hits are 0). No float atomics, deterministic. Rows of tokens with at
 * most 16 hits are summed in the CPU loop's exact order (bit-exact); rows of
 * tokens with more hits are summed in position chunks of ~32 hits combined in
 * chunk order. Replaces BackendOps.embedding_backward (tensor.rs:1139;
 * cpu:920-980; cuda:1412-1464).
 * scratch: NULL or vh_embedding_bwd_scratch_bytes(n, V, D) bytes. */
int vh_embedding_bwd(const float* ids, const float* dy, float* dW, int64_t n,
                     int64_t V, int64_t D, void* scratch, size_t scratch_bytes,
                     void* stream);
size_t vh_embedding_bwd_scratch_bytes(int64_t n, int64_t V, int64_t D);

/* ----------------------------------------------- hot path: cross-entropy -- */

/* loss[0] = mean over B rows of -log_softmax(logits[b])[target[b]];
 * logits [B, V], targets [B] f32. Replaces BackendOps.cross_entropy
 * (tensor.rs:1141; cpu:982-1051; cuda:1466-1534).
 * scratch: NULL or vh_cross_entropy_fwd_scratch_bytes(B) bytes. */
int vh_cross_entropy_fwd(const float* logits, const float* targets, float* loss,
                         int64_t B, int64_t V, void* scratch, size_t scratch_bytes,
                         void* stream);
size_t vh_cross_entropy_fwd_scratch_bytes(int64_t B);
/* dlogits[B, V] = go * (softmax(logits) - onehot(target)) / B, with go the
 * device scalar grad_out[0]. Replaces BackendOps.cross_entropy_backward
 * (tensor.rs:1143; cpu:1053-1127; cuda:1536-1592). */
int vh_cross_entropy_bwd(const float* logits, const float* targets,
                         const float* grad_out, float* dlogits, int64_t B, int64_t V,
                         void* stream);
/* The same with a row stride ld >= V for logits and dlogits (a rank-2 view
 * with unit column stride, as the reference's CPU path accepts any strides).
 * The backward writes only the first V columns of each dlogits row. */
int vh_cross_entropy_fwd_ld(const float* logits, int64_t ld, const float* targets,
                            float* loss, int64_t B, int64_t V, void* scratch,
                            size_t scratch_bytes, void* stream);
int vh_cross_entropy_bwd_ld(const float* logits, int64_t ld, const float* targets,
                            const float* grad_out, float* dlogits, int64_t B, int64_t V,
                            void* stream);
/* The forward above that also keeps, per row b, row_stats[2b] = max_c logits[b, c]
 * and row_stats[2b + 1] = sum_c exp(logits[b, c] - that max) (row_stats: [B, 2]
 * floats, 8-byte aligned) -- the two values the reference's backward recomputes
 * from the logits (cpu:1102-1114). Loss as vh_cross_entropy_fwd_ld. Replaces
 * BackendOps.cross_entropy (tensor.rs:1141; cpu:982-1051) for a caller that keeps
 * per-row state between its forward and backward (autograd's saved tensors).
 * scratch: NULL or vh_cross_entropy_fwd_scratch_bytes(B) bytes. */
int vh_cross_entropy_fwd_rs_ld(const float* logits, int64_t ld, const float* targets,
                               float* loss, float* row_stats, int64_t B, int64_t V,
                               void* scratch, size_t scratch_bytes, void* stream);
/* Backward from those statistics: one streaming pass, no reduction. dlogits has
 * the same bits as vh_cross_entropy_bwd_ld's when row_stats came from
 * vh_cross_entropy_fwd_rs_ld on the same logits, V and ld; dlogits may alias
 * logits. Replaces BackendOps.cross_entropy_backward (tensor.rs:1143;
 * cpu:1053-1127) for that caller. Grid: B * ceil((V / 4 + 1) / 512) workgroups
 * when logits and dlogits are 16-byte aligned, else B * ceil(V / 4096); at most
 * INT32_MAX. */
int vh_cross_entropy_bwd_rs_ld(const float* logits, int64_t ld, const float* targets,
                               const float* row_stats, const float* grad_out, float* dlogits,
                               int64_t B, int64_t V, void* stream);
/* Forward and backward in one read of the logits, for a caller that knows
 * grad_out before running the forward (the training step: the seed gradient of
 * loss.backward() is 1, autograd:795-798). Same loss and dlogits as
 * vh_cross_entropy_fwd_ld followed by vh_cross_entropy_bwd_ld.
 * scratch: NULL or vh_cross_entropy_fwd_scratch_bytes(B) bytes. */
int vh_cross_entropy_fwd_bwd_ld(const float* logits, int64_t ld, const float* targets,
                                const float* grad_out, float* loss, float* dlogits, int64_t B,
                                int64_t V, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------- composites the autograd arms drive -- */

#define VH_OP_ADD 0
#define VH_OP_SUB 1
#define VH_OP_MUL 2
#define VH_OP_DIV 3

/* out = l (op) r with NumPy broadcasting over strided operands; out is
 * contiguous with the broadcast shape. Replaces BackendOps.add/sub/mul/div
 * (tensor.rs:1113-1119; cpu:160-238; cuda binary_op, cuda:832-899) -- the
 * layouts travel as kernel arguments, not as a per-call H2D info array. */
int vh_binary(int op, const float* l, const vh_layout* ll, const float* r,
              const vh_layout* rl, float* out, void* stream);
/* Sum (mean != 0: mean) of x over axis `dim`; out is contiguous with the
 * reduced shape (keep_dim only changes the shape, not the data). Replaces
 * BackendOps.sum / mean (tensor.rs:1125-1127; cpu:566-653; cuda:1012-1090). */
int vh_reduce(int mean, const float* x, const vh_layout* xl, int dim, float* out,
              void* stream);
/* dst (contiguous) = src read through its layout. Device replacement for the
 * host round-trip of Tensor::contiguous (tensor.rs:349-368). */
int vh_strided_copy(const float* src, const vh_layout* sl, float* dst, void* stream);

/* Sum of the rows of x[rows, C] into out[C]: the reduce_to of a [rows, C]
 * gradient onto a broadcast [C] bias (autograd:316-361, run on the host there).
 * Fixed grouping (per-workgroup row chains, then a fixed-order column sum):
 * deterministic, within f32 rounding of the CPU's single chain.
 * scratch: NULL or vh_sum_rows_scratch_bytes(rows, C) bytes. */
int vh_sum_rows(const float* x, int64_t rows, int64_t C, float* out, void* scratch,
                size_t scratch_bytes, void* stream);
size_t vh_sum_rows_scratch_bytes(int64_t rows, int64_t C);

/* ------------------------------- config[4] block step: matmul and attention -- */

/* vh_gemm_desc.causal: the structure of an attention score block. Skipped
 * parts are exactly zero (or never read), so no result changes. */
#define VH_GEMM_DENSE 0
#define VH_GEMM_SKIP_UPPER 1 /* C[m, n] with n > m is not needed (tiles above the diagonal are skipped) */
#define VH_GEMM_K_LE_M 2     /* A[m, k] == 0 for k > m (M == K) */
#define VH_GEMM_K_GE_M 3     /* A[m, k] == 0 for k < m (M == K) */

/* vh_gemm_desc.engine: which kernels carry the product. The default is this
 * library's own matrix-core kernels, chosen by shape (large dense unbatched
 * products: the persistent 256-row-tile kernel; everything else: the tiled
 * kernel, split along K where the output alone cannot fill the chip). TILED
 * forces the tiled kernel (tests of its split-K path); LIBRARY hands the
 * dense unbatched products hipBLASLt supports to it (an A/B reference for
 * benchmarks) and runs the rest as DEFAULT; WIDE is DEFAULT with the
 * persistent kernel's 256 x 256 tile wherever that kernel runs (tests of the
 * tile DEFAULT picks only for long k loops over many tiles). No counterpart
 * in the reference. */
#define VH_GEMM_ENGINE_DEFAULT 0
#define VH_GEMM_ENGINE_TILED 1
#define VH_GEMM_ENGINE_LIBRARY 2
#define VH_GEMM_ENGINE_WIDE 3

/* C[m, n] = (C[m, n] +) alpha * sum_k A[m, k] B[k, n] (+ E[m, n]) over two batch
 * dims, on the f32 matrix cores. The epilogue order is v = acc*alpha;
 * v = v + E; v = C + v, i.e. the separate scale / mask / bias-add / gradient
 * accumulation ops the reference applies after its matmul. */
typedef struct vh_gemm_desc {
  int64_t M, N, K;
  const float* a;
  int64_t a_sm, a_sk; /* A[m, k] = a[m*a_sm + k*a_sk]; a_sm == 1 or a_sk == 1 */
  const float* b;
  int64_t b_sk, b_sn; /* B[k, n] = b[k*b_sk + n*b_sn]; b_sk == 1 or b_sn == 1 */
  float* c;
  int64_t c_sm;       /* C[m, n] = c[m*c_sm + n] */
  int64_t batch[2];   /* batch dims (1 when unused) */
  int64_t a_sb[2], b_sb[2], c_sb[2]; /* batch strides (0 broadcasts) */
  const float* e;     /* optional addend, NULL for none */
  int64_t e_sm, e_sn;
  int64_t e_sb[2];
  float alpha;
  int32_t accumulate; /* 1: add into C */
  int32_t causal;     /* VH_GEMM_* */
  int32_t engine;     /* VH_GEMM_ENGINE_* (0 in a zero-initialised descriptor) */
} vh_gemm_desc;
int vh_gemm(const vh_gemm_desc* d, void* stream);
/* Which kernels carried the calling thread's last successful vh_gemm (the main
 * product; a ragged K tail of the persistent kernel runs on the tiled one):
 * VH_GEMM_PATH_* (0 before any call, or for an empty product). A diagnostic
 * for tests and benchmarks, no counterpart in the reference. */
#define VH_GEMM_PATH_NONE 0
#define VH_GEMM_PATH_TILED 1       /* 128-row tiles, one pass over K */
#define VH_GEMM_PATH_SPLIT_K 2     /* 128-row tiles over K ranges + fixed-order reduce */
#define VH_GEMM_PATH_PERSISTENT 3  /* persistent 256 x 192 tiles, stream-K last round */
#define VH_GEMM_PATH_LIBRARY 4     /* hipBLASLt */
#define VH_GEMM_PATH_BATCHED 5     /* persistent walk over batched short-K products */
int vh_gemm_last_path(void);

/* out = lhs @ rhs with broadcast batch dims; any strides (operands with no
 * unit stride in their last two dims are copied first, as the reference makes
 * both contiguous); out is contiguous [batch..., M, N]. Replaces
 * BackendOps.matmul (tensor.rs:1121, 1475-1495; cpu:266-417; cuda:914-1010). */
int vh_matmul(const float* lhs, const vh_layout* ll, const float* rhs,
              const vh_layout* rl, float* out, void* stream);

/* Scaled dot-product attention over [B, H, S, Dk] layouts (any strides, unit
 * stride on Dk): out = softmax(q k^T / sqrt(Dk) + mask) v, with the CPU fused
 * kernel's normalisation p = e * (1/(sum + 1e-9)). mask: NULL or any layout that
 * broadcasts right-aligned to [B, H, S, S] (additive). causal = 0 computes
 * every block; causal = 1 declares that keys past the query are masked (as the
 * model's -1e9 upper triangle does), which skips their work; it may be
 * combined with a mask. causal = VH_ATTN_CAUSAL_AUTO (2) decides on the
 * device, with no host wait: one pass over the mask and operands (the test of
 * vh_attention_mask_is_causal) sets a flag that the launches read, so the
 * masked blocks are skipped exactly when that gives the dense form's bits
 * (without a mask AUTO is causal = 0). Replaces
 * BackendOps.fused_attention / fused_attention_backward (tensor.rs:1172-1174,
 * 1709-1739; cpu:2366-2630; the CUDA backend runs these on the CPU,
 * cuda:1595-1636). The backward recomputes the probabilities from q and k as
 * the reference does. scratch: NULL or
 * vh_fused_attention_scratch_bytes(B, H, S, backward) bytes (the score block). */
#define VH_ATTN_CAUSAL_AUTO 2
int vh_fused_attention_fwd(const float* q, const vh_layout* ql, const float* k,
                           const vh_layout* kl, const float* v, const vh_layout* vl,
                           const float* mask, const vh_layout* ml, int causal, float* out,
                           const vh_layout* ol, void* scratch, size_t scratch_bytes,
                           void* stream);
int vh_fused_attention_bwd(const float* q, const vh_layout* ql, const float* k,
                           const vh_layout* kl, const float* v, const vh_layout* vl,
                           const float* mask, const vh_layout* ml, int causal,
                           const float* dout, const vh_layout* dol, float* dq,
                           const vh_layout* dql, float* dk, const vh_layout* dkl, float* dv,
                           const vh_layout* dvl, void* scratch, size_t scratch_bytes,
                           void* stream);
size_t vh_fused_attention_scratch_bytes(int64_t B, int64_t H, int64_t S, int backward);
/* Whether this call's additive mask may be dropped for causal = 1 with the
 * same results: *is_causal = 1 when the mask's last two dims are [S, S], its
 * entries on and below the diagonal are +-0 and those above are at most -1,
 * q, k, v (and dout, when not NULL) are finite, and the smallest masked |value|
 * exceeds twice the largest score the product can form (scale * Dk *
 * max|q| * max|k|) by enough that every masked exp() underflows to exactly 0
 * -- so the skipped blocks would have contributed exact zeros. One pass over
 * the operands and the mask on `stream`, then a host wait for the answer: the
 * call synchronizes `stream` and returns after it drains. On a stream under
 * graph capture (where that wait is not allowed) it launches nothing and
 * answers 0. No counterpart in the reference; the attention entries' causal =
 * VH_ATTN_CAUSAL_AUTO makes the same decision on the device instead. */
int vh_attention_mask_is_causal(const float* q, const vh_layout* ql, const float* k,
                                const vh_layout* kl, const float* v, const vh_layout* vl,
                                const float* dout, const vh_layout* dol, const float* mask,
                                const vh_layout* ml, int* is_causal, void* stream);
/* The backward from the probabilities the forward computed: a caller-supplied
 * forward scratch holds P [B, H, S, S] on return, and passing it here as P skips
 * recomputing it (same results as vh_fused_attention_bwd; P already carries the
 * mask). With causal = 1 the forward leaves the 128 x 128 tiles of P wholly
 * above the diagonal unwritten and this call does not read them. No
 * counterpart in the reference, whose backward always recomputes; for a
 * training step that keeps the forward's scratch alive.
 * scratch: NULL or vh_fused_attention_scratch_bytes(B, H, S, 0) bytes. */
int vh_fused_attention_bwd_probs(const float* P, const float* q, const vh_layout* ql,
                                 const float* k, const vh_layout* kl, const float* v,
                                 const vh_layout* vl, int causal, const float* dout,
                                 const vh_layout* dol, float* dq, const vh_layout* dql, float* dk,
                                 const vh_layout* dkl, float* dv, const vh_layout* dvl,
                                 void* scratch, size_t scratch_bytes, void* stream);

/* AdamW update of one parameter tensor in place, moments m and v in device
 * memory, step count t >= 1. Replaces Tensor::adamw_step (tensor.rs:931-1023,
 * whose device path copies the parameter to the host and back) with the same
 * operation order. */
int vh_adamw_step(float* param, const float* grad, float* m, float* v, int64_t n, int32_t t,
                  float lr, float beta1, float beta2, float eps, float weight_decay,
                  void* stream);
/* vh_adamw_step over `count` tensors (arrays of device pointers and sizes in
 * host memory) in as few launches as possible (up to 32 tensors per launch),
 * each element updated exactly as vh_adamw_step updates it. For an optimizer
 * that steps every parameter at once (AdamW::step's loop over parameters,
 * crates/vearo-optim/src/lib.rs:105-123); no counterpart entry in the
 * reference. */
int vh_adamw_step_multi(int count, float* const* params, const float* const* grads, float* const* ms,
                        float* const* vs, const int64_t* ns, int32_t t, float lr, float beta1, float beta2,
                        float eps, float weight_decay, void* stream);

/* --------------------------------------------- .ve checkpoints of device tensors -- */

/* The `.ve` weight checkpoint (crates/vearo/src/checkpoint.rs:9-33): u32 tensor
 * count, then per tensor u32 rank, u32 dims, u32 element count and the f32
 * data, all little-endian. tensors[i] is a device pointer with layout
 * layouts[i]; each must be contiguous (the reference's to_vec_f32 asserts it,
 * tensor.rs:751-755), and every dim and element count must fit a u32 (the
 * reference truncates silently; this returns VH_ERR_UNSUPPORTED). Data leaves
 * the device through two pinned staging buffers, so the file writes overlap
 * the copies. Queued work on `stream` that writes the tensors is waited for;
 * returns after the file is complete and closed. Replaces save_checkpoint. */
int vh_checkpoint_save(const char* path, int32_t n, const float* const* tensors,
                       const vh_layout* layouts, void* stream);

/* Reads a `.ve` checkpoint into n device tensors in order (checkpoint.rs:40-91),
 * with the reference's checks and texts, which vh_last_error() reports:
 *   count differs   -> VH_ERR_INVALID "Checkpoint tensor count does not match
 *                      model parameter count";
 *   dims differ     -> VH_ERR_INVALID "Checkpoint shape does not match parameter
 *                      shape";
 *   not contiguous  -> VH_ERR_INVALID "copy_from_slice requires contiguous tensor";
 *   element count   -> VH_ERR_INVALID "Source slice length must match tensor numel"
 *   differs            (tensor.rs:816-826);
 *   short file, open or read failure -> VH_ERR_IO.
 * Tensors before the failing one keep their loaded values, as in the reference.
 * The copies run on `stream`; returns once they are done. Replaces
 * load_checkpoint. */
int vh_checkpoint_load(const char* path, int32_t n, float* const* tensors,
                       const vh_layout* layouts, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VEARO_HIP_H */
