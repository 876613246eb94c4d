/*
 * vearo_cpu_ref.h -- CPU oracle: a C restatement of vearo-backend-cpu's hot-path
 * functions, used ONLY as a test checker and as the timed CPU baseline.
 *
 * TEST INFRASTRUCTURE. Nothing in the product (libvearo_hip.so, the vearo_amd
 * package) links, loads or calls this code. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may use it.
 *
 * Every function follows the loop order and f32 accumulation order of the Rust
 * source it cites (paths relative to the reference checkout):
 *   cpu:      crates/vearo-backend-cpu/src/lib.rs
 *   autograd: crates/vearo-autograd/src/lib.rs
 *   shape:    crates/vearo-core/src/shape.rs
 * It is compiled with -ffp-contract=off and without fast-math, so a*b+c is two
 * roundings exactly as in Rust (which never contracts), and it calls glibc
 * expf/tanhf/logf/sqrtf, the libm Rust's f32::exp/tanh/ln/sqrt reach on linux-gnu.
 *
 * Layouts mirror vearo-core's Tensor: dims + element strides, no storage offset
 * (views in vearo only permute/transpose strides, tensor.rs:537-620).
 */
#ifndef VEARO_CPU_REF_H
#define VEARO_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VO_MAX_RANK 8

typedef struct {
  int32_t rank;
  int64_t dims[VO_MAX_RANK];
  int64_t strides[VO_MAX_RANK];
} vo_layout;

/* Return codes: 0 = ok, 1 = the reference would panic (message in err). */
#define VO_OK 0
#define VO_PANIC 1
#define VO_IOERR 2 /* the reference returns an io::Error (message in err) */

/* Binary broadcast ops (cpu:160-238). op: 0 add, 1 sub, 2 mul, 3 div.
 * out_shape must be the broadcast of the two shapes; out is contiguous. */
int vo_binary(int op, const float* lhs, const vo_layout* ll, const float* rhs,
              const vo_layout* rl, float* out, const vo_layout* out_shape,
              char* err, size_t errlen);

/* gelu, tanh approximation (cpu:458-497). */
void vo_gelu(const float* x, const vo_layout* xl, float* out);

/* Softmax over `dim` (cpu:501-563). */
int vo_softmax(const float* x, const vo_layout* xl, int dim, float* out,
               char* err, size_t errlen);

/* Single-axis sum / mean (cpu:566-653). out has the reduced shape. */
int vo_sum(const float* x, const vo_layout* xl, int dim, int keep_dim, float* out,
           char* err, size_t errlen);
int vo_mean(const float* x, const vo_layout* xl, int dim, int keep_dim, float* out,
            char* err, size_t errlen);

/* LayerNorm forward / backward over the last dim (cpu:665-858). */
int vo_layernorm(const float* x, const vo_layout* xl, const float* w,
                 const vo_layout* wl, const float* b, const vo_layout* bl, float eps,
                 float* out, char* err, size_t errlen);
int vo_layernorm_backward(const float* x, const vo_layout* xl, const float* w,
                          const vo_layout* wl, const vo_layout* bl, const float* go,
                          const vo_layout* gol, float eps, float* gx, float* gw,
                          float* gb, char* err, size_t errlen);

/* Embedding forward / backward (cpu:860-980). ids are f32 (the API contract). */
int vo_embedding(const float* ids, const vo_layout* il, const float* w,
                 const vo_layout* wl, float* out, char* err, size_t errlen);
int vo_embedding_backward(const float* ids, const vo_layout* il, const vo_layout* wl,
                          const float* go, const vo_layout* gol, float* gw, char* err,
                          size_t errlen);

/* Cross-entropy forward (mean loss, one float) / backward (cpu:982-1127). */
int vo_cross_entropy(const float* logits, const vo_layout* ll, const float* tgt,
                     const vo_layout* tl, float* loss, char* err, size_t errlen);
int vo_cross_entropy_backward(const float* logits, const vo_layout* ll,
                              const float* tgt, const vo_layout* tl,
                              const float* grad_out, int64_t grad_out_numel,
                              float* gl, char* err, size_t errlen);

/* Autograd helpers that run on the host in the reference. */
void vo_gelu_grad_mask(const float* x_contig, int64_t n, float* mask); /* autograd:383-403 */
int vo_reduce_to(const float* grad_contig, const vo_layout* gshape, const int64_t* target,
                 int target_rank, float* out, char* err, size_t errlen); /* autograd:316-361 */

/* Composite paths the unchanged autograd arms drive, restated end to end. */
/* Softmax arm (autograd:547-553): y = softmax(x); s = sum(dy*y, dim, keep);
 * dx = y * (dy - s). x and dy contiguous with the same shape. */
int vo_softmax_backward_composite(const float* x, const float* dy, const vo_layout* xl,
                                  int dim, float* dx, char* err, size_t errlen);
/* Gelu arm (autograd:542-546) on a bias-add input: h = x + bias (cpu:160-202
 * broadcast), y = gelu(h) forward; backward dh = dy * gelu_mask(h),
 * dbias = reduce_to(dh, [C]). x, dy: [rows, C] contiguous. */
void vo_gelu_bias_forward(const float* x, const float* bias, int64_t rows, int64_t C,
                          float* y);
void vo_gelu_bias_backward(const float* x, const float* bias, const float* dy,
                           int64_t rows, int64_t C, float* dx, float* dbias);

/* Shortest round-trip positional formatting of an f32, as Rust's `{}` prints it. */
void vo_format_f32(float v, char* buf, size_t len);

/* Layout helpers. */
void vo_contiguous_layout(vo_layout* l, int rank, const int64_t* dims);

/* ---- part 2 (vearo_cpu_gpt.c): matmul, fused attention, AdamW, SimpleGPT ---- */

/* Threads used by the blocked loops (default: $VO_THREADS, $OMP_NUM_THREADS,
 * else all online CPUs). Thread count never changes a result. */
void vo_set_threads(int n);

/* Batched matmul with broadcast batch dims (cpu:266-417); lhs, rhs contiguous
 * (the reference makes them contiguous first); out contiguous
 * [broadcast batch..., M, N]. */
int vo_matmul(const float* lhs, const vo_layout* ll, const float* rhs, const vo_layout* rl,
              float* out, char* err, size_t errlen);

/* Fused attention forward / backward (cpu:2366-2630). q, k, v, go, out, dq,
 * dk, dv: contiguous [B, H, S, Dk]. mask: NULL or contiguous, right-aligned to
 * rank 4 and broadcast (cpu:2395-2404). */
int vo_fused_attention(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                       int64_t S, int64_t Dk, const float* mask, const vo_layout* ml, float* out);
int vo_fused_attention_backward(const float* q, const float* k, const float* v, int64_t B,
                                int64_t H, int64_t S, int64_t Dk, const float* mask,
                                const vo_layout* ml, const float* go, float* dq, float* dk,
                                float* dv);

/* The unfused attention of MultiHeadAttention::forward with
 * VEARO_USE_FUSED_ATTENTION=0 (nn:603-613): scores = q.matmul(k^T).mul(scale)
 * (+ mask), probs = scores.softmax(3), out = probs.matmul(v), each op the CPU
 * backend's own; the backward walks that tape's arms (Matmul, Softmax, Add,
 * Mul, Matmul, Transpose; autograd:474-599). Same layouts as the fused form. */
int vo_attention_unfused(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t S,
                         int64_t Dk, const float* mask, const vo_layout* ml, float* out, char* err, size_t errlen);
int vo_attention_unfused_backward(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                                  int64_t S, int64_t Dk, const float* mask, const vo_layout* ml, const float* go,
                                  float* dq, float* dk, float* dv, char* err, size_t errlen);

/* Tensor::adamw_step on one parameter (tensor.rs:931-986), t >= 1. */
void vo_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, int t, float lr,
                   float beta1, float beta2, float eps, float wd);

/* SimpleGPT with one TransformerBlock (nn:666-791): B x S token ids, model
 * width D, H heads, MLP width F, vocabulary V, P = max_seq_len. */
typedef struct {
  int64_t B, S, D, H, F, V, P;
} vo_gpt_config;

/* Parameters in SimpleGPT::parameters() order (nn:797-807). */
enum {
  VO_P_WTE, VO_P_WPE, VO_P_LN1_W, VO_P_LN1_B, VO_P_Q_W, VO_P_Q_B, VO_P_K_W, VO_P_K_B,
  VO_P_V_W, VO_P_V_B, VO_P_O_W, VO_P_O_B, VO_P_LN2_W, VO_P_LN2_B, VO_P_FC1_W, VO_P_FC1_B,
  VO_P_FC2_W, VO_P_FC2_B, VO_P_LNF_W, VO_P_LNF_B, VO_P_LM_W, VO_GPT_NPARAMS
};
void vo_gpt_param_numel(const vo_gpt_config* c, int64_t* numel);

/* Forward (loss, the mean cross-entropy as one float) and, when grads is not
 * NULL, the autograd backward into grads[i] (same shapes as params[i]),
 * following the reverse tape order of autograd:429-760. The causal mask is the
 * model's own [S, S] tensor with -1e9 above the diagonal (nn:763-771). */
int vo_gpt_step(const vo_gpt_config* c, const float* const* params, const float* ids,
                const float* targets, float* loss, float* const* grads, char* err, size_t errlen);
/* The same step with the attention on the unfused path when `unfused` is
 * nonzero (VEARO_USE_FUSED_ATTENTION=0, nn:603-613). */
int vo_gpt_step_ex(const vo_gpt_config* c, const float* const* params, const float* ids,
                   const float* targets, int unfused, float* loss, float* const* grads, char* err,
                   size_t errlen);

/* y[i] = expf / logf / tanhf (x[i]) (which = 0 / 1 / 2): the C library's
 * functions, as every oracle function above calls them (the reference's f32
 * `exp`, `ln`, `tanh` call the same libm on Linux). For tests that bound their
 * rounding against correctly rounded values. */
void vo_math(int which, const float* x, float* y, int64_t n);

/* `.ve` weight checkpoint (crates/vearo/src/checkpoint.rs:9-91), host tensors. */
int vo_checkpoint_save(const char* path, int n, const float* const* data, const vo_layout* layouts, char* err,
                       size_t errlen);
int vo_checkpoint_load(const char* path, int n, float* const* data, const vo_layout* layouts, char* err,
                       size_t errlen);

#ifdef __cplusplus
}
#endif
#endif
