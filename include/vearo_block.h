/*
 * vearo_block.h -- C ABI of the config[4] training step: SimpleGPT with one
 * TransformerBlock (token + position embedding, pre-LN block with fused causal
 * attention and a GELU MLP, final layernorm, lm_head, cross-entropy), its
 * autograd backward and one AdamW update, run entirely on one MI355X.
 *
 * This replaces, for this model, the reference's host-driven chain
 *   SimpleGPT::forward        (crates/vearo-nn/src/lib.rs:745-791, 666-675)
 *   loss.backward()           (crates/vearo-autograd/src/lib.rs:429-760)
 *   AdamW::step               (crates/vearo-optim/src/lib.rs:105-123,
 *                              Tensor::adamw_step tensor.rs:931-1023)
 * issuing the same op sequence -- the forward modules' ops and, in reverse tape
 * order, the autograd arms' ops -- through libvearo_hip.so. The model lives in
 * device memory owned by the handle: parameters, gradients, AdamW moments and
 * every activation the backward needs, allocated once. The causal mask is the
 * model's -1e9 upper triangle, passed to the attention as its causal flag
 * (identical results: exp underflows to exactly 0 either way).
 *
 * Parameters are numbered in SimpleGPT::parameters() order (nn:797-807):
 *   0 wte[V,D] 1 wpe[P,D] 2 ln1.w[D] 3 ln1.b[D] 4 q.w[D,D] 5 q.b[D] 6 k.w 7 k.b
 *   8 v.w 9 v.b 10 out.w 11 out.b 12 ln2.w 13 ln2.b 14 fc1.w[F,D] 15 fc1.b[F]
 *   16 fc2.w[D,F] 17 fc2.b[D] 18 ln_f.w 19 ln_f.b 20 lm_head.w[V,D]
 * All entry points return VH_OK (0) or a VH_ERR_* code; vh_last_error() has the
 * text. vh_init() must have been called.
 */
#ifndef VEARO_BLOCK_H
#define VEARO_BLOCK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VB_GPT_NPARAMS 21

/* B x S tokens, model width D, H heads, MLP width F, vocabulary V,
 * P = max_seq_len (>= S). D % H == 0. */
typedef struct {
  int64_t B, S, D, H, F, V, P;
} vb_gpt_config;

typedef struct vb_gpt vb_gpt;

/* Allocates the model (parameters zero, LayerNorm weights one, AdamW moments
 * zero, step count 0). Upload parameters through vb_gpt_param. */
int vb_gpt_create(const vb_gpt_config* cfg, vb_gpt** out);
void vb_gpt_destroy(vb_gpt* g);

/* Device pointer and element count of parameter i, of its gradient (valid after
 * a backward), and of the per-step token ids / targets buffers ([B, S] f32,
 * the API's f32 ids) that vb_gpt_step reads. */
int vb_gpt_param(vb_gpt* g, int i, float** ptr, int64_t* numel);
int vb_gpt_grad(vb_gpt* g, int i, float** ptr, int64_t* numel);
int vb_gpt_inputs(vb_gpt* g, float** ids, float** targets);

/* One forward (and with backward != 0 the whole autograd backward) on the
 * current ids/targets. The loss (mean cross-entropy, one float) is written to
 * device memory at *loss_dev (vb_gpt_loss_ptr). Asynchronous on the library's
 * stream; vh_sync() waits. */
int vb_gpt_forward_backward(vb_gpt* g, int backward);
float* vb_gpt_loss_ptr(vb_gpt* g);

/* AdamW::step: increments the step count and updates every parameter from its
 * gradient (optim:105-123), lr/betas/eps/weight decay as AdamW::new takes them. */
int vb_gpt_adamw(vb_gpt* g, float lr, float beta1, float beta2, float eps, float weight_decay);

/* Text of the last error of a vb_* call on this thread (a failing vh_* call's
 * own text included). */
const char* vb_last_error(void);

/* The parameters as a `.ve` checkpoint, SimpleGPT::parameters() order and
 * shapes (crates/vearo/src/checkpoint.rs:9-33 on model.parameters()), and back
 * (checkpoint.rs:40-91; the reference's count/shape checks and texts). The
 * file is the one the reference's save_checkpoint writes for the same model.
 * Waits for queued work on the library's stream. */
int vb_gpt_save(vb_gpt* g, const char* path);
int vb_gpt_load(vb_gpt* g, const char* path);

/* The vh_gemm engine (VH_GEMM_ENGINE_*) of the step's dense products (the
 * Linear layers and lm_head; attention's batched products always run on this
 * library's kernels): DEFAULT, or LIBRARY for the benchmarks' hipBLASLt A/B.
 * No counterpart in the reference. */
int vb_gpt_set_gemm_engine(vb_gpt* g, int engine);

/* The config[4] training step: forward + backward + AdamW. */
int vb_gpt_train_step(vb_gpt* g, float lr, float beta1, float beta2, float eps, float weight_decay);

/* ---------------------------------------------------------------------------
 * The same model and step issued op by op through the HIP BackendOps table
 * (the C++ mirror of tensor.rs:1108-1196), in the order the reference's own
 * code issues them: SimpleGPT::forward's Tensor ops recording a tape
 * (nn:584-621, 666-675, 745-791; autograd lib.rs:150-188), loss.backward()
 * walking it in reverse through the backward_impl arms (autograd
 * lib.rs:429-792), then AdamW::step (optim:105-123). This is what an unchanged
 * vearo program gets from this backend, op for op; vb_gpt above fuses the same
 * chain. reduce_to, the Gelu arm's mask and adamw_step, host loops in the
 * reference, run on the device (sum slot, vh_gelu_grad_mul, vh_adamw_step).
 * Parameters are numbered as for vb_gpt; the model starts like vb_gpt_create's.
 * Every call is synchronous except vb_dropin_step with loss == NULL and
 * timing == 0. No counterpart entry point in the reference: the drop-in
 * step's measurement and parity harness.
 * ------------------------------------------------------------------------- */
#define VB_DROPIN_NPHASES 23

typedef struct vb_dropin vb_dropin;

int vb_dropin_create(const vb_gpt_config* cfg, vb_dropin** out);
void vb_dropin_destroy(vb_dropin* d);
/* MultiHeadAttention's path: fused != 0 the fused_attention slot (the
 * default), 0 the unfused chain q.matmul(k^T).mul(scale).add(mask).softmax(3)
 * .matmul(v) with its autograd arms (crates/vearo-nn/src/lib.rs:603-613).
 * vb_dropin_create starts from the reference's switch, the environment
 * variable VEARO_USE_FUSED_ATTENTION ("0" or "false": unfused). */
int vb_dropin_set_fused_attention(vb_dropin* d, int fused);
int vb_dropin_fused_attention(const vb_dropin* d);
/* The Matmul arm's gradient of a 2-D right operand shared by every batch (the
 * Linear weights and the lm_head, [..., S, K] x [K, N]): fold = 1 (the
 * default) computes reduce_to(l^T g, [K, N]) as one product over all leading
 * rows, g.reshape([rows, N]).transpose(0, 1).matmul(l.reshape([rows, K]))
 * passed on as its [K, N] transpose (the weight's gradient then arrives
 * contiguous), the same sum in another grouping; fold = 0 issues the reference's arm, the
 * per-batch product then reduce_to over the batch (autograd lib.rs:502-519,
 * 316-361). No counterpart in the reference: a one-arm change a HIP-aware
 * autograd would make. */
int vb_dropin_set_fold_weight_grads(vb_dropin* d, int fold);
int vb_dropin_fold_weight_grads(const vb_dropin* d);
/* Host copies of parameter i (numel must match) and of its last gradient
 * (after a step with backward != 0). */
int vb_dropin_set_param(vb_dropin* d, int i, const float* host, int64_t numel);
int vb_dropin_get_param(vb_dropin* d, int i, float* host, int64_t numel);
int vb_dropin_get_grad(vb_dropin* d, int i, float* host, int64_t numel);
/* Token ids and targets, host [B, S] f32. */
int vb_dropin_set_inputs(vb_dropin* d, const float* ids, const float* targets);
/* One forward, with backward != 0 the autograd backward, with adamw != 0 (needs
 * backward) one AdamW step. timing != 0 records an event after every op and
 * waits for the step, for vb_dropin_phase_ms. loss != NULL waits and stores
 * the loss. */
int vb_dropin_step(vb_dropin* d, int backward, int adamw, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int timing, float* loss);
/* Milliseconds per phase of the last timed step (n >= VB_DROPIN_NPHASES), and
 * the phases' names ("fwd.matmul", "bwd.reduce_to", "adamw.update", ...). */
int vb_dropin_phase_ms(vb_dropin* d, double* ms, int n);
const char* vb_dropin_phase_name(int i);

#ifdef __cplusplus
}
#endif
#endif /* VEARO_BLOCK_H */
