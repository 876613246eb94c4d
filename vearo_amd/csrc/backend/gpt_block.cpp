// gpt_block.cpp -- the config[4] training step on the C ABI (include/vearo_block.h).
//
// Forward follows SimpleGPT::forward (crates/vearo-nn/src/lib.rs:745-791) with one
// TransformerBlock::forward (nn:666-675); the backward issues, in reverse tape
// order, what the autograd arms (crates/vearo-autograd/src/lib.rs:429-760) compute
// for those ops; AdamW follows optim:105-123. Where the reference runs two ops
// back to back, a fused kernel with the same rounding sequence stands in:
//   Linear: x W^T then + b            -> one GEMM, bias in its epilogue
//   residual x + Linear(..)           -> the GEMM accumulating into a copy of x
//   gelu(x W^T + b) / its Gelu + Add  -> vh_gelu_bias_fwd / vh_gelu_bias_bwd
//   reduce_to(grad, [C]) for a bias   -> vh_sum_rows (fixed grouping)
//   x^T.matmul(dy) per batch + reduce_to over the batch -> one GEMM over all
//     B*S rows (same sum, f32 rounding of a different grouping)
//   the q, k and v Linears (same input) -> one GEMM against the three weights
//     stacked [3D, D] (the parameter block stores q.w, k.w, v.w back to back,
//     and their biases); its backward is one GEMM for ln1's gradient (the sum
//     dq Wq + dk Wk + dv Wv in one chain instead of three added in tape order),
//     one for the stacked weight gradient, one row sum for the three biases
// The attention's q/k/v/out stay in the Linear layout [B, S, H, Dk] (q, k, v as
// column blocks of one [B*S, 3D] buffer); the reshape/transpose views of
// nn:585-601 are passed as strides, so no copy runs.
// The logits and their gradient have rows padded to Vp = V rounded up to 32
// (zero columns), and lm_head's weight is followed by Vp - V zero rows, so the
// three lm_head products run on 128-bit loads and the dx product (K = Vp) in
// whole k tiles, with no tail product; the padding adds exact zeros.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/vearo_block.h"
#include "../../../include/vearo_hip.h"
#include "vb_internal.h"

namespace {
thread_local std::string g_err;
}  // namespace

int vb_fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

namespace {

#define VB(expr)                                                  \
  do {                                                            \
    int rc_ = (expr);                                             \
    if (rc_ != VH_OK) return vb_fail(rc_, std::string(#expr) + ": " + vh_last_error()); \
  } while (0)

constexpr float kEps = 1e-5f;  // LayerNorm::new(n_embd, 1e-5) (nn:652, 742)

vh_layout contiguous(std::initializer_list<int64_t> dims) {
  vh_layout l{};
  l.rank = (int32_t)dims.size();
  int i = 0;
  for (int64_t d : dims) l.dims[i++] = d;
  int64_t acc = 1;
  for (int j = l.rank - 1; j >= 0; --j) {
    l.strides[j] = acc;
    acc *= l.dims[j];
  }
  return l;
}

}  // namespace

struct vb_gpt {
  vb_gpt_config c{};
  int64_t R = 0, Dk = 0, Vp = 0;
  int64_t off[VB_GPT_NPARAMS] = {}, numel[VB_GPT_NPARAMS] = {};
  size_t block_floats = 0;
  float *P = nullptr, *G = nullptr, *M = nullptr, *Vm = nullptr;  // params, grads, AdamW m and v
  int t = 0;
  int engine = VH_GEMM_ENGINE_DEFAULT;  // vh_gemm engine of the dense products
  // forward activations
  float *ids, *tg, *pos, *tok, *pe, *h0, *ln1, *qkv, *att, *h1, *ln2, *y1, *g, *h2, *lnf, *logits;
  float *loss, *one;
  // backward buffers
  float *dlogits, *dlnf, *dh, *dg, *df1, *lnx, *dh1, *datt, *dqkv, *dln1, *dh0;
  float* wT = nullptr;  // lm_head.w transposed [D, Vp] for dx
  float *attP = nullptr, *attG = nullptr;  // attention probabilities (kept for the backward), workspace
  size_t att_bytes = 0;
  std::vector<void*> allocs;

  float* p(int i) { return P + off[i]; }
  float* gr(int i) { return G + off[i]; }

  int alloc(float** out, int64_t n, int zero = 0) {
    void* ptr = nullptr;
    VB(vh_alloc((size_t)std::max<int64_t>(n, 1) * sizeof(float), zero, &ptr));
    allocs.push_back(ptr);
    *out = static_cast<float*>(ptr);
    return VH_OK;
  }
  ~vb_gpt() {
    for (void* a : allocs) vh_free(a);
  }

  // out[R, Dout] = x[R, Din] W^T (+ bias) (+ out when accumulate): Linear::forward.
  int linear(const float* x, int64_t Din, const float* W, int64_t Dout, const float* bias, float* out,
             int accumulate, int64_t ldc = 0) {
    vh_gemm_desc d{};
    d.M = R;
    d.N = Dout;
    d.K = Din;
    d.a = x;
    d.a_sm = Din;
    d.a_sk = 1;
    d.b = W;  // B[k][n] = W[n][k]
    d.b_sk = 1;
    d.b_sn = Din;
    d.c = out;
    d.c_sm = ldc ? ldc : Dout;
    d.batch[0] = d.batch[1] = 1;
    d.e = bias;
    d.e_sm = 0;
    d.e_sn = 1;
    d.alpha = 1.0f;
    d.accumulate = accumulate;
    d.engine = engine;
    VB(vh_gemm(&d, nullptr));
    return VH_OK;
  }

  // The Matmul arm's input gradient dx[R, Din] (+)= dy[R, Dout] W (autograd:502-519).
  int linear_dx(const float* dy, int64_t Dout, const float* W, int64_t Din, float* dx, int accumulate) {
    vh_gemm_desc d{};
    d.M = R;
    d.N = Din;
    d.K = Dout;
    d.a = dy;
    d.a_sm = Dout;
    d.a_sk = 1;
    d.b = W;  // B[k=o][n=i] = W[o][i]
    d.b_sk = Din;
    d.b_sn = 1;
    d.c = dx;
    d.c_sm = Din;
    d.batch[0] = d.batch[1] = 1;
    d.alpha = 1.0f;
    d.accumulate = accumulate;
    d.engine = engine;
    VB(vh_gemm(&d, nullptr));
    return VH_OK;
  }

  // The weight gradient dW[Dout, Din] = dy^T x over all R rows (the Matmul arm's
  // lhs^T.matmul(grad), reduce_to over the batch, then the Transpose arm).
  int linear_dw(const float* dy, int64_t Dout, const float* x, int64_t Din, float* dW) {
    vh_gemm_desc d{};
    d.M = Dout;
    d.N = Din;
    d.K = R;
    d.a = dy;  // A[m=o][k=r] = dy[r][o]
    d.a_sm = 1;
    d.a_sk = Dout;
    d.b = x;  // B[k=r][n=i] = x[r][i]
    d.b_sk = Din;
    d.b_sn = 1;
    d.c = dW;
    d.c_sm = Din;
    d.batch[0] = d.batch[1] = 1;
    d.alpha = 1.0f;
    d.engine = engine;
    VB(vh_gemm(&d, nullptr));
    return VH_OK;
  }

  // [B, H, S, Dk] view of a [B, S, D] tensor stored with row stride ld
  // (reshape + transpose(1, 2)).
  vh_layout heads(int64_t ld) const {
    vh_layout l{};
    l.rank = 4;
    l.dims[0] = c.B;
    l.dims[1] = c.H;
    l.dims[2] = c.S;
    l.dims[3] = Dk;
    l.strides[0] = c.S * ld;
    l.strides[1] = Dk;
    l.strides[2] = ld;
    l.strides[3] = 1;
    return l;
  }

  // with_grad: the cross-entropy arm of the backward (autograd:594-599, seed
  // gradient 1, autograd:795-798) runs together with the forward loss, in one
  // read of the logits.
  int forward(bool with_grad) {
    const int64_t D = c.D, F = c.F, V = c.V;
    const vh_layout lrd = contiguous({R, D});
    VB(vh_embedding_fwd(ids, p(0), tok, R, V, D, nullptr));
    VB(vh_embedding_fwd(pos, p(1), pe, R, c.P, D, nullptr));
    VB(vh_binary(VH_OP_ADD, tok, &lrd, pe, &lrd, h0, nullptr));
    VB(vh_layernorm_fwd(h0, p(2), p(3), ln1, R, D, kEps, nullptr));
    VB(linear(ln1, D, p(4), 3 * D, p(5), qkv, 0));  // [q | k | v] = ln1 [Wq; Wk; Wv]^T + [bq | bk | bv]
    const vh_layout hq = heads(3 * D), ha = heads(D);
    VB(vh_fused_attention_fwd(qkv, &hq, qkv + D, &hq, qkv + 2 * D, &hq, nullptr, nullptr, 1, att, &ha, attP,
                              att_bytes, nullptr));
    VB(vh_d2d(h1, h0, (size_t)(R * D) * sizeof(float), nullptr));
    VB(linear(att, D, p(10), D, p(11), h1, 1));  // h1 = h0 + (att W_o^T + b_o)
    VB(vh_layernorm_fwd(h1, p(12), p(13), ln2, R, D, kEps, nullptr));
    VB(linear(ln2, D, p(14), F, nullptr, y1, 0));
    VB(vh_gelu_bias_fwd(y1, p(15), g, R, F, nullptr));  // gelu(y1 + b_fc1)
    VB(vh_d2d(h2, h1, (size_t)(R * D) * sizeof(float), nullptr));
    VB(linear(g, F, p(16), D, p(17), h2, 1));  // h2 = h1 + (g W_fc2^T + b_fc2)
    VB(vh_layernorm_fwd(h2, p(18), p(19), lnf, R, D, kEps, nullptr));
    VB(linear(lnf, D, p(20), V, nullptr, logits, 0, Vp));
    if (with_grad)
      VB(vh_cross_entropy_fwd_bwd_ld(logits, Vp, tg, one, loss, dlogits, R, V, nullptr, 0, nullptr));
    else
      VB(vh_cross_entropy_fwd_ld(logits, Vp, tg, loss, R, V, nullptr, 0, nullptr));
    return VH_OK;
  }

  int backward() {
    const int64_t D = c.D, F = c.F, V = c.V;
    const vh_layout lrd = contiguous({R, D});
    // dlogits came with the forward (forward(true)). lm_head (rank-2 input, no bias), over the padded vocabulary: the zero
    // columns of dlogits meet the zero rows after the weight.
    // dx = dlogits W reads W through a transposed copy: both operands are then
    // k-contiguous, which the large-product kernel runs faster than W's
    // row-contiguous form (8.6 against 8.8 ms; the 154 MB copy costs ~90 us).
    {
      const vh_layout wl{2, 0, {D, Vp}, {1, D}};
      VB(vh_strided_copy(p(20), &wl, wT, nullptr));
      vh_gemm_desc d{};
      d.M = R;
      d.N = D;
      d.K = Vp;
      d.a = dlogits;
      d.a_sm = Vp;
      d.a_sk = 1;
      d.b = wT;  // B[k=v][n=d] = W[v][d] = wT[d][v]
      d.b_sk = 1;
      d.b_sn = Vp;
      d.c = dlnf;
      d.c_sm = D;
      d.batch[0] = d.batch[1] = 1;
      d.alpha = 1.0f;
      d.engine = engine;
      VB(vh_gemm(&d, nullptr));
    }
    // dW = dlogits^T lnf straight into the gradient's [Vp, D] layout: A is
    // dlogits read row-contiguous (m-contiguous), B is lnf; the large-product
    // kernel's wide tile runs it at 8.93 ms, against 8.92 ms for the
    // transposed product plus ~100 us of transposing copies on either side.
    {
      vh_gemm_desc d{};
      d.M = Vp;
      d.N = D;
      d.K = R;
      d.a = dlogits;  // A[m=v][k=r] = dlogits[r][v]
      d.a_sm = 1;
      d.a_sk = Vp;
      d.b = lnf;  // B[k=r][n=d] = lnf[r][d]
      d.b_sk = D;
      d.b_sn = 1;
      d.c = gr(20);  // dW [Vp, D] (the rows past V meet dlogits' zero columns)
      d.c_sm = D;
      d.batch[0] = d.batch[1] = 1;
      d.alpha = 1.0f;
      d.engine = engine;
      VB(vh_gemm(&d, nullptr));
    }
    VB(vh_layernorm_bwd(h2, p(18), dlnf, dh, gr(18), gr(19), R, D, kEps, nullptr, 0, nullptr));
    // h2 = h1 + f2: h1 and f2 both receive dh.
    VB(vh_sum_rows(dh, R, D, gr(17), nullptr, 0, nullptr));
    VB(linear_dx(dh, D, p(16), F, dg, 0));
    VB(linear_dw(dh, D, g, F, gr(16)));
    VB(vh_gelu_bias_bwd(y1, p(15), dg, df1, gr(15), R, F, nullptr, 0, nullptr));
    VB(linear_dx(df1, F, p(14), D, lnx, 0));
    VB(linear_dw(df1, F, ln2, D, gr(14)));
    // ln_2 arm, then h1's gradient accumulates: existing (dh) + new.
    VB(vh_layernorm_bwd(h1, p(12), lnx, dln1, gr(12), gr(13), R, D, kEps, nullptr, 0, nullptr));
    VB(vh_binary(VH_OP_ADD, dh, &lrd, dln1, &lrd, dh1, nullptr));
    // h1 = h0 + o: out_proj.
    VB(vh_sum_rows(dh1, R, D, gr(11), nullptr, 0, nullptr));
    VB(linear_dx(dh1, D, p(10), D, datt, 0));
    VB(linear_dw(dh1, D, att, D, gr(10)));
    const vh_layout hq = heads(3 * D), ha = heads(D);
    // The Fused attention arm (autograd:600-612) from the forward's probabilities.
    VB(vh_fused_attention_bwd_probs(attP, qkv, &hq, qkv + D, &hq, qkv + 2 * D, &hq, 1, datt, &ha, dqkv, &hq,
                                    dqkv + D, &hq, dqkv + 2 * D, &hq, attG, att_bytes, nullptr));
    // The q, k, v Linears at once: bias sums, ln1's gradient, stacked weight gradient.
    VB(vh_sum_rows(dqkv, R, 3 * D, gr(5), nullptr, 0, nullptr));
    VB(linear_dx(dqkv, 3 * D, p(4), D, dln1, 0));
    VB(linear_dw(dqkv, 3 * D, ln1, D, gr(4)));
    VB(vh_layernorm_bwd(h0, p(2), dln1, lnx, gr(2), gr(3), R, D, kEps, nullptr, 0, nullptr));
    VB(vh_binary(VH_OP_ADD, dh1, &lrd, lnx, &lrd, dh0, nullptr));
    // h0 = tok + pe; the embeddings' arms (position recorded last, runs first).
    VB(vh_embedding_bwd(pos, dh0, gr(1), R, c.P, D, nullptr, 0, nullptr));
    VB(vh_embedding_bwd(ids, dh0, gr(0), R, V, D, nullptr, 0, nullptr));
    return VH_OK;
  }
};

extern "C" {

const char* vb_last_error(void) { return g_err.c_str(); }

int vb_gpt_create(const vb_gpt_config* cfg, vb_gpt** out) {
  if (!cfg || !out) return vb_fail(VH_ERR_INVALID, "vb_gpt_create: null pointer");
  *out = nullptr;
  const vb_gpt_config c = *cfg;
  if (c.B <= 0 || c.S <= 0 || c.D <= 0 || c.H <= 0 || c.F <= 0 || c.V <= 0 || c.P <= 0)
    return vb_fail(VH_ERR_INVALID, "vb_gpt_create: sizes must be positive");
  if (c.D % c.H != 0) return vb_fail(VH_ERR_INVALID, "n_embd must be divisible by n_head");
  if (c.S > c.P) return vb_fail(VH_ERR_INVALID, "vb_gpt_create: sequence longer than max_seq_len");
  auto* g = new vb_gpt();
  g->c = c;
  g->R = c.B * c.S;
  g->Dk = c.D / c.H;
  g->Vp = (c.V + 31) / 32 * 32;
  const int64_t D = c.D, F = c.F;
  const int64_t sizes[VB_GPT_NPARAMS] = {c.V * D, c.P * D, D, D, D * D, D, D * D, D, D * D, D, D * D, D,
                                         D,       D,       F * D, F, D * F, D, D, D, c.V * D};
  // Memory order: q.w, k.w, v.w back to back (a [3D, D] stack), then q.b, k.b,
  // v.b (a [3D] vector); every other tensor starts 256-byte aligned.
  const int order[VB_GPT_NPARAMS] = {0, 1, 2, 3, 4, 6, 8, 5, 7, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20};
  size_t o = 0;
  for (int j = 0; j < VB_GPT_NPARAMS; ++j) {
    const int i = order[j];
    g->off[i] = (int64_t)o;
    g->numel[i] = sizes[i];
    const bool packed = i == 4 || i == 6 || i == 5 || i == 7;  // followed by the next of its stack
    o += packed ? (size_t)sizes[i] : (((size_t)sizes[i] + 63) & ~size_t(63));
  }
  o += (((size_t)((g->Vp - c.V) * D)) + 63) & ~size_t(63);  // zero rows after lm_head.w
  g->block_floats = o;
  const int64_t R = g->R, Vp = g->Vp;
  int rc = VH_OK;
  auto A = [&](float** p, int64_t n, int zero = 0) {
    if (rc == VH_OK) rc = g->alloc(p, n, zero);
  };
  A(&g->P, (int64_t)o, 1);
  A(&g->G, (int64_t)o, 1);
  A(&g->M, (int64_t)o, 1);
  A(&g->Vm, (int64_t)o, 1);
  for (float** p : {&g->ids, &g->tg, &g->pos}) A(p, R, 1);
  for (float** p : {&g->tok, &g->pe, &g->h0, &g->ln1, &g->att, &g->h1, &g->ln2, &g->h2, &g->lnf, &g->dlnf,
                    &g->dh, &g->lnx, &g->dh1, &g->datt, &g->dln1, &g->dh0})
    A(p, R * D);
  A(&g->qkv, 3 * R * D);
  A(&g->dqkv, 3 * R * D);
  for (float** p : {&g->y1, &g->g, &g->dg, &g->df1}) A(p, R * F);
  A(&g->logits, R * Vp, 1);
  A(&g->dlogits, R * Vp, 1);
  A(&g->wT, D * Vp);
  g->att_bytes = vh_fused_attention_scratch_bytes(c.B, c.H, c.S, 0);
  A(&g->attP, (int64_t)(g->att_bytes / sizeof(float)));
  A(&g->attG, (int64_t)(g->att_bytes / sizeof(float)));
  A(&g->loss, 1, 1);
  A(&g->one, 1);
  if (rc == VH_OK) {
    // Positions 0..S-1 for every batch row (nn:753-761), LayerNorm weights 1
    // (nn:524-529), the backward's seed gradient 1 (autograd:795-798).
    std::vector<float> pos((size_t)R);
    for (int64_t r = 0; r < R; ++r) pos[(size_t)r] = (float)(r % c.S);
    rc = vh_h2d(g->pos, pos.data(), pos.size() * sizeof(float));
    for (int i : {2, 12, 18})
      if (rc == VH_OK) rc = vh_fill_f32(g->p(i), 1.0f, g->numel[i], nullptr);
    if (rc == VH_OK) rc = vh_fill_f32(g->one, 1.0f, 1, nullptr);
    if (rc == VH_OK) rc = vh_sync();
    if (rc != VH_OK) vb_fail(rc, std::string("vb_gpt_create: ") + vh_last_error());
  }
  if (rc != VH_OK) {
    delete g;
    return rc;
  }
  *out = g;
  return VH_OK;
}

void vb_gpt_destroy(vb_gpt* g) { delete g; }

int vb_gpt_param(vb_gpt* g, int i, float** ptr, int64_t* numel) {
  if (!g || i < 0 || i >= VB_GPT_NPARAMS || !ptr || !numel) return vb_fail(VH_ERR_INVALID, "vb_gpt_param: bad argument");
  *ptr = g->p(i);
  *numel = g->numel[i];
  return VH_OK;
}

int vb_gpt_grad(vb_gpt* g, int i, float** ptr, int64_t* numel) {
  if (!g || i < 0 || i >= VB_GPT_NPARAMS || !ptr || !numel) return vb_fail(VH_ERR_INVALID, "vb_gpt_grad: bad argument");
  *ptr = g->gr(i);
  *numel = g->numel[i];
  return VH_OK;
}

int vb_gpt_inputs(vb_gpt* g, float** ids, float** targets) {
  if (!g || !ids || !targets) return vb_fail(VH_ERR_INVALID, "vb_gpt_inputs: null pointer");
  *ids = g->ids;
  *targets = g->tg;
  return VH_OK;
}

float* vb_gpt_loss_ptr(vb_gpt* g) { return g ? g->loss : nullptr; }

int vb_gpt_set_gemm_engine(vb_gpt* g, int engine) {
  if (!g) return vb_fail(VH_ERR_INVALID, "vb_gpt_set_gemm_engine: null handle");
  if (engine != VH_GEMM_ENGINE_DEFAULT && engine != VH_GEMM_ENGINE_LIBRARY)
    return vb_fail(VH_ERR_INVALID, "vb_gpt_set_gemm_engine: engine must be DEFAULT or LIBRARY");
  g->engine = engine;
  return VH_OK;
}

int vb_gpt_forward_backward(vb_gpt* g, int backward) {
  if (!g) return vb_fail(VH_ERR_INVALID, "vb_gpt_forward_backward: null handle");
  int rc = g->forward(backward != 0);
  if (rc == VH_OK && backward) rc = g->backward();
  return rc;
}

int vb_gpt_adamw(vb_gpt* g, float lr, float beta1, float beta2, float eps, float weight_decay) {
  if (!g) return vb_fail(VH_ERR_INVALID, "vb_gpt_adamw: null handle");
  g->t += 1;
  // One launch over the whole parameter block: the 256-byte padding between
  // tensors holds zeros in p, g, m and v and stays zero under the update.
  VB(vh_adamw_step(g->P, g->G, g->M, g->Vm, (int64_t)g->block_floats, g->t, lr, beta1, beta2, eps, weight_decay,
                   nullptr));
  return VH_OK;
}

namespace {
// Parameter i's layout in SimpleGPT::parameters() order (nn:797-807).
vh_layout param_layout(const vb_gpt_config& c, int i) {
  const int64_t D = c.D;
  int64_t r = D, k = 0;  // [r, k]; k == 0: rank 1 [r]
  switch (i) {
    case 0: case 20: r = c.V; k = D; break;
    case 1: r = c.P; k = D; break;
    case 4: case 6: case 8: case 10: k = D; break;
    case 14: r = c.F; k = D; break;
    case 15: r = c.F; break;
    case 16: k = c.F; break;
    default: break;
  }
  vh_layout l{};
  l.rank = k ? 2 : 1;
  l.dims[0] = r;
  l.strides[0] = k ? k : 1;
  if (k) {
    l.dims[1] = k;
    l.strides[1] = 1;
  }
  return l;
}
}  // namespace

int vb_gpt_save(vb_gpt* g, const char* path) {
  if (!g) return vb_fail(VH_ERR_INVALID, "vb_gpt_save: null handle");
  const float* ptrs[VB_GPT_NPARAMS];
  vh_layout lays[VB_GPT_NPARAMS];
  for (int i = 0; i < VB_GPT_NPARAMS; ++i) {
    ptrs[i] = g->p(i);
    lays[i] = param_layout(g->c, i);
  }
  VB(vh_checkpoint_save(path, VB_GPT_NPARAMS, ptrs, lays, nullptr));
  return VH_OK;
}

int vb_gpt_load(vb_gpt* g, const char* path) {
  if (!g) return vb_fail(VH_ERR_INVALID, "vb_gpt_load: null handle");
  float* ptrs[VB_GPT_NPARAMS];
  vh_layout lays[VB_GPT_NPARAMS];
  for (int i = 0; i < VB_GPT_NPARAMS; ++i) {
    ptrs[i] = g->p(i);
    lays[i] = param_layout(g->c, i);
  }
  VB(vh_checkpoint_load(path, VB_GPT_NPARAMS, ptrs, lays, nullptr));
  return VH_OK;
}

int vb_gpt_train_step(vb_gpt* g, float lr, float beta1, float beta2, float eps, float weight_decay) {
  int rc = vb_gpt_forward_backward(g, 1);
  if (rc != VH_OK) return rc;
  return vb_gpt_adamw(g, lr, beta1, beta2, eps, weight_decay);
}

}  // extern "C"
