// dropin_gpt.cpp -- the config[4] training step issued op by op through the HIP
// BackendOps table (vearo_backend.h), in the order vearo's own code issues it:
//
//   forward   SimpleGPT::forward (crates/vearo-nn/src/lib.rs:745-791) with one
//             TransformerBlock::forward (nn:666-675), MultiHeadAttention::forward
//             (nn:584-621) on its default fused path or, as the reference does
//             with VEARO_USE_FUSED_ATTENTION=0 (read at create, or set with
//             vb_dropin_set_fused_attention), its unfused path: q.matmul(k^T)
//             .mul(scale).add(mask).softmax(3).matmul(v) (nn:603-613), and
//             Linear::forward (nn:119-127). Every Tensor op with an input that needs a gradient
//             records a tape node holding its inputs; a parameter becomes a leaf
//             node on first use (Tape::push, autograd lib.rs:150-188).
//   backward  loss.backward(): the tape walked in reverse with the arms of
//             backward_impl (autograd lib.rs:429-792, arms 474-599); a gradient
//             reaching a node twice is accumulated with `add` in walk order.
//   AdamW     AdamW::step (crates/vearo-optim/src/lib.rs:105-123): each
//             gradient made contiguous, then its parameter updated.
//
// Three steps of that chain are host loops in the reference, above the backend:
// reduce_to (autograd:316-361), gelu_grad_mask (383-403) and the device branch
// of Tensor::adamw_step (tensor.rs:989-1019). Here they stay on the device:
// reduce_to as `sum` slot calls, the Gelu arm's mask-and-multiply as one
// vh_gelu_grad_mul, adamw_step as vh_adamw_step -- what a HIP-aware autograd and
// optimizer would issue. The position ids, the causal mask (-1e9 above the
// diagonal, nn:763-771), the unfused path's scale 1/sqrt(d_k) (nn:606) and the
// backward's seed gradient 1.0 (autograd:795-798) are device tensors built
// once instead of host tensors built every call.
// Gradients of interior nodes and the tape's saved inputs are released as the
// walk passes them (the reference holds them to the end of backward_impl).
//
// One arm is folded by default (vb_dropin_set_fold_weight_grads(d, 0) keeps
// the reference's own): the Matmul arm's right-operand gradient when that
// operand is a 2-D weight shared by every batch ([..., S, K] x [K, N], every
// Linear layer and the lm_head). The reference computes lᵀ·g per batch and
// then reduce_to's the [B, K, N] result over the batch (autograd:502-519,
// 316-361); folded, it is one product over all B·S rows,
// g.reshape([B·S, N]).transpose(0, 1).matmul(l.reshape([B·S, K])) ([N, K],
// the weight's own layout) passed on transposed, with the same slots
// (reshape and transpose are views of contiguous tensors). The same sum in
// another grouping, and no per-batch [B, K, N] intermediate.
//
// With timing on, an event follows each op on the library's stream and the
// time between consecutive events is charged to that op's phase (launch gaps
// included), so the phases add up to the step.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "../../../include/vearo_block.h"
#include "../../../include/vearo_hip.h"
#include "vb_internal.h"
#include "vearo_backend.h"

using vearo_hip::Shape;
using vearo_hip::Tensor;

namespace {

enum Phase : int {
  F_EMBED, F_LN, F_MATMUL, F_ADD, F_COPY, F_ATTN, F_GELU, F_XENT,
  B_XENT, B_MATMUL, B_REDUCE, B_ACC, B_COPY, B_LN, B_ATTN, B_GELU, B_EMBED,
  O_CONTIG, O_ADAMW, F_MUL, F_SOFTMAX, B_MUL, B_SOFTMAX, NPHASE
};
static_assert(NPHASE == VB_DROPIN_NPHASES, "phase table");

const char* const kPhase[NPHASE] = {
    "fwd.embedding",      "fwd.layernorm",       "fwd.matmul",           "fwd.add",
    "fwd.reshape_copy",   "fwd.fused_attention", "fwd.gelu",             "fwd.cross_entropy",
    "bwd.cross_entropy",  "bwd.matmul",          "bwd.reduce_to",        "bwd.grad_accumulate",
    "bwd.reshape_copy",   "bwd.layernorm",       "bwd.fused_attention",  "bwd.gelu",
    "bwd.embedding",      "adamw.grad_contiguous", "adamw.update",       "fwd.mul",
    "fwd.softmax",        "bwd.mul",             "bwd.softmax"};

constexpr float kEps = 1e-5f;  // LayerNorm::new(n_embd, 1e-5) (nn:652, 742)

enum class Op { Leaf, Add, Mul, Matmul, Reshape, Transpose, Gelu, Softmax, LayerNorm, Embedding, CrossEntropy,
                Attention };

struct Node {
  Op op = Op::Leaf;
  std::vector<int> in;        // tape index per input; -1: no gradient flows there
  std::vector<Tensor> saved;  // the inputs (empty for a leaf)
  int d0 = 0, d1 = 0;         // Transpose dims; Softmax: d0 = dim
};

// A tensor and its tape node; `rg` mirrors requires_grad.
struct Var {
  Tensor t;
  int node = -1;
  bool rg = false;
};

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

struct vb_dropin {
  vb_gpt_config c{};
  std::vector<Tensor> P, G, M, V;  // parameters, last gradients, AdamW moments
  Tensor ids, tg, pos, mask, seed, scale;
  bool fused_attention = true;  // MultiHeadAttention's path (nn:603-613)
  bool fold_weight_grads = true;  // the Matmul arm's shared-weight gradient as one product
  int t = 0;
  std::vector<Var> pv;
  std::vector<Node> tape;
  hipStream_t s = nullptr;
  bool timing = false;
  std::vector<hipEvent_t> ev;
  std::vector<int> ev_phase;
  size_t nev = 0;
  double phase_ms[NPHASE] = {};

  ~vb_dropin() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }

  // ------------------------------------------------------------- timing --
  void mark(int phase) {
    if (!timing) return;
    if (nev == ev.size()) {
      hipEvent_t e;
      hip_check(hipEventCreate(&e), "hipEventCreate");
      ev.push_back(e);
      ev_phase.push_back(0);
    }
    hip_check(hipEventRecord(ev[nev], s), "hipEventRecord");
    ev_phase[nev++] = phase;
  }

  void collect() {
    if (!timing || nev < 2) return;
    hip_check(hipEventSynchronize(ev[nev - 1]), "hipEventSynchronize");
    for (size_t i = 1; i < nev; ++i) {
      float ms = 0.f;
      hip_check(hipEventElapsedTime(&ms, ev[i - 1], ev[i]), "hipEventElapsedTime");
      phase_ms[ev_phase[i]] += ms;
    }
  }

  // -------------------------------------------------------------- tape --
  Var rec(Tensor out, Op op, std::initializer_list<Var*> ins, int d0 = 0, int d1 = 0) {
    Var o{std::move(out), -1, false};
    bool any = false;
    for (Var* v : ins) any = any || v->rg;
    if (!any) return o;
    Node n;
    n.op = op;
    n.d0 = d0;
    n.d1 = d1;
    for (Var* v : ins) {
      if (v->node < 0 && v->rg) {  // first use of a parameter: a leaf node
        tape.emplace_back();
        v->node = (int)tape.size() - 1;
      }
      n.in.push_back(v->node);
      n.saved.push_back(v->t);
    }
    tape.push_back(std::move(n));
    o.rg = true;
    o.node = (int)tape.size() - 1;
    return o;
  }

  // ------------------------------------------------- forward (Tensor ops) --
  Var add(Var& a, Var& b) {
    Tensor o = a.t.add(b.t);
    mark(F_ADD);
    return rec(o, Op::Add, {&a, &b});
  }
  Var matmul(Var& a, Var& b) {
    Tensor o = a.t.matmul(b.t);
    mark(F_MATMUL);
    return rec(o, Op::Matmul, {&a, &b});
  }
  Var mul(Var& a, Var& b) {
    Tensor o = a.t.mul(b.t);
    mark(F_MUL);
    return rec(o, Op::Mul, {&a, &b});
  }
  Var softmax(Var& x, int dim) {
    Tensor o = x.t.softmax((size_t)dim);
    mark(F_SOFTMAX);
    return rec(o, Op::Softmax, {&x}, dim);
  }
  Var transpose(Var& a, int d0, int d1) { return rec(a.t.transpose(d0, d1), Op::Transpose, {&a}, d0, d1); }
  Var reshape(Var& a, const Shape& sh) {
    const bool copies = !a.t.is_contiguous();
    Tensor o = a.t.reshape(sh);
    if (copies) mark(F_COPY);
    return rec(o, Op::Reshape, {&a});
  }
  Var layernorm(Var& x, Var& w, Var& b) {
    Tensor o = x.t.layernorm(w.t, b.t, kEps);
    mark(F_LN);
    return rec(o, Op::LayerNorm, {&x, &w, &b});
  }
  Var gelu(Var& x) {
    Tensor o = x.t.gelu();
    mark(F_GELU);
    return rec(o, Op::Gelu, {&x});
  }
  Var embedding(Var& i, Var& w) {
    Tensor o = i.t.embedding(w.t);
    mark(F_EMBED);
    return rec(o, Op::Embedding, {&i, &w});
  }
  Var cross_entropy(Var& logits, Var& targets) {
    Tensor o = logits.t.cross_entropy(targets.t);
    mark(F_XENT);
    return rec(o, Op::CrossEntropy, {&logits, &targets});
  }
  Var attention(Var& q, Var& k, Var& v, Var& m) {
    Tensor o = q.t.fused_attention(k.t, v.t, &m.t);
    mark(F_ATTN);
    return rec(o, Op::Attention, {&q, &k, &v, &m});
  }
  // Linear::forward (nn:119-127): input.matmul(weight.transpose(0, 1)) [+ bias].
  Var linear(Var& x, Var& w, Var* b) {
    Var wt = transpose(w, 0, 1);
    Var o = matmul(x, wt);
    return b ? add(o, *b) : o;
  }

  Var forward() {
    const int64_t B = c.B, S = c.S, D = c.D, H = c.H, Dk = c.D / c.H;
    pv.assign(P.size(), Var{});
    for (size_t i = 0; i < P.size(); ++i) pv[i] = Var{P[i], -1, true};
    Var vids{ids}, vpos{pos}, vtg{tg}, vmask{mask}, vscale{scale};
    // SimpleGPT::forward (nn:745-791)
    Var tok = embedding(vids, pv[0]);
    Var pe = embedding(vpos, pv[1]);
    Var h = add(tok, pe);
    // TransformerBlock::forward (nn:666-675)
    Var x1 = layernorm(h, pv[2], pv[3]);
    // MultiHeadAttention::forward (nn:584-621)
    Var q = linear(x1, pv[4], &pv[5]);
    Var k = linear(x1, pv[6], &pv[7]);
    Var v = linear(x1, pv[8], &pv[9]);
    const Shape heads{B, S, H, Dk};
    Var qr = reshape(q, heads), q4 = transpose(qr, 1, 2);
    Var kr = reshape(k, heads), k4 = transpose(kr, 1, 2);
    Var vr = reshape(v, heads), v4 = transpose(vr, 1, 2);
    Var a;
    if (fused_attention) {
      a = attention(q4, k4, v4, vmask);
    } else {  // nn:604-612
      Var kt = transpose(k4, 2, 3);
      Var raw = matmul(q4, kt);
      Var scaled = mul(raw, vscale);
      Var scores = add(scaled, vmask);
      Var probs = softmax(scores, 3);
      a = matmul(probs, v4);
    }
    Var at = transpose(a, 1, 2);
    Var a3 = reshape(at, Shape{B, S, D});
    Var o = linear(a3, pv[10], &pv[11]);
    Var hx = add(h, o);
    Var x2 = layernorm(hx, pv[12], pv[13]);
    Var f1 = linear(x2, pv[14], &pv[15]);
    Var fg = gelu(f1);
    Var f2 = linear(fg, pv[16], &pv[17]);
    Var hy = add(hx, f2);
    Var xf = layernorm(hy, pv[18], pv[19]);
    Var flat = reshape(xf, Shape{B * S, D});
    Var logits = linear(flat, pv[20], nullptr);
    Var tflat = reshape(vtg, Shape{B * S});
    return cross_entropy(logits, tflat);
  }

  // ------------------------------------------------------------ backward --
  // reduce_to (autograd:316-361): sums a broadcast gradient down to `target`.
  Tensor reduce_to(const Tensor& g, const Shape& target) {
    if (g.shape() == target) return g;
    if (g.shape().numel() == 0) return Tensor::zeros(target, g.device());
    const int gr = g.shape().rank, tr = target.rank;
    if (gr < tr)
      throw vearo_hip::Panic("Grad rank " + std::to_string(gr) + " must be >= target rank " + std::to_string(tr));
    bool trailing = true;
    for (int d = 0; d < tr; ++d) trailing = trailing && target[d] == g.shape()[gr - tr + d];
    Tensor r;
    if (trailing) {  // the leading dims collapse to rows: one column sum
      const int64_t n = target.numel();
      r = g.reshape(Shape{g.shape().numel() / n, n}).sum(0, false).reshape(target);
    } else {
      r = g;
      while (r.shape().rank > tr) r = r.sum(0, false);
      for (int d = 0; d < tr; ++d)
        if (target[d] == 1 && r.shape()[d] != 1) r = r.sum((size_t)d, true);
    }
    mark(B_REDUCE);
    return r;
  }

  void backward(const Var& loss) {
    const int n = (int)tape.size();
    std::vector<Tensor> gm(n);
    std::vector<char> has(n, 0);
    gm[loss.node] = seed;
    has[loss.node] = 1;
    for (int id = n - 1; id >= 0; --id) {
      if (!has[id]) continue;
      Node& nd = tape[id];
      if (nd.saved.empty()) continue;  // a leaf
      const Tensor g = gm[id];
      std::vector<Tensor> gin(nd.in.size());
      switch (nd.op) {
        case Op::Add:
          gin[0] = reduce_to(g, nd.saved[0].shape());
          gin[1] = reduce_to(g, nd.saved[1].shape());
          break;
        case Op::Mul: {  // autograd:480-489
          const Tensor gl = g.mul(nd.saved[1]);
          mark(B_MUL);
          const Tensor gr = g.mul(nd.saved[0]);
          mark(B_MUL);
          gin[0] = reduce_to(gl, nd.saved[0].shape());
          gin[1] = reduce_to(gr, nd.saved[1].shape());
          break;
        }
        case Op::Softmax: {  // autograd:547-553, y recomputed from the saved input
          const size_t dim = (size_t)nd.d0;
          const Tensor y = nd.saved[0].softmax(dim);
          mark(B_SOFTMAX);
          const Tensor gy = g.mul(y);
          mark(B_SOFTMAX);
          const Tensor sgy = gy.sum(dim, true);
          mark(B_SOFTMAX);
          const Tensor d = g.sub(sgy);
          mark(B_SOFTMAX);
          gin[0] = y.mul(d);
          mark(B_SOFTMAX);
          break;
        }
        case Op::Matmul: {
          const Tensor& l = nd.saved[0];
          const Tensor& r = nd.saved[1];
          const int lr = l.shape().rank, rr = r.shape().rank;
          const Tensor lt = l.transpose(lr - 2, lr - 1), rt = r.transpose(rr - 2, rr - 1);
          const Tensor gl = g.matmul(rt);
          mark(B_MATMUL);
          if (fold_weight_grads && rr == 2 && lr > 2 && l.is_contiguous() && g.is_contiguous()) {
            // reduce_to(lᵀ·g, [K, N]) as one product over the B·S rows,
            // computed as its transpose gᵀ·l ([N, K], contiguous) and handed
            // on as a [K, N] view: r is the transposed view of a Linear weight
            // [N, K], so the Transpose arm's view of this is that weight's
            // gradient, contiguous, and AdamW's contiguous() copies nothing.
            const int64_t K = l.shape()[lr - 1], N = g.shape()[g.shape().rank - 1];
            const int64_t rows = l.shape().numel() / K;
            const Tensor gwt = g.reshape(Shape{rows, N}).transpose(0, 1).matmul(l.reshape(Shape{rows, K}));
            gin[1] = gwt.transpose(0, 1);
            mark(B_MATMUL);
          } else {
            const Tensor gr = lt.matmul(g);
            mark(B_MATMUL);
            gin[1] = reduce_to(gr, r.shape());
          }
          gin[0] = reduce_to(gl, l.shape());
          break;
        }
        case Op::Reshape: {
          const bool copies = !g.is_contiguous();
          gin[0] = g.reshape(nd.saved[0].shape());
          if (copies) mark(B_COPY);
          break;
        }
        case Op::Transpose:
          gin[0] = g.transpose(nd.d0, nd.d1);
          break;
        case Op::Gelu:
          gin[0] = vearo_hip::gelu_backward_fused(nd.saved[0], g);
          mark(B_GELU);
          break;
        case Op::LayerNorm: {
          auto [gx, gw, gb] = nd.saved[0].layernorm_backward(nd.saved[1], nd.saved[2], g, kEps);
          mark(B_LN);
          gin[0] = gx;
          gin[1] = gw;
          gin[2] = gb;
          break;
        }
        case Op::Embedding:
          gin[1] = nd.saved[0].embedding_backward(nd.saved[1], g);
          mark(B_EMBED);
          break;
        case Op::CrossEntropy:
          gin[0] = nd.saved[0].cross_entropy_backward(nd.saved[1], g);
          mark(B_XENT);
          break;
        case Op::Attention: {
          auto [dq, dk, dv] = nd.saved[0].fused_attention_backward(nd.saved[1], nd.saved[2], &nd.saved[3], g);
          mark(B_ATTN);
          gin[0] = dq;
          gin[1] = dk;
          gin[2] = dv;
          break;
        }
        case Op::Leaf:
          break;
      }
      gm[id] = Tensor();
      nd.saved.clear();
      for (size_t i = 0; i < nd.in.size(); ++i) {
        const int j = nd.in[i];
        if (j < 0) continue;
        if (has[j]) {
          gm[j] = gm[j].add(gin[i]);
          mark(B_ACC);
        } else {
          gm[j] = gin[i];
          has[j] = 1;
        }
      }
    }
    for (size_t i = 0; i < pv.size(); ++i) {
      const int j = pv[i].node;
      G[i] = (j >= 0 && has[j]) ? gm[j] : Tensor();
    }
  }

  // AdamW::step (optim:105-123).
  // AdamW::step (optim:105-123): every gradient made contiguous, then every
  // parameter updated -- in one vh_adamw_step_multi launch, each element as
  // the per-parameter vh_adamw_step updates it (one launch per parameter left
  // the small ones launch-bound: 21 launches, 0.52-0.60 ms a step).
  void adamw(float lr, float b1, float b2, float eps, float wd) {
    ++t;
    std::vector<float*> ps, ms, vs;
    std::vector<const float*> gs;
    std::vector<int64_t> ns;
    for (size_t i = 0; i < P.size(); ++i) {
      if (!G[i].storage_id()) continue;
      if (!G[i].is_contiguous()) {
        G[i] = G[i].contiguous();
        mark(O_CONTIG);
      }
      ps.push_back(P[i].data());
      gs.push_back(G[i].data());
      ms.push_back(M[i].data());
      vs.push_back(V[i].data());
      ns.push_back(P[i].shape().numel());
    }
    const int rc = vh_adamw_step_multi((int)ps.size(), ps.data(), gs.data(), ms.data(), vs.data(), ns.data(), t, lr,
                                       b1, b2, eps, wd, nullptr);
    if (rc != VH_OK) throw std::runtime_error(std::string("vh_adamw_step_multi: ") + vh_last_error());
    mark(O_ADAMW);
  }
};

namespace {

std::vector<Shape> param_shapes(const vb_gpt_config& c) {
  const int64_t D = c.D, F = c.F, V = c.V, P = c.P;
  return {Shape{V, D}, Shape{P, D}, Shape{D}, Shape{D}, Shape{D, D}, Shape{D}, Shape{D, D},
          Shape{D},    Shape{D, D}, Shape{D}, Shape{D, D}, Shape{D}, Shape{D}, Shape{D},
          Shape{F, D}, Shape{F},    Shape{D, F}, Shape{D}, Shape{D}, Shape{D}, Shape{V, D}};
}

template <class F>
int guarded(const char* fn, F f) {
  try {
    f();
    return VH_OK;
  } catch (const vearo_hip::Panic& e) {
    return vb_fail(VH_ERR_INVALID, std::string(fn) + ": " + e.what());
  } catch (const std::exception& e) {
    return vb_fail(VH_ERR_HIP, std::string(fn) + ": " + e.what());
  }
}

void vh_ok(int rc, const char* what) {
  if (rc != VH_OK) throw std::runtime_error(std::string(what) + ": " + vh_last_error());
}

}  // namespace

extern "C" {

int vb_dropin_create(const vb_gpt_config* cfg, vb_dropin** out) {
  if (!cfg || !out) return vb_fail(VH_ERR_INVALID, "vb_dropin_create: null pointer");
  const vb_gpt_config c = *cfg;
  if (c.B <= 0 || c.S <= 0 || c.D <= 0 || c.H <= 0 || c.F <= 0 || c.V <= 0 || c.P <= 0)
    return vb_fail(VH_ERR_INVALID, "vb_dropin_create: sizes must be positive");
  if (c.D % c.H != 0) return vb_fail(VH_ERR_INVALID, "n_embd must be divisible by n_head");
  if (c.S > c.P) return vb_fail(VH_ERR_INVALID, "vb_dropin_create: sequence longer than max_seq_len");
  vb_dropin* d = nullptr;
  const int rc = guarded("vb_dropin_create", [&] {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    vearo_hip::init(dev);
    d = new vb_dropin();
    d->c = c;
    d->s = static_cast<hipStream_t>(vh_stream());
    const std::vector<Shape> shapes = param_shapes(c);
    for (size_t i = 0; i < shapes.size(); ++i) {
      d->P.push_back(Tensor::zeros(shapes[i]));
      d->M.push_back(Tensor::zeros(shapes[i]));
      d->V.push_back(Tensor::zeros(shapes[i]));
    }
    d->G.assign(shapes.size(), Tensor());
    for (int i : {2, 12, 18})  // LayerNorm weights start at 1 (nn:521)
      d->P[i] = Tensor::from_f32(std::vector<float>((size_t)c.D, 1.0f), shapes[i]);
    d->ids = Tensor::zeros(Shape{c.B, c.S});
    d->tg = Tensor::zeros(Shape{c.B, c.S});
    std::vector<float> pos((size_t)(c.B * c.S));
    for (int64_t r = 0; r < c.B; ++r)
      for (int64_t j = 0; j < c.S; ++j) pos[(size_t)(r * c.S + j)] = (float)j;
    d->pos = Tensor::from_f32(pos, Shape{c.B, c.S});
    std::vector<float> mask((size_t)(c.S * c.S), 0.0f);
    for (int64_t r = 0; r < c.S; ++r)
      for (int64_t j = r + 1; j < c.S; ++j) mask[(size_t)(r * c.S + j)] = -1e9f;
    d->mask = Tensor::from_f32(mask, Shape{c.S, c.S});
    d->seed = Tensor::from_f32({1.0f}, Shape{1});
    d->scale = Tensor::from_f32({1.0f / std::sqrt((float)(c.D / c.H))}, Shape{1});
    // nn:603: the fused path unless VEARO_USE_FUSED_ATTENTION is "0" or "false".
    const char* env = std::getenv("VEARO_USE_FUSED_ATTENTION");
    d->fused_attention = !(env && (std::strcmp(env, "0") == 0 || std::strcmp(env, "false") == 0));
  });
  if (rc != VH_OK) {
    delete d;
    return rc;
  }
  *out = d;
  return VH_OK;
}

void vb_dropin_destroy(vb_dropin* d) { delete d; }

int vb_dropin_set_fused_attention(vb_dropin* d, int fused) {
  if (!d) return vb_fail(VH_ERR_INVALID, "vb_dropin_set_fused_attention: null handle");
  d->fused_attention = fused != 0;
  return VH_OK;
}

int vb_dropin_fused_attention(const vb_dropin* d) { return d && d->fused_attention ? 1 : 0; }

int vb_dropin_set_fold_weight_grads(vb_dropin* d, int fold) {
  if (!d) return vb_fail(VH_ERR_INVALID, "vb_dropin_set_fold_weight_grads: null handle");
  d->fold_weight_grads = fold != 0;
  return VH_OK;
}

int vb_dropin_fold_weight_grads(const vb_dropin* d) { return d && d->fold_weight_grads ? 1 : 0; }

int vb_dropin_set_param(vb_dropin* d, int i, const float* host, int64_t numel) {
  if (!d || !host || i < 0 || i >= VB_GPT_NPARAMS) return vb_fail(VH_ERR_INVALID, "vb_dropin_set_param: bad argument");
  if (numel != d->P[i].shape().numel()) return vb_fail(VH_ERR_INVALID, "vb_dropin_set_param: element count differs");
  return guarded("vb_dropin_set_param",
                 [&] { vh_ok(vh_h2d(d->P[i].data(), host, (size_t)numel * sizeof(float)), "vh_h2d"); });
}

int vb_dropin_get_param(vb_dropin* d, int i, float* host, int64_t numel) {
  if (!d || !host || i < 0 || i >= VB_GPT_NPARAMS) return vb_fail(VH_ERR_INVALID, "vb_dropin_get_param: bad argument");
  if (numel != d->P[i].shape().numel()) return vb_fail(VH_ERR_INVALID, "vb_dropin_get_param: element count differs");
  return guarded("vb_dropin_get_param", [&] {
    const std::vector<float> v = d->P[i].to_vec_f32();
    std::memcpy(host, v.data(), v.size() * sizeof(float));
  });
}

int vb_dropin_get_grad(vb_dropin* d, int i, float* host, int64_t numel) {
  if (!d || !host || i < 0 || i >= VB_GPT_NPARAMS) return vb_fail(VH_ERR_INVALID, "vb_dropin_get_grad: bad argument");
  if (!d->G[i].storage_id()) return vb_fail(VH_ERR_INVALID, "vb_dropin_get_grad: no gradient (run a backward)");
  if (numel != d->G[i].shape().numel()) return vb_fail(VH_ERR_INVALID, "vb_dropin_get_grad: element count differs");
  return guarded("vb_dropin_get_grad", [&] {
    const std::vector<float> v = d->G[i].to_vec_f32();
    std::memcpy(host, v.data(), v.size() * sizeof(float));
  });
}

int vb_dropin_set_inputs(vb_dropin* d, const float* ids, const float* targets) {
  if (!d || !ids || !targets) return vb_fail(VH_ERR_INVALID, "vb_dropin_set_inputs: null pointer");
  const size_t bytes = (size_t)(d->c.B * d->c.S) * sizeof(float);
  return guarded("vb_dropin_set_inputs", [&] {
    vh_ok(vh_h2d(d->ids.data(), ids, bytes), "vh_h2d");
    vh_ok(vh_h2d(d->tg.data(), targets, bytes), "vh_h2d");
  });
}

int vb_dropin_step(vb_dropin* d, int backward, int adamw, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int timing, float* loss) {
  if (!d) return vb_fail(VH_ERR_INVALID, "vb_dropin_step: null handle");
  if (adamw && !backward) return vb_fail(VH_ERR_INVALID, "vb_dropin_step: AdamW needs the backward's gradients");
  const int rc = guarded("vb_dropin_step", [&] {
    d->timing = timing != 0;
    d->nev = 0;
    if (d->timing) {
      std::memset(d->phase_ms, 0, sizeof(d->phase_ms));
      d->mark(0);
    }
    d->tape.clear();
    const Var l = d->forward();
    if (backward) d->backward(l);
    d->tape.clear();
    if (adamw) d->adamw(lr, beta1, beta2, eps, weight_decay);
    d->collect();
    if (loss) {
      const std::vector<float> v = l.t.to_vec_f32();
      *loss = v[0];
    }
  });
  d->tape.clear();
  d->timing = false;
  return rc;
}

int vb_dropin_phase_ms(vb_dropin* d, double* ms, int n) {
  if (!d || !ms || n < NPHASE) return vb_fail(VH_ERR_INVALID, "vb_dropin_phase_ms: bad argument");
  for (int i = 0; i < NPHASE; ++i) ms[i] = d->phase_ms[i];
  return VH_OK;
}

const char* vb_dropin_phase_name(int i) { return (i >= 0 && i < NPHASE) ? kPhase[i] : nullptr; }

}  // extern "C"
