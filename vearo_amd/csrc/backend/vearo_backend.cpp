// vearo_backend.cpp -- the HIP BackendOps table over the C ABI of libvearo_hip.so.
//
// Each slot follows the reference CPU backend's contract
// (crates/vearo-backend-cpu/src/lib.rs): validate shapes with the same panic
// messages, return a fresh contiguous tensor, accept strided inputs. Strided
// inputs are gathered on the device (vh_strided_copy) instead of the host
// round-trip the CUDA backend takes (tensor.rs:349-368), and binary ops and
// reductions read strided operands directly.
#include "vearo_backend.h"

#include <algorithm>
#include <mutex>
#include <sstream>

#include "../../../include/vearo_hip.h"

namespace vearo_hip {

namespace {

void check(int rc) {
  if (rc == VH_OK) return;
  const std::string msg = vh_last_error();
  if (rc == VH_ERR_DEVICE_PANIC) throw Panic(msg);
  throw std::runtime_error("vearo-backend-hip: " + msg);
}

void panic_if(bool cond, const std::string& msg) {
  if (cond) throw Panic(msg);
}

vh_layout layout_of(const Tensor& t) {
  vh_layout l{};
  l.rank = t.shape().rank;
  for (int i = 0; i < l.rank; ++i) {
    l.dims[i] = t.shape()[i];
    l.strides[i] = t.strides()[i];
  }
  return l;
}

std::mutex g_ops_mu;
const BackendOps* g_ops[NUM_BACKENDS] = {nullptr, nullptr, nullptr, nullptr};

}  // namespace

// ------------------------------------------------------------------ Shape --

Shape::Shape(std::initializer_list<int64_t> dims) : Shape(std::vector<int64_t>(dims)) {}

Shape::Shape(const std::vector<int64_t>& dims) {
  panic_if((int)dims.size() > MAX_RANK, "Vearo only supports shapes up to rank 8, but got rank " +
                                            std::to_string(dims.size()));
  rank = (int)dims.size();
  for (int i = 0; i < rank; ++i) d[i] = dims[i];
}

int64_t Shape::numel() const {
  int64_t n = 1;
  for (int i = 0; i < rank; ++i) n *= d[i];
  return n;
}

Shape Shape::contiguous_strides() const {
  Shape s;
  s.rank = rank;
  int64_t acc = 1;
  for (int i = rank - 1; i >= 0; --i) {
    s.d[i] = acc;
    acc *= d[i];
  }
  return s;
}

bool Shape::operator==(const Shape& o) const {
  if (rank != o.rank) return false;
  for (int i = 0; i < rank; ++i)
    if (d[i] != o.d[i]) return false;
  return true;
}

std::string Shape::str() const {
  std::ostringstream os;
  os << "[";
  for (int i = 0; i < rank; ++i) os << (i ? ", " : "") << d[i];
  os << "]";
  return os.str();
}

// ---------------------------------------------------------------- Storage --

Storage::~Storage() {
  if (ptr) vh_free(ptr);
}

static std::shared_ptr<Storage> alloc_storage(int64_t numel, bool zero) {
  auto s = std::make_shared<Storage>();
  s->bytes = (size_t)std::max<int64_t>(numel, 1) * sizeof(float);
  check(vh_alloc(s->bytes, zero ? 1 : 0, &s->ptr));
  return s;
}

// ----------------------------------------------------------------- Tensor --

Tensor make_view(const Tensor& base, const Shape& shape, const Shape& strides) {
  Tensor t;
  t.storage_ = base.storage_;
  t.shape_ = shape;
  t.strides_ = strides;
  t.device_ = base.device_;
  return t;
}

Tensor Tensor::zeros(const Shape& s, Device dev) {
  Tensor t;
  t.storage_ = alloc_storage(s.numel(), true);
  t.shape_ = s;
  t.strides_ = s.contiguous_strides();
  t.device_ = dev;
  return t;
}

Tensor Tensor::empty(const Shape& s, Device dev) {
  Tensor t;
  t.storage_ = alloc_storage(s.numel(), false);
  t.shape_ = s;
  t.strides_ = s.contiguous_strides();
  t.device_ = dev;
  return t;
}

Tensor Tensor::from_f32(const std::vector<float>& data, const Shape& s, Device dev) {
  panic_if((int64_t)data.size() != s.numel(), "Data length must match shape");
  Tensor t = empty(s, dev);
  check(vh_h2d(t.storage_->ptr, data.data(), data.size() * sizeof(float)));
  return t;
}

bool Tensor::is_contiguous() const { return strides_ == shape_.contiguous_strides(); }

Tensor Tensor::transpose(int a, int b) const {
  Shape s = shape_, st = strides_;
  std::swap(s.d[a], s.d[b]);
  std::swap(st.d[a], st.d[b]);
  return make_view(*this, s, st);
}

Tensor Tensor::permute(const std::vector<int>& axes) const {
  panic_if((int)axes.size() != shape_.rank, "Number of permutation axes must match rank");
  Shape s, st;
  s.rank = st.rank = shape_.rank;
  unsigned seen = 0;
  for (int i = 0; i < shape_.rank; ++i) {
    panic_if(axes[i] < 0 || axes[i] >= shape_.rank, "Axis index out of bounds");
    panic_if(seen & (1u << axes[i]), "Duplicate permutation axes are not allowed");
    seen |= 1u << axes[i];
    s.d[i] = shape_.d[axes[i]];
    st.d[i] = strides_.d[axes[i]];
  }
  return make_view(*this, s, st);
}

Tensor Tensor::reshape(const Shape& s) const {
  panic_if(s.numel() != shape_.numel(), "Reshape must preserve the number of elements");
  const Tensor src = is_contiguous() ? *this : contiguous();
  return make_view(src, s, s.contiguous_strides());
}

Tensor Tensor::contiguous() const {
  if (is_contiguous()) return *this;
  Tensor out = empty(shape_, device_);
  const vh_layout l = layout_of(*this);
  check(vh_strided_copy(data(), &l, out.data(), nullptr));
  return out;
}

std::vector<float> Tensor::to_vec_f32() const {
  const Tensor c = contiguous();
  std::vector<float> v((size_t)shape_.numel());
  check(vh_sync());
  if (!v.empty()) check(vh_d2h(v.data(), c.data(), v.size() * sizeof(float)));
  return v;
}

static const BackendOps& ops_for(Device d) {
  const BackendOps* o = get_backend_ops(d);
  if (!o) throw Panic("No backend registered for this device. Did you call the backend's init()?");
  return *o;
}

Tensor Tensor::add(const Tensor& o) const { return ops_for(device_).add(*this, o); }
Tensor Tensor::sub(const Tensor& o) const { return ops_for(device_).sub(*this, o); }
Tensor Tensor::mul(const Tensor& o) const { return ops_for(device_).mul(*this, o); }
Tensor Tensor::div(const Tensor& o) const { return ops_for(device_).div(*this, o); }
Tensor Tensor::sum(size_t dim, bool keep) const { return ops_for(device_).sum(*this, dim, keep); }
Tensor Tensor::mean(size_t dim, bool keep) const { return ops_for(device_).mean(*this, dim, keep); }
Tensor Tensor::gelu() const { return ops_for(device_).gelu(*this); }
Tensor Tensor::softmax(size_t dim) const { return ops_for(device_).softmax(*this, dim); }
Tensor Tensor::layernorm(const Tensor& w, const Tensor& b, float eps) const {
  return ops_for(device_).layernorm(*this, w, b, eps);
}
std::tuple<Tensor, Tensor, Tensor> Tensor::layernorm_backward(const Tensor& w, const Tensor& b,
                                                              const Tensor& g, float eps) const {
  return ops_for(device_).layernorm_backward(*this, w, b, g, eps);
}
// Embedding dispatches on the ids' device (tensor.rs:1655-1669).
Tensor Tensor::embedding(const Tensor& w) const { return ops_for(device_).embedding(*this, w); }
Tensor Tensor::embedding_backward(const Tensor& w, const Tensor& g) const {
  return ops_for(device_).embedding_backward(*this, w, g);
}
Tensor Tensor::cross_entropy(const Tensor& t) const { return ops_for(device_).cross_entropy(*this, t); }
Tensor Tensor::cross_entropy_backward(const Tensor& t, const Tensor& g) const {
  return ops_for(device_).cross_entropy_backward(*this, t, g);
}
Tensor Tensor::matmul(const Tensor& o) const {
  panic_if(!(o.device() == device_), "Tensors must reside on the same device");
  return ops_for(device_).matmul(*this, o);
}
Tensor Tensor::fused_attention(const Tensor& k, const Tensor& v, const Tensor* mask) const {
  return ops_for(device_).fused_attention(*this, k, v, mask);
}
std::tuple<Tensor, Tensor, Tensor> Tensor::fused_attention_backward(const Tensor& k, const Tensor& v,
                                                                    const Tensor* mask,
                                                                    const Tensor& g) const {
  return ops_for(device_).fused_attention_backward(*this, k, v, mask, g);
}

// ------------------------------------------------------------- registry --

void register_backend_ops(Device device, const BackendOps& ops) {
  std::lock_guard<std::mutex> lk(g_ops_mu);
  const int i = device.backend_idx();
  if (!g_ops[i]) g_ops[i] = new BackendOps(ops);
}

const BackendOps* get_backend_ops(Device device) {
  std::lock_guard<std::mutex> lk(g_ops_mu);
  return g_ops[device.backend_idx()];
}

void synchronize() { check(vh_sync()); }

// ============================================================ HIP ops ===
namespace ops {

static Tensor binary(int op, const Tensor& l, const Tensor& r) {
  // Shape::broadcast (shape.rs:91-124).
  const int R = std::max(l.shape().rank, r.shape().rank);
  std::vector<int64_t> od(R);
  for (int i = 0; i < R; ++i) {
    const int li = l.shape().rank - R + i, ri = r.shape().rank - R + i;
    const int64_t a = li >= 0 ? l.shape()[li] : 1, b = ri >= 0 ? r.shape()[ri] : 1;
    panic_if(!(a == b || a == 1 || b == 1), "Shapes are not broadcastable");
    od[i] = a == 1 ? b : a;
  }
  Tensor out = Tensor::empty(Shape(od), l.device());
  if (out.shape().numel() == 0) return out;
  const vh_layout ll = layout_of(l), rl = layout_of(r);
  check(vh_binary(op, l.data(), &ll, r.data(), &rl, out.data(), nullptr));
  return out;
}
Tensor add(const Tensor& l, const Tensor& r) { return binary(VH_OP_ADD, l, r); }
Tensor sub(const Tensor& l, const Tensor& r) { return binary(VH_OP_SUB, l, r); }
Tensor mul(const Tensor& l, const Tensor& r) { return binary(VH_OP_MUL, l, r); }
Tensor div(const Tensor& l, const Tensor& r) { return binary(VH_OP_DIV, l, r); }

static Tensor reduce(const Tensor& x, size_t dim, bool keep, int mean) {
  panic_if((int)dim >= x.shape().rank, "Reduction dim out of range");
  std::vector<int64_t> od = x.shape().dims();
  if (keep) od[dim] = 1;
  else od.erase(od.begin() + dim);
  Tensor out = Tensor::zeros(Shape(od), x.device());
  if (out.shape().numel() == 0) return out;
  const vh_layout l = layout_of(x);
  check(vh_reduce(mean, x.data(), &l, (int)dim, out.data(), nullptr));
  return out;
}
Tensor sum(const Tensor& x, size_t dim, bool keep) { return reduce(x, dim, keep, 0); }
Tensor mean(const Tensor& x, size_t dim, bool keep) { return reduce(x, dim, keep, 1); }

Tensor gelu(const Tensor& x) {
  Tensor out = Tensor::empty(x.shape(), x.device());
  const int64_t n = x.shape().numel();
  if (n == 0) return out;
  const Tensor xc = x.contiguous();
  check(vh_gelu_fwd(xc.data(), out.data(), n, nullptr));
  return out;
}

Tensor softmax(const Tensor& x, size_t dim) {
  const int rank = x.shape().rank;
  panic_if((int)dim >= rank, "Softmax dim out of range");
  Tensor out = Tensor::empty(x.shape(), x.device());
  if (x.shape().numel() == 0) return out;
  if ((int)dim == rank - 1) {
    const Tensor xc = x.contiguous();
    const int64_t T = x.shape()[rank - 1];
    check(vh_softmax_fwd(xc.data(), out.data(), x.shape().numel() / T, T, 0, nullptr));
    return out;
  }
  // Move `dim` last, run the row kernel, move it back.
  std::vector<int> perm;
  for (int i = 0; i < rank; ++i)
    if (i != (int)dim) perm.push_back(i);
  perm.push_back((int)dim);
  const Tensor moved = x.permute(perm).contiguous();
  const Tensor y = softmax(moved, rank - 1);
  std::vector<int> inv(rank);
  for (int i = 0; i < rank; ++i) inv[perm[i]] = i;
  return y.permute(inv).contiguous();
}

static void ln_checks(const Tensor& x, const Tensor& w, const Tensor& b) {
  panic_if(x.shape().rank < 1, "LayerNorm input must be at least rank 1");
  const int64_t C = x.shape()[x.shape().rank - 1];
  panic_if(w.shape().rank != 1, "LayerNorm weight must be rank 1");
  panic_if(b.shape().rank != 1, "LayerNorm bias must be rank 1");
  panic_if(w.shape()[0] != C, "Weight dimension must match norm_dim");
  panic_if(b.shape()[0] != C, "Bias dimension must match norm_dim");
}

Tensor layernorm(const Tensor& x, const Tensor& w, const Tensor& b, float eps) {
  Tensor out = Tensor::empty(x.shape(), x.device());
  if (x.shape().numel() == 0) return out;
  ln_checks(x, w, b);
  const int64_t C = x.shape()[x.shape().rank - 1];
  const Tensor xc = x.contiguous(), wc = w.contiguous(), bc = b.contiguous();
  check(vh_layernorm_fwd(xc.data(), wc.data(), bc.data(), out.data(), x.shape().numel() / C, C, eps,
                         nullptr));
  return out;
}

std::tuple<Tensor, Tensor, Tensor> layernorm_backward(const Tensor& x, const Tensor& w, const Tensor& b,
                                                      const Tensor& g, float eps) {
  if (x.shape().numel() == 0)
    return {Tensor::zeros(x.shape(), x.device()), Tensor::zeros(w.shape(), w.device()),
            Tensor::zeros(b.shape(), b.device())};
  ln_checks(x, w, b);
  // vh_layernorm_bwd writes every element of the three gradients.
  Tensor gx = Tensor::empty(x.shape(), x.device());
  Tensor gw = Tensor::empty(w.shape(), w.device());
  Tensor gb = Tensor::empty(b.shape(), b.device());
  const int64_t C = x.shape()[x.shape().rank - 1];
  const Tensor xc = x.contiguous(), wc = w.contiguous(), gc = g.contiguous();
  check(vh_layernorm_bwd(xc.data(), wc.data(), gc.data(), gx.data(), gw.data(), gb.data(),
                         x.shape().numel() / C, C, eps, nullptr, 0, nullptr));
  return {gx, gw, gb};
}

Tensor embedding(const Tensor& ids, const Tensor& w) {
  panic_if(w.shape().rank != 2, "Weight must be rank 2 (vocab_size, embedding_dim)");
  const int64_t V = w.shape()[0], D = w.shape()[1];
  std::vector<int64_t> od = ids.shape().dims();
  od.push_back(D);
  Tensor out = Tensor::empty(Shape(od), ids.device());
  const int64_t n = ids.shape().numel();
  if (n == 0) return out;
  const Tensor ic = ids.contiguous(), wc = w.contiguous();
  check(vh_embedding_fwd(ic.data(), wc.data(), out.data(), n, V, D, nullptr));
  return out;
}

Tensor embedding_backward(const Tensor& ids, const Tensor& w, const Tensor& g) {
  panic_if(w.shape().rank != 2, "Weight must be rank 2 (vocab_size, embedding_dim)");
  const int64_t V = w.shape()[0], D = w.shape()[1];
  std::vector<int64_t> expect = ids.shape().dims();
  expect.push_back(D);
  panic_if(g.shape() != Shape(expect), "grad_out shape must be x.shape() + [embedding_dim]");
  Tensor gw = Tensor::empty(w.shape(), w.device());
  const Tensor ic = ids.contiguous(), gc = g.contiguous();
  check(vh_embedding_bwd(ic.data(), gc.data(), gw.data(), ids.shape().numel(), V, D, nullptr, 0, nullptr));
  return gw;
}

static void ce_checks(const Tensor& logits, const Tensor& targets) {
  panic_if(logits.shape().rank != 2, "Logits must be rank 2 (batch_size, vocab_size)");
  panic_if(targets.shape().rank != 1, "Targets must be rank 1 (batch_size)");
  panic_if(logits.shape()[0] <= 0, "Batch size must be greater than 0");
  panic_if(targets.shape()[0] != logits.shape()[0], "Targets shape must match batch size");
}

Tensor cross_entropy(const Tensor& logits, const Tensor& targets) {
  ce_checks(logits, targets);
  const int64_t B = logits.shape()[0], V = logits.shape()[1];
  Tensor loss = Tensor::empty(Shape{1}, logits.device());
  const Tensor lc = logits.contiguous(), tc = targets.contiguous();
  check(vh_cross_entropy_fwd(lc.data(), tc.data(), loss.data(), B, V, nullptr, 0, nullptr));
  return loss;
}

Tensor cross_entropy_backward(const Tensor& logits, const Tensor& targets, const Tensor& g) {
  ce_checks(logits, targets);
  panic_if(g.shape().numel() != 1, "grad_out must be a scalar");
  const int64_t B = logits.shape()[0], V = logits.shape()[1];
  Tensor out = Tensor::empty(logits.shape(), logits.device());
  const Tensor lc = logits.contiguous(), tc = targets.contiguous(), gc = g.contiguous();
  check(vh_cross_entropy_bwd(lc.data(), tc.data(), gc.data(), out.data(), B, V, nullptr));
  return out;
}

[[noreturn]] static void out_of_scope(const char* op) {
  throw Panic(std::string("vearo-backend-hip: ") + op +
              " is not part of this backend (fused layer kernels only)");
}
// cpu:266-417: batched matmul with broadcast batch dims; a fresh contiguous
// output (zeros when it is empty).
Tensor matmul(const Tensor& l, const Tensor& r) {
  const int lr = l.shape().rank, rr = r.shape().rank;
  panic_if(lr < 2 || rr < 2, "Matmul requires rank >= 2");
  const int64_t M = l.shape()[lr - 2], K = l.shape()[lr - 1], K2 = r.shape()[rr - 2], N = r.shape()[rr - 1];
  panic_if(K != K2, "Incompatible dimensions for matmul");
  const int lb = lr - 2, rb = rr - 2, ob = std::max(lb, rb);
  std::vector<int64_t> od(ob);
  for (int i = 0; i < ob; ++i) {
    const int li = i - (ob - lb), ri = i - (ob - rb);
    const int64_t a = li >= 0 ? l.shape()[li] : 1, b = ri >= 0 ? r.shape()[ri] : 1;
    panic_if(!(a == b || a == 1 || b == 1), "Batch shapes are not broadcastable");
    od[i] = std::max(a, b);
  }
  od.push_back(M);
  od.push_back(N);
  // vh_matmul writes every output element (K == 0 gives zeros); an empty
  // product returns the zeros tensor the reference returns.
  const Shape os(od);
  if (os.numel() == 0) return Tensor::zeros(os, l.device());
  Tensor out = Tensor::empty(os, l.device());
  const vh_layout ll = layout_of(l), rl = layout_of(r);
  check(vh_matmul(l.data(), &ll, r.data(), &rl, out.data(), nullptr));
  return out;
}

Tensor relu(const Tensor&) { out_of_scope("relu"); }
Tensor conv2d(const Tensor&, const Tensor&, const Tensor&, size_t, size_t) { out_of_scope("conv2d"); }
std::tuple<Tensor, Tensor, Tensor> conv2d_backward(const Tensor&, const Tensor&, const Tensor&, size_t,
                                                   size_t) {
  out_of_scope("conv2d_backward");
}
Tensor maxpool2d(const Tensor&, size_t, size_t, size_t) { out_of_scope("maxpool2d"); }
Tensor maxpool2d_backward(const Tensor&, const Tensor&, size_t, size_t, size_t) {
  out_of_scope("maxpool2d_backward");
}
Tensor avgpool2d(const Tensor&, size_t, size_t, size_t) { out_of_scope("avgpool2d"); }
Tensor avgpool2d_backward(const Tensor&, const Tensor&, size_t, size_t, size_t) {
  out_of_scope("avgpool2d_backward");
}
Tensor batchnorm(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, bool, float,
                 float) {
  out_of_scope("batchnorm");
}
std::tuple<Tensor, Tensor, Tensor> batchnorm_backward(const Tensor&, const Tensor&, const Tensor&,
                                                      const Tensor&, const Tensor&, const Tensor&, bool,
                                                      float) {
  out_of_scope("batchnorm_backward");
}
// Operands of the attention kernels need a unit stride on the last dim.
static Tensor unit_last(const Tensor& t) {
  const int r = t.shape().rank;
  return (r > 0 && t.strides()[r - 1] != 1 && t.shape()[r - 1] != 1) ? t.contiguous() : t;
}

static void attention_checks(const Tensor& q, const Tensor& k, const Tensor& v) {
  // cpu:2376-2383: [B, H, S, Dk] and k, v of q's shape.
  panic_if(q.shape().rank != 4, "fused attention expects [B, H, S, Dk]");
  panic_if(k.shape() != q.shape(), "assertion `left == right` failed: k shape " + k.shape().str() +
                                       " != q shape " + q.shape().str());
  panic_if(v.shape() != q.shape(), "assertion `left == right` failed: v shape " + v.shape().str() +
                                       " != q shape " + q.shape().str());
}

// An additive mask that is the causal triangle (exact zeros on and below the
// diagonal, at most -1 above) with scores small enough that every masked
// exponent underflows to exactly 0 -- SimpleGPT's -1e9 mask (nn:763-771) with
// any ordinary activations -- gives the same bits as the causal kernels,
// which skip the masked blocks. With a mask the slots ask for
// VH_ATTN_CAUSAL_AUTO: one pass over the operands and the mask proves that
// per call on the device, and the launches choose their form from its flag
// (no host wait).
static int causal_mode(const float* mask) { return mask ? VH_ATTN_CAUSAL_AUTO : 0; }

// cpu:2366-2464: softmax(q k^T / sqrt(Dk) + mask) v, mask broadcast from the right.
Tensor fused_attention(const Tensor& q0, const Tensor& k0, const Tensor& v0, const Tensor* mask) {
  attention_checks(q0, k0, v0);
  const Tensor q = unit_last(q0), k = unit_last(k0), v = unit_last(v0);
  if (q.shape().numel() == 0) return Tensor::zeros(q.shape(), q.device());
  Tensor out = Tensor::empty(q.shape(), q.device());  // the P v product writes all of it
  const vh_layout ql = layout_of(q), kl = layout_of(k), vl = layout_of(v), ol = layout_of(out);
  vh_layout ml{};
  if (mask) ml = layout_of(*mask);
  const float* mp = mask ? mask->data() : nullptr;
  check(vh_fused_attention_fwd(q.data(), &ql, k.data(), &kl, v.data(), &vl, mp, mp ? &ml : nullptr,
                               causal_mode(mp), out.data(), &ol, nullptr, 0, nullptr));
  return out;
}

// cpu:2467-2630: (dq, dk, dv), recomputing the probabilities from q and k.
std::tuple<Tensor, Tensor, Tensor> fused_attention_backward(const Tensor& q0, const Tensor& k0,
                                                            const Tensor& v0, const Tensor* mask,
                                                            const Tensor& g0) {
  attention_checks(q0, k0, v0);
  panic_if(g0.shape() != q0.shape(), "grad_out must have the attention output's shape");
  const Tensor q = unit_last(q0), k = unit_last(k0), v = unit_last(v0), g = unit_last(g0);
  if (q.shape().numel() == 0)
    return {Tensor::zeros(q.shape(), q.device()), Tensor::zeros(q.shape(), q.device()),
            Tensor::zeros(q.shape(), q.device())};
  // Each gradient is one product that writes all of it.
  Tensor dq = Tensor::empty(q.shape(), q.device()), dk = Tensor::empty(q.shape(), q.device()),
         dv = Tensor::empty(q.shape(), q.device());
  const vh_layout ql = layout_of(q), kl = layout_of(k), vl = layout_of(v), gl = layout_of(g),
                  dl = layout_of(dq);
  vh_layout ml{};
  if (mask) ml = layout_of(*mask);
  const float* mp = mask ? mask->data() : nullptr;
  check(vh_fused_attention_bwd(q.data(), &ql, k.data(), &kl, v.data(), &vl, mp, mp ? &ml : nullptr,
                               causal_mode(mp), g.data(), &gl, dq.data(), &dl, dk.data(), &dl, dv.data(), &dl,
                               nullptr, 0, nullptr));
  return {dq, dk, dv};
}

}  // namespace ops

BackendOps hip_backend_ops() {
  BackendOps o;
  o.add = ops::add;
  o.sub = ops::sub;
  o.mul = ops::mul;
  o.div = ops::div;
  o.matmul = ops::matmul;
  o.relu = ops::relu;
  o.sum = ops::sum;
  o.mean = ops::mean;
  o.gelu = ops::gelu;
  o.softmax = ops::softmax;
  o.layernorm = ops::layernorm;
  o.layernorm_backward = ops::layernorm_backward;
  o.embedding = ops::embedding;
  o.embedding_backward = ops::embedding_backward;
  o.cross_entropy = ops::cross_entropy;
  o.cross_entropy_backward = ops::cross_entropy_backward;
  o.conv2d = ops::conv2d;
  o.conv2d_backward = ops::conv2d_backward;
  o.maxpool2d = ops::maxpool2d;
  o.maxpool2d_backward = ops::maxpool2d_backward;
  o.avgpool2d = ops::avgpool2d;
  o.avgpool2d_backward = ops::avgpool2d_backward;
  o.batchnorm = ops::batchnorm;
  o.batchnorm_backward = ops::batchnorm_backward;
  o.fused_attention = ops::fused_attention;
  o.fused_attention_backward = ops::fused_attention_backward;
  return o;
}

void init(int device) {
  check(vh_init(device));
  register_backend_ops(Device::hip(device), hip_backend_ops());
}

// The Softmax arm (autograd lib.rs:547-553) exactly as dispatched there.
Tensor softmax_backward_arm(const Tensor& x, const Tensor& grad_out, size_t dim) {
  const Tensor y = x.softmax(dim);
  const Tensor sum_grad_y = grad_out.mul(y).sum(dim, true);
  return y.mul(grad_out.sub(sum_grad_y));
}

Tensor softmax_backward_fused(const Tensor& x, const Tensor& grad_out) {
  const int rank = x.shape().rank;
  panic_if(rank < 1, "Softmax dim out of range");
  Tensor out = Tensor::empty(x.shape(), x.device());
  if (x.shape().numel() == 0) return out;
  const int64_t T = x.shape()[rank - 1];
  const Tensor xc = x.contiguous(), gc = grad_out.contiguous();
  check(vh_softmax_bwd(xc.data(), gc.data(), out.data(), x.shape().numel() / T, T, 1, 0, nullptr));
  return out;
}

namespace {
// The checkpoint entries report the reference's panics as VH_ERR_INVALID with
// the panic text, and its io::Errors as VH_ERR_IO.
void check_checkpoint(int rc) {
  if (rc == VH_OK) return;
  const std::string msg = vh_last_error();
  if (rc == VH_ERR_IO) throw IoError(msg);
  if (rc == VH_ERR_INVALID) throw Panic(msg);
  check(rc);
}
}  // namespace

void save_checkpoint(const std::vector<Tensor>& params, const std::string& path) {
  std::vector<const float*> ptrs;
  std::vector<vh_layout> lays;
  for (const Tensor& t : params) {
    ptrs.push_back(t.data());
    lays.push_back(layout_of(t));
  }
  check_checkpoint(vh_checkpoint_save(path.c_str(), (int32_t)params.size(), ptrs.data(), lays.data(), nullptr));
}

void load_checkpoint(const std::vector<Tensor>& params, const std::string& path) {
  std::vector<float*> ptrs;
  std::vector<vh_layout> lays;
  for (Tensor t : params) {  // a handle copy shares the storage it writes
    ptrs.push_back(t.data());
    lays.push_back(layout_of(t));
  }
  check_checkpoint(vh_checkpoint_load(path.c_str(), (int32_t)params.size(), ptrs.data(), lays.data(), nullptr));
}

Tensor gelu_backward_fused(const Tensor& x, const Tensor& grad_out) {
  panic_if(x.shape() != grad_out.shape(), "Shapes are not broadcastable");
  Tensor out = Tensor::empty(x.shape(), x.device());
  if (x.shape().numel() == 0) return out;
  const Tensor xc = x.contiguous(), gc = grad_out.contiguous();
  check(vh_gelu_grad_mul(xc.data(), gc.data(), out.data(), x.shape().numel(), nullptr));
  return out;
}

}  // namespace vearo_hip
