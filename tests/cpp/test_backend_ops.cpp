// test_backend_ops.cpp -- the HIP BackendOps mirror exercised the way the
// reference's own tests exercise its CUDA backend
// (crates/vearo-backend-cuda/src/lib.rs:1638-1826): CPU <-> device parity on
// small known inputs, every hot op on a non-contiguous input against the same
// op on `.contiguous()`, panics with the CPU backend's messages, empty tensors,
// the autograd arms, and a memory-regression loop (crates/vearo/tests/memory_regression.rs).
// The CPU oracle (oracle/vearo_cpu_ref.c) is the checker. Needs a gfx950 GPU.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/vearo_hip.h"
#include "vearo_backend.h"
#include "vearo_cpu_ref.h"

using namespace vearo_hip;

static int g_fail = 0, g_pass = 0;
static std::string g_where;

#define CHECK(cond, msg)                                                                         \
  do {                                                                                           \
    if (!(cond)) throw std::runtime_error(std::string("check failed: ") + (msg) + " [" #cond "]"); \
  } while (0)

static void run(const char* name, const std::function<void()>& f) {
  std::printf("[ run ] %s\n", name);
  std::fflush(stdout);
  try {
    f();
    ++g_pass;
    std::printf("[  ok ] %s\n", name);
  } catch (const std::exception& e) {
    ++g_fail;
    std::printf("[FAIL] %s: %s\n", name, e.what());
  }
  std::fflush(stdout);
}

static vo_layout contig(const std::vector<int64_t>& dims) {
  vo_layout l;
  vo_contiguous_layout(&l, (int)dims.size(), dims.data());
  return l;
}

// |gpu - cpu| <= 1e-5 + 1e-4 |cpu| elementwise.
static void expect_close(const std::vector<float>& gpu, const std::vector<float>& cpu, const char* what,
                         double atol = 1e-5, double rtol = 1e-4) {
  CHECK(gpu.size() == cpu.size(), std::string(what) + ": size mismatch");
  for (size_t i = 0; i < gpu.size(); ++i) {
    const double d = std::fabs((double)gpu[i] - (double)cpu[i]);
    if (!(d <= atol + rtol * std::fabs((double)cpu[i])) && !(gpu[i] == cpu[i])) {
      char buf[256];
      std::snprintf(buf, sizeof buf, "%s: element %zu gpu=%.9g cpu=%.9g", what, i, gpu[i], cpu[i]);
      throw std::runtime_error(buf);
    }
  }
}

static double maxdiff(const std::vector<float>& a, const std::vector<float>& b) {
  double m = 0;
  for (size_t i = 0; i < a.size(); ++i) m = std::max(m, (double)std::fabs(a[i] - b[i]));
  return m;
}

template <typename F>
static void expect_panic(F&& f, const std::string& substr) {
  try {
    f();
  } catch (const Panic& p) {
    CHECK(std::string(p.what()).find(substr) != std::string::npos,
          "panic text '" + std::string(p.what()) + "' lacks '" + substr + "'");
    return;
  }
  throw std::runtime_error("expected a panic containing '" + substr + "'");
}

static std::vector<float> randn(size_t n, unsigned seed, float scale = 1.0f) {
  std::vector<float> v(n);
  unsigned long long s = 0x9E3779B97F4A7C15ull * (seed + 1);
  for (size_t i = 0; i < n; ++i) {
    // SplitMix64 -> two uniforms -> Box-Muller.
    auto next = [&]() {
      unsigned long long z = (s += 0x9E3779B97F4A7C15ull);
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      return ((z ^ (z >> 31)) >> 11) * (1.0 / 9007199254740992.0);
    };
    const double u1 = next() + 1e-300, u2 = next();
    v[i] = (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2)) * scale;
  }
  return v;
}

static void vh_ok(int rc) {
  if (rc != VH_OK) throw std::runtime_error(std::string("vh call failed: ") + vh_last_error());
}

static std::vector<unsigned char> file_bytes(const std::string& path) {
  std::vector<unsigned char> out;
  if (std::FILE* f = std::fopen(path.c_str(), "rb")) {
    unsigned char buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.insert(out.end(), buf, buf + n);
    std::fclose(f);
  }
  return out;
}

// The device-written file is byte for byte the oracle's save of the same values.
static void check_file_is_oracle_save(const std::string& path, const std::vector<std::vector<float>>& data,
                                      const std::vector<std::vector<int64_t>>& dims) {
  std::vector<const float*> ptrs;
  std::vector<vo_layout> lays;
  for (size_t i = 0; i < data.size(); ++i) {
    ptrs.push_back(data[i].data());
    lays.push_back(contig(dims[i]));
  }
  const std::string opath = path + ".oracle";
  char err[256];
  CHECK(vo_checkpoint_save(opath.c_str(), (int)data.size(), ptrs.data(), lays.data(), err, sizeof err) == VO_OK,
        "oracle save");
  const std::vector<unsigned char> a = file_bytes(path), b = file_bytes(opath);
  std::remove(opath.c_str());
  CHECK(!a.empty() && a == b, "device checkpoint file equals the oracle's");
}

int main() {
  init(0);

  run("dispatch_registry", [] {
    CHECK(get_backend_ops(Device::hip()) != nullptr, "HIP backend registered");
    CHECK(get_backend_ops(Device{Device::Cpu, 0}) == nullptr, "no CPU backend in this process");
    CHECK(Device::hip().backend_idx() == 2, "HIP uses the reserved backend slot 2");
    init(0);  // idempotent (first registration wins, tensor.rs:1186-1190)
  });

  // crates/vearo-backend-cuda/src/lib.rs:1643-1673 (elementwise add, exact).
  run("test_hip_parity", [] {
    Tensor a = Tensor::from_f32({1, 2, 3, 4}, Shape{2, 2});
    Tensor b = Tensor::from_f32({5, 6, 7, 8}, Shape{2, 2});
    const std::vector<float> c = a.add(b).to_vec_f32();
    CHECK((c == std::vector<float>{6, 8, 10, 12}), "add");
    const std::vector<float> d = a.div(b).to_vec_f32();
    CHECK(d[0] == 1.0f / 5.0f && d[3] == 4.0f / 8.0f, "div");
  });

  // crates/vearo-backend-cuda/src/lib.rs:1715-1826: every op on a non-contiguous input
  // against the same op on .contiguous() (tol 1e-3), and against the CPU oracle.
  run("test_hip_noncontiguous_parity", [] {
    std::vector<std::string> fails;
    auto check = [&](const char* name, const Tensor& nc, const Tensor& c) {
      const auto a = nc.to_vec_f32(), b = c.to_vec_f32();
      bool bad = false;
      for (float v : a) bad |= !std::isfinite(v);
      const double m = a.size() == b.size() ? maxdiff(a, b) : 1e30;
      if (bad || m > 1e-3) fails.push_back(std::string(name) + " maxdiff=" + std::to_string(m));
    };
    Tensor a = Tensor::from_f32({1, 2, 3, 4, 5, 6, 7, 8, 9}, Shape{3, 3});
    Tensor b = Tensor::from_f32({9, 8, 7, 6, 5, 4, 3, 2, 1}, Shape{3, 3});
    Tensor bt = b.transpose(0, 1);
    check("add(rhs_nc)", a.add(bt), a.add(bt.contiguous()));
    check("sub(rhs_nc)", a.sub(bt), a.sub(bt.contiguous()));
    check("mul(rhs_nc)", a.mul(bt), a.mul(bt.contiguous()));
    check("div(rhs_nc)", a.div(bt), a.div(bt.contiguous()));
    Tensor at = a.transpose(0, 1);
    check("add(lhs_nc)", at.add(b), at.contiguous().add(b));

    Tensor x = Tensor::from_f32({-2, -1, 0.5, 1, 2, 3, -0.5, 4, -3, 0, 1.5, -1.5}, Shape{3, 4});
    Tensor xt = x.transpose(0, 1);
    check("gelu(nc)", xt.gelu(), xt.contiguous().gelu());
    check("sum(nc,d0)", xt.sum(0, false), xt.contiguous().sum(0, false));
    check("sum(nc,d1)", xt.sum(1, true), xt.contiguous().sum(1, true));
    check("mean(nc,d0)", xt.mean(0, false), xt.contiguous().mean(0, false));
    check("softmax(nc,d0)", xt.softmax(0), xt.contiguous().softmax(0));
    check("softmax(nc,d1)", xt.softmax(1), xt.contiguous().softmax(1));

    std::vector<float> lnv(24);
    for (int i = 0; i < 24; ++i) lnv[i] = i * 0.1f;
    Tensor ln = Tensor::from_f32(lnv, Shape{2, 3, 4});
    Tensor lnp = ln.permute({1, 0, 2});
    Tensor w = Tensor::from_f32({1, 0.5, 2, 1.5}, Shape{4});
    Tensor bb = Tensor::from_f32({0.1f, -0.1f, 0.2f, 0}, Shape{4});
    check("layernorm(nc)", lnp.layernorm(w, bb, 1e-5f), lnp.contiguous().layernorm(w, bb, 1e-5f));

    Tensor idx = Tensor::from_f32({0, 2, 1, 1, 0, 2}, Shape{2, 3});
    Tensor idxt = idx.transpose(0, 1);
    Tensor emb_w = Tensor::from_f32({10, 11, 20, 21, 30, 31}, Shape{3, 2});
    check("embedding(nc)", idxt.embedding(emb_w), idxt.contiguous().embedding(emb_w));

    Tensor logits_base = Tensor::from_f32({1, 4, 2, 5, 3, 6}, Shape{3, 2});
    Tensor logits_nc = logits_base.transpose(0, 1);
    Tensor tgt = Tensor::from_f32({0, 2}, Shape{2});
    check("cross_entropy(nc)", logits_nc.cross_entropy(tgt), logits_nc.contiguous().cross_entropy(tgt));
    if (!fails.empty()) {
      std::string all;
      for (auto& f : fails) all += f + "; ";
      throw std::runtime_error("ops that mishandle non-contiguous inputs: " + all);
    }

    // The same strided inputs through the CPU oracle.
    std::vector<float> host = {-2, -1, 0.5, 1, 2, 3, -0.5, 4, -3, 0, 1.5, -1.5};
    vo_layout tl;
    tl.rank = 2;
    tl.dims[0] = 4; tl.dims[1] = 3; tl.strides[0] = 1; tl.strides[1] = 4;
    std::vector<float> ref(12);
    vo_gelu(host.data(), &tl, ref.data());
    expect_close(xt.gelu().to_vec_f32(), ref, "gelu(nc) vs oracle");
    char err[256];
    CHECK(vo_softmax(host.data(), &tl, 0, ref.data(), err, sizeof err) == 0, "oracle softmax");
    expect_close(xt.softmax(0).to_vec_f32(), ref, "softmax(nc,d0) vs oracle");
    vo_layout lp;
    lp.rank = 3;
    lp.dims[0] = 3; lp.dims[1] = 2; lp.dims[2] = 4;
    lp.strides[0] = 4; lp.strides[1] = 12; lp.strides[2] = 1;
    std::vector<float> lref(24), wv = {1, 0.5, 2, 1.5}, bv = {0.1f, -0.1f, 0.2f, 0};
    vo_layout l4 = contig({4});
    CHECK(vo_layernorm(lnv.data(), &lp, wv.data(), &l4, bv.data(), &l4, 1e-5f, lref.data(), err, sizeof err) == 0,
          "oracle layernorm");
    expect_close(lnp.layernorm(w, bb, 1e-5f).to_vec_f32(), lref, "layernorm(nc) vs oracle");
  });

  run("hot_ops_vs_oracle_gpt2_rows", [] {
    const int rows = 512, C = 768;
    auto xv = randn((size_t)rows * C, 1), dyv = randn((size_t)rows * C, 2);
    auto wv = randn(C, 3, 0.02f), bv = randn(C, 4, 0.02f);
    for (auto& v : wv) v += 1.0f;
    Tensor x = Tensor::from_f32(xv, Shape{rows, C}), dy = Tensor::from_f32(dyv, Shape{rows, C});
    Tensor w = Tensor::from_f32(wv, Shape{C}), b = Tensor::from_f32(bv, Shape{C});
    auto [gx, gw, gb] = x.layernorm_backward(w, b, dy, 1e-5f);
    vo_layout xl = contig({rows, C}), cl = contig({C});
    std::vector<float> y(xv.size()), dx(xv.size()), dw(C), db(C);
    char err[256];
    CHECK(vo_layernorm(xv.data(), &xl, wv.data(), &cl, bv.data(), &cl, 1e-5f, y.data(), err, sizeof err) == 0, "ln");
    CHECK(vo_layernorm_backward(xv.data(), &xl, wv.data(), &cl, &cl, dyv.data(), &xl, 1e-5f, dx.data(), dw.data(),
                                db.data(), err, sizeof err) == 0, "ln bwd");
    expect_close(x.layernorm(w, b, 1e-5f).to_vec_f32(), y, "layernorm");
    expect_close(gx.to_vec_f32(), dx, "layernorm dx");
    expect_close(gw.to_vec_f32(), dw, "layernorm dgamma", 1e-4, 1e-4);
    expect_close(gb.to_vec_f32(), db, "layernorm dbeta", 1e-4, 1e-4);
    // Softmax arm: the 5-op composite and the fused kernel agree with the oracle.
    std::vector<float> sdx(xv.size());
    CHECK(vo_softmax_backward_composite(xv.data(), dyv.data(), &xl, 1, sdx.data(), err, sizeof err) == 0, "sm");
    expect_close(softmax_backward_arm(x, dy, 1).to_vec_f32(), sdx, "softmax arm (composite)");
    expect_close(softmax_backward_fused(x, dy).to_vec_f32(), sdx, "softmax arm (fused)");
    // Gelu arm.
    std::vector<float> mask(xv.size()), gref(xv.size());
    vo_gelu_grad_mask(xv.data(), (int64_t)xv.size(), mask.data());
    for (size_t i = 0; i < xv.size(); ++i) gref[i] = dyv[i] * mask[i];
    expect_close(gelu_backward_fused(x, dy).to_vec_f32(), gref, "gelu arm (fused)");
  });

  run("embedding_and_cross_entropy_vs_oracle", [] {
    const int V = 1000, D = 64, n = 300;
    std::vector<float> ids(n);
    for (int i = 0; i < n; ++i) ids[i] = (float)((i * 7919) % V);
    for (int i = 0; i < n; i += 5) ids[i] = 3.0f;  // a heavy token
    auto wv = randn((size_t)V * D, 5), dyv = randn((size_t)n * D, 6);
    Tensor I = Tensor::from_f32(ids, Shape{n}), W = Tensor::from_f32(wv, Shape{V, D});
    Tensor DY = Tensor::from_f32(dyv, Shape{n, D});
    vo_layout il = contig({n}), wl = contig({V, D}), gl = contig({n, D});
    std::vector<float> out((size_t)n * D), dw((size_t)V * D);
    char err[256];
    CHECK(vo_embedding(ids.data(), &il, wv.data(), &wl, out.data(), err, sizeof err) == 0, "emb");
    CHECK(vo_embedding_backward(ids.data(), &il, &wl, dyv.data(), &gl, dw.data(), err, sizeof err) == 0, "emb bwd");
    CHECK(I.embedding(W).to_vec_f32() == out, "embedding forward is bit-exact");
    // Rows of tokens with <= 16 hits are summed in the CPU's order (bit-exact);
    // the heavy token 3 (60 hits) is summed in position chunks (tolerance).
    const std::vector<float> gdw = I.embedding_backward(W, DY).to_vec_f32();
    std::vector<int> hits(V, 0);
    for (float f : ids) hits[(int)std::lround(f)]++;
    for (int v = 0; v < V; ++v) {
      const std::vector<float> g(gdw.begin() + v * D, gdw.begin() + (v + 1) * D);
      const std::vector<float> c(dw.begin() + v * D, dw.begin() + (v + 1) * D);
      if (hits[v] <= 16) CHECK(g == c, "light embedding-gradient row is bit-exact");
      else expect_close(g, c, "heavy embedding-gradient row");
    }
    CHECK(hits[3] > 16, "the test covers a heavy row");

    const int B = 33, Vc = 517;
    auto lv = randn((size_t)B * Vc, 7, 2.0f);
    std::vector<float> tg(B);
    for (int i = 0; i < B; ++i) tg[i] = (float)((i * 31) % Vc);
    Tensor L = Tensor::from_f32(lv, Shape{B, Vc}), T = Tensor::from_f32(tg, Shape{B});
    Tensor go = Tensor::from_f32({0.7f}, Shape{1});
    vo_layout ll = contig({B, Vc}), tl = contig({B});
    float loss;
    std::vector<float> dl(lv.size());
    CHECK(vo_cross_entropy(lv.data(), &ll, tg.data(), &tl, &loss, err, sizeof err) == 0, "ce");
    float gov = 0.7f;
    CHECK(vo_cross_entropy_backward(lv.data(), &ll, tg.data(), &tl, &gov, 1, dl.data(), err, sizeof err) == 0,
          "ce bwd");
    Tensor lt = L.cross_entropy(T);
    CHECK(lt.shape() == Shape{1}, "loss is a [1] tensor as on the CPU backend (cpu lib.rs:1050)");
    expect_close(lt.to_vec_f32(), {loss}, "cross_entropy");
    expect_close(L.cross_entropy_backward(T, go).to_vec_f32(), dl, "cross_entropy_backward", 1e-9, 1e-4);
  });

  // crates/vearo-backend-cpu/src/lib.rs:2866-2899 and the shape asserts.
  run("panics_match_cpu_backend", [] {
    Tensor W = Tensor::zeros(Shape{2, 3});
    expect_panic([&] { Tensor::from_f32({-1, 0}, Shape{2}).embedding(W).to_vec_f32(); },
                 "Token ID cannot be negative: -1");
    expect_panic([&] { Tensor::from_f32({2, 0}, Shape{2}).embedding(W).to_vec_f32(); },
                 "Token ID 2 out of vocabulary bound 2");
    Tensor logits = Tensor::zeros(Shape{2, 3});
    expect_panic([&] { logits.cross_entropy(Tensor::from_f32({-1, 0}, Shape{2})).to_vec_f32(); },
                 "Target class cannot be negative: -1");
    expect_panic([&] { logits.cross_entropy(Tensor::from_f32({3, 0}, Shape{2})).to_vec_f32(); },
                 "Target class 3 out of vocab bounds 3");
    expect_panic([&] { logits.cross_entropy_backward(Tensor::from_f32({0, 1}, Shape{2}), Tensor::zeros(Shape{2})); },
                 "grad_out must be a scalar");
    expect_panic([&] { logits.softmax(2); }, "Softmax dim out of range");
    expect_panic([&] { logits.sum(2, false); }, "Reduction dim out of range");
    expect_panic([&] { logits.add(Tensor::zeros(Shape{4})); }, "Shapes are not broadcastable");
    expect_panic([&] { logits.layernorm(Tensor::zeros(Shape{4}), Tensor::zeros(Shape{3}), 1e-5f); },
                 "Weight dimension must match norm_dim");
    expect_panic([&] { Tensor::from_f32({1}, Shape{1}).embedding_backward(W, Tensor::zeros(Shape{1, 2})); },
                 "grad_out shape must be x.shape() + [embedding_dim]");
    expect_panic([&] { get_backend_ops(Device::hip())->relu(logits); }, "relu is not part of this backend");
    expect_panic([&] { logits.matmul(logits); }, "Incompatible dimensions for matmul");
    expect_panic([&] { Tensor::zeros(Shape{3}).matmul(logits); }, "Matmul requires rank >= 2");
    expect_panic([&] { Tensor::zeros(Shape{2, 2, 3}).matmul(Tensor::zeros(Shape{3, 3, 2})); },
                 "Batch shapes are not broadcastable");
  });

  // crates/vearo-backend-cuda/src/lib.rs:1676-1699: matmul with a transposed,
  // non-contiguous rhs -- exactly what backward feeds it -- equals the CPU.
  run("test_hip_matmul_transposed", [] {
    Tensor a = Tensor::from_f32({1, 2, 3, 4, 5, 6}, Shape{2, 3});
    Tensor b = Tensor::from_f32({7, 8, 9, 10, 11, 12}, Shape{2, 3});
    const std::vector<float> c = a.matmul(b.transpose(0, 1)).to_vec_f32();
    const std::vector<float> bt = b.transpose(0, 1).to_vec_f32();
    std::vector<float> ref(4);
    char err[256];
    vo_layout al = contig({2, 3}), bl = contig({3, 2});
    CHECK(vo_matmul(std::vector<float>{1, 2, 3, 4, 5, 6}.data(), &al, bt.data(), &bl, ref.data(), err, sizeof err) == 0,
          "oracle matmul");
    CHECK(c == ref, "transposed rhs matches the CPU exactly");
    CHECK((c == std::vector<float>{50, 68, 122, 167}), "known values");
  });

  // Linear::forward at GPT-2 width: x [256, 768] @ W^T with W [512, 768] ~ N(0, 0.02).
  run("matmul_linear_vs_oracle", [] {
    const auto xv = randn(256 * 768, 21), wv = randn(512 * 768, 22, 0.02f);
    Tensor X = Tensor::from_f32(xv, Shape{256, 768}), W = Tensor::from_f32(wv, Shape{512, 768});
    const std::vector<float> y = X.matmul(W.transpose(0, 1)).to_vec_f32();
    std::vector<float> wt(768 * 512), ref(256 * 512);
    for (int o = 0; o < 512; ++o)
      for (int i = 0; i < 768; ++i) wt[(size_t)i * 512 + o] = wv[(size_t)o * 768 + i];
    char err[256];
    vo_layout xl = contig({256, 768}), tl = contig({768, 512});
    CHECK(vo_matmul(xv.data(), &xl, wt.data(), &tl, ref.data(), err, sizeof err) == 0, "oracle matmul");
    expect_close(y, ref, "linear");
  });

  // crates/vearo/tests/fused_attention_parity.rs: the fused op against the
  // unfused chain of backend ops, same inputs and bounds; and its backward
  // against the CPU fused backward.
  run("fused_attention_matches_unfused_reference", [] {
    const int B = 2, H = 2, S = 4, DK = 8, n = B * H * S * DK;
    auto fill = [&](float phase) {
      std::vector<float> v(n);
      for (int i = 0; i < n; ++i) {
        const float x = (float)i;
        v[i] = std::sin(x * 0.37f + phase) * 0.5f + std::cos(x * 0.11f + phase) * 0.25f;
      }
      return v;
    };
    const auto qv = fill(0.0f), kv = fill(1.3f), vv = fill(2.7f);
    std::vector<float> mv(S * S, 0.0f), cv(n);
    for (int r = 0; r < S; ++r)
      for (int c = 0; c < S; ++c)
        if (c > r) mv[r * S + c] = -1e9f;
    for (int i = 0; i < n; ++i) cv[i] = std::sin((float)i * 0.19f) + 1.5f;
    const Shape sh{B, H, S, DK};
    Tensor q = Tensor::from_f32(qv, sh), k = Tensor::from_f32(kv, sh), v = Tensor::from_f32(vv, sh);
    Tensor mask = Tensor::from_f32(mv, Shape{S, S});
    Tensor scale = Tensor::from_f32({1.0f / std::sqrt((float)DK)}, Shape{1});
    const auto out_ref = q.matmul(k.transpose(2, 3)).mul(scale).add(mask).softmax(3).matmul(v).to_vec_f32();
    const auto out = q.fused_attention(k, v, &mask).to_vec_f32();
    double maxabs = 0;
    for (float x : out_ref) maxabs = std::max(maxabs, (double)std::fabs(x));
    CHECK(maxabs > 1e-4, "reference output is not degenerate");
    CHECK(maxdiff(out_ref, out) < 1e-5, "fused output within 1e-5 of the unfused chain");
    Tensor go = Tensor::from_f32(cv, sh);
    auto [dq, dk, dv] = q.fused_attention_backward(k, v, &mask, go);
    std::vector<float> rq(n), rk(n), rv(n);
    vo_layout ml = contig({S, S});
    vo_fused_attention_backward(qv.data(), kv.data(), vv.data(), B, H, S, DK, mv.data(), &ml, cv.data(), rq.data(),
                                rk.data(), rv.data());
    CHECK(maxdiff(dq.to_vec_f32(), rq) < 1e-4, "dq");
    CHECK(maxdiff(dk.to_vec_f32(), rk) < 1e-4, "dk");
    CHECK(maxdiff(dv.to_vec_f32(), rv) < 1e-4, "dv");
  });

  // The slot skips the blocks SimpleGPT's -1e9 triangle (nn:763-771) masks
  // only when the device-side probe (VH_ATTN_CAUSAL_AUTO) proves every masked
  // exp() is exactly 0: out, dq, dk and dv are the dense masked form's bits
  // whichever form runs.
  run("fused_attention_causal_mask_same_bits", [] {
    const int B = 2, H = 3, S = 200, DK = 32, n = B * H * S * DK;
    const auto qv = randn(n, 71), kv = randn(n, 72), vv = randn(n, 73), gv = randn(n, 74);
    const Shape sh{B, H, S, DK};
    auto dense = [&](const std::vector<float>& mv, const std::vector<float>& qx) {
      Tensor q = Tensor::from_f32(qx, sh), k = Tensor::from_f32(kv, sh), v = Tensor::from_f32(vv, sh);
      Tensor m = Tensor::from_f32(mv, Shape{S, S}), g = Tensor::from_f32(gv, sh);
      Tensor o = Tensor::zeros(sh), dq = Tensor::zeros(sh), dk = Tensor::zeros(sh), dv = Tensor::zeros(sh);
      vh_layout l{}, ml{};
      l.rank = 4;
      const int64_t d[4] = {B, H, S, DK}, st[4] = {(int64_t)H * S * DK, (int64_t)S * DK, DK, 1};
      for (int i = 0; i < 4; ++i) { l.dims[i] = d[i]; l.strides[i] = st[i]; }
      ml.rank = 2;
      ml.dims[0] = ml.dims[1] = S;
      ml.strides[0] = S;
      ml.strides[1] = 1;
      vh_ok(vh_fused_attention_fwd(q.data(), &l, k.data(), &l, v.data(), &l, m.data(), &ml, 0, o.data(), &l,
                                   nullptr, 0, nullptr));
      vh_ok(vh_fused_attention_bwd(q.data(), &l, k.data(), &l, v.data(), &l, m.data(), &ml, 0, g.data(), &l,
                                   dq.data(), &l, dk.data(), &l, dv.data(), &l, nullptr, 0, nullptr));
      return std::vector<std::vector<float>>{o.to_vec_f32(), dq.to_vec_f32(), dk.to_vec_f32(), dv.to_vec_f32()};
    };
    auto slot = [&](const std::vector<float>& mv, const std::vector<float>& qx) {
      Tensor q = Tensor::from_f32(qx, sh), k = Tensor::from_f32(kv, sh), v = Tensor::from_f32(vv, sh);
      Tensor m = Tensor::from_f32(mv, Shape{S, S}), g = Tensor::from_f32(gv, sh);
      const auto o = q.fused_attention(k, v, &m).to_vec_f32();
      auto [dq, dk, dv] = q.fused_attention_backward(k, v, &m, g);
      return std::vector<std::vector<float>>{o, dq.to_vec_f32(), dk.to_vec_f32(), dv.to_vec_f32()};
    };
    auto same_bits = [](const std::vector<float>& a, const std::vector<float>& b) {
      return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
    };
    std::vector<float> tri(S * S, 0.0f);
    for (int r = 0; r < S; ++r)
      for (int c = r + 1; c < S; ++c) tri[r * S + c] = -1e9f;
    std::vector<float> shallow = tri;  // masked at -50: exponents that need not underflow
    for (float& x : shallow)
      if (x != 0.0f) x = -50.0f;
    std::vector<float> qbig = qv;  // scores near 1e9 defeat the proof
    qbig[5] = 4e9f;
    const char* names[4] = {"out", "dq", "dk", "dv"};
    for (int c = 0; c < 3; ++c) {
      const auto& mv = c == 1 ? shallow : tri;
      const auto& qx = c == 2 ? qbig : qv;
      const auto a = dense(mv, qx), b = slot(mv, qx);
      for (int i = 0; i < 4; ++i)
        CHECK(same_bits(a[i], b[i]), std::string("case ") + std::to_string(c) + " " + names[i] + " bits");
    }
  });

  run("empty_tensors", [] {
    // crates/vearo-backend-cpu/src/lib.rs:2832-2864.
    Tensor x = Tensor::zeros(Shape{2, 0, 4});
    Tensor out = x.layernorm(Tensor::from_f32({1, 1, 1, 1}, Shape{4}), Tensor::zeros(Shape{4}), 1e-5f);
    CHECK(out.shape() == (Shape{2, 0, 4}), "layernorm of an empty input keeps its shape");
    Tensor z = Tensor::zeros(Shape{0, 6}).add(Tensor::zeros(Shape{0, 6}));
    CHECK(z.shape() == (Shape{0, 6}) && z.to_vec_f32().empty(), "empty add");
    auto [gx, gw, gb] = x.layernorm_backward(Tensor::from_f32({1, 1, 1, 1}, Shape{4}), Tensor::zeros(Shape{4}), x, 1e-5f);
    CHECK(gw.to_vec_f32() == std::vector<float>(4, 0.0f), "empty layernorm backward gives zero dgamma");
  });

  run("checkpoint_save_load", [] {
    // crates/vearo/src/checkpoint.rs:97-120 on device tensors.
    Tensor t1 = Tensor::from_f32({1.0f, 2.0f, 3.0f, 4.0f}, Shape{2, 2});
    Tensor t2 = Tensor::from_f32({-0.5f, 0.5f}, Shape{2});
    const std::vector<Tensor> params{t1, t2};
    const std::string path = "/tmp/vearo_hip_model_checkpoint.ve";
    save_checkpoint(params, path);
    check_file_is_oracle_save(path, {{1.0f, 2.0f, 3.0f, 4.0f}, {-0.5f, 0.5f}}, {{2, 2}, {2}});
    vh_ok(vh_h2d(t1.data(), std::vector<float>(4, 0.0f).data(), 16));
    vh_ok(vh_h2d(t2.data(), std::vector<float>(2, 0.0f).data(), 8));
    load_checkpoint(params, path);
    CHECK(t1.to_vec_f32() == (std::vector<float>{1.0f, 2.0f, 3.0f, 4.0f}), "t1 restored");
    CHECK(t2.to_vec_f32() == (std::vector<float>{-0.5f, 0.5f}), "t2 restored");
    // The reference's asserts (checkpoint.rs:50-54, 64-68; tensor.rs:817-820).
    expect_panic([&] { load_checkpoint({t1}, path); },
                 "Checkpoint tensor count does not match model parameter count");
    expect_panic([&] { load_checkpoint({t2, t1}, path); }, "Checkpoint shape does not match parameter shape");
    expect_panic([&] { load_checkpoint({t1.transpose(0, 1), t2}, path); },
                 "copy_from_slice requires contiguous tensor");
    Tensor sq = Tensor::from_f32({1.0f, 2.0f, 3.0f, 4.0f}, Shape{2, 2});
    expect_panic([&] { save_checkpoint({sq.transpose(0, 1)}, path + ".t"); }, "to_vec_f32 requires contiguous tensor");
    bool io = false;
    try {
      load_checkpoint(params, "/tmp/vearo_hip_no_such_dir/none.ve");
    } catch (const IoError&) {
      io = true;
    }
    CHECK(io, "a missing file is an io error, not a panic");
    std::remove(path.c_str());
  });

  run("memory_regression", [] {
    // crates/vearo/tests/memory_regression.rs:103: live device memory must not grow.
    vh_mem_stats s0, s1;
    auto step = [] {
      Tensor x = Tensor::from_f32(randn(64 * 96, 9), Shape{64, 96});
      Tensor w = Tensor::from_f32(std::vector<float>(96, 1.0f), Shape{96});
      Tensor b = Tensor::zeros(Shape{96});
      Tensor y = x.layernorm(w, b, 1e-5f).gelu().softmax(1);
      auto [gx, gw, gb] = x.layernorm_backward(w, b, y, 1e-5f);
      (void)gx.sum(0, false).to_vec_f32();
    };
    step();
    synchronize();
    vh_mem_stats_get(&s0);
    for (int i = 0; i < 25; ++i) step();
    synchronize();
    vh_mem_stats_get(&s1);
    CHECK(s1.live_bytes == s0.live_bytes, "live bytes stable over 25 steps");
    CHECK(s1.hip_bytes == s0.hip_bytes, "no new hipMalloc after the first step (arena reuse)");
  });

  std::printf("%d passed, %d failed\n", g_pass, g_fail);
  return g_fail == 0 ? 0 : 1;
}
