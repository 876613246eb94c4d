// blaslt.cpp -- the A/B engine: plain f32 products through hipBLASLt.
//
// The default engine never comes here: every product runs on this library's
// own kernels (kernels/gemm_big.h, kernels/gemm.h). A caller that sets
// vh_gemm_desc.engine = VH_GEMM_ENGINE_LIBRARY (or vb_gpt_set_gemm_engine)
// hands the products the library takes -- no batch, no causal range, an
// addend E that is absent or a bias over the output columns, with or without
// accumulation into C -- to hipBLASLt instead, so its kernels can be timed
// beside the own ones on the same step: D = alpha A B (+ C) (+ bias), the
// bias through hipBLASLt's bias epilogue, compute type HIPBLAS_COMPUTE_32F
// (f32 products and sums). Anything it does not take runs on the own kernels.
//
// libhipblaslt.so.1 is not a link-time dependency: it is opened with dlopen
// on the first library-engine call, so a deployment that never asks for the
// A/B engine does not need it installed. Without it that call fails with
// VH_ERR_HIP and a message naming the library.
//
// hipBLASLt is column-major: the row-major C[M, N] = A[M, K] B[K, N] is issued
// as the column-major C^T[N, M] = B^T[N, K] A^T[K, M], each operand transposed
// or not by which of its dims has the unit stride. Descriptors and the
// heuristic's algorithm are cached per problem.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <dlfcn.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>

#include "../../include/vearo_hip.h"
#include "rt_internal.h"

namespace {

using vh_rt::fail;

constexpr size_t kWorkspace = size_t(64) << 20;  // bytes the algorithms may use

// The hipBLASLt entry points this file calls, resolved from the library at
// its first use (the header supplies only their types).
struct Api {
  void* so = nullptr;
  decltype(&hipblasLtCreate) Create = nullptr;
  decltype(&hipblasLtDestroy) Destroy = nullptr;
  decltype(&hipblasLtMatmulDescCreate) MatmulDescCreate = nullptr;
  decltype(&hipblasLtMatmulDescDestroy) MatmulDescDestroy = nullptr;
  decltype(&hipblasLtMatmulDescSetAttribute) MatmulDescSetAttribute = nullptr;
  decltype(&hipblasLtMatrixLayoutCreate) MatrixLayoutCreate = nullptr;
  decltype(&hipblasLtMatrixLayoutDestroy) MatrixLayoutDestroy = nullptr;
  decltype(&hipblasLtMatmulPreferenceCreate) MatmulPreferenceCreate = nullptr;
  decltype(&hipblasLtMatmulPreferenceDestroy) MatmulPreferenceDestroy = nullptr;
  decltype(&hipblasLtMatmulPreferenceSetAttribute) MatmulPreferenceSetAttribute = nullptr;
  decltype(&hipblasLtMatmulAlgoGetHeuristic) MatmulAlgoGetHeuristic = nullptr;
  decltype(&hipblasLtMatmul) Matmul = nullptr;
};

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t lx = nullptr, ly = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool usable = false;  // the heuristic returned an algorithm
};

// M, N, K, ldx, ldy, ldc, tx, ty, bias epilogue
using Key = std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, int>;

struct Lib {
  std::mutex mu;
  Api api;
  hipblasLtHandle_t handle = nullptr;
  // One workspace per stream: products on different streams may overlap, and
  // the work in one stream is ordered, so each stream reuses its own.
  std::map<hipStream_t, void*> ws;
  std::map<Key, Plan> plans;
} g_lib;

int status(hipblasStatus_t st, const char* what) {
  if (st == HIPBLAS_STATUS_SUCCESS) return VH_OK;
  return fail(VH_ERR_HIP, std::string("hipBLASLt ") + what + " failed: status " + std::to_string((int)st));
}

// Opens libhipblaslt.so.1 and resolves every entry point (once; the caller
// holds g_lib.mu). A missing library or symbol is an error, not a fallback:
// the caller asked for this engine by name.
int load_api() {
  Api& a = g_lib.api;
  if (a.so) return VH_OK;
  void* so = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
  if (!so) so = dlopen("libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
  if (!so) {
    const char* e = dlerror();
    return fail(VH_ERR_HIP, std::string("the hipBLASLt A/B engine needs libhipblaslt.so.1: ") + (e ? e : "not found"));
  }
  Api t;
  t.so = so;
  bool ok = true;
  auto sym = [&](auto& fp, const char* name) {
    fp = reinterpret_cast<std::remove_reference_t<decltype(fp)>>(dlsym(so, name));
    ok = ok && fp != nullptr;
  };
  sym(t.Create, "hipblasLtCreate");
  sym(t.Destroy, "hipblasLtDestroy");
  sym(t.MatmulDescCreate, "hipblasLtMatmulDescCreate");
  sym(t.MatmulDescDestroy, "hipblasLtMatmulDescDestroy");
  sym(t.MatmulDescSetAttribute, "hipblasLtMatmulDescSetAttribute");
  sym(t.MatrixLayoutCreate, "hipblasLtMatrixLayoutCreate");
  sym(t.MatrixLayoutDestroy, "hipblasLtMatrixLayoutDestroy");
  sym(t.MatmulPreferenceCreate, "hipblasLtMatmulPreferenceCreate");
  sym(t.MatmulPreferenceDestroy, "hipblasLtMatmulPreferenceDestroy");
  sym(t.MatmulPreferenceSetAttribute, "hipblasLtMatmulPreferenceSetAttribute");
  sym(t.MatmulAlgoGetHeuristic, "hipblasLtMatmulAlgoGetHeuristic");
  sym(t.Matmul, "hipblasLtMatmul");
  if (!ok) {
    dlclose(so);
    return fail(VH_ERR_HIP, "libhipblaslt.so.1 lacks an entry point the A/B engine calls");
  }
  a = t;
  return VH_OK;
}

#define LT(expr, what)                       \
  do {                                       \
    int rc_ = status((expr), what);          \
    if (rc_ != VH_OK) return rc_;            \
  } while (0)

void destroy(Plan& p) {
  if (p.op) g_lib.api.MatmulDescDestroy(p.op);
  if (p.lx) g_lib.api.MatrixLayoutDestroy(p.lx);
  if (p.ly) g_lib.api.MatrixLayoutDestroy(p.ly);
  if (p.lc) g_lib.api.MatrixLayoutDestroy(p.lc);
  p = Plan{};
}

// Descriptors for the problem and the heuristic's best algorithm within the
// workspace (usable = false if it has none). Nothing leaks on a failure.
int make_plan(const Key& k, Plan* out) {
  const auto [M, N, K, ldx, ldy, ldc, tx, ty, bias] = k;
  Plan p;
  // X = B^T: [N, K] as stored (tx = 0) or the transpose of a stored [K, N].
  // Y = A^T: [K, M] as stored (ty = 0) or the transpose of a stored [M, K].
  const hipblasOperation_t opx = tx ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t opy = ty ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  hipblasLtMatmulPreference_t pref = nullptr;
  auto build = [&]() -> int {
    LT(g_lib.api.MatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F), "MatmulDescCreate");
    LT(g_lib.api.MatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &opx, sizeof(opx)), "set TRANSA");
    LT(g_lib.api.MatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &opy, sizeof(opy)), "set TRANSB");
    if (bias) {
      // A bias of length N (D's rows in the column-major view) on every column.
      const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
      const int32_t bt = HIP_R_32F;
      LT(g_lib.api.MatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)), "set EPILOGUE");
      LT(g_lib.api.MatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)),
         "set BIAS_DATA_TYPE");
    }
    LT(g_lib.api.MatrixLayoutCreate(&p.lx, HIP_R_32F, tx ? K : N, tx ? N : K, ldx), "layout X");
    LT(g_lib.api.MatrixLayoutCreate(&p.ly, HIP_R_32F, ty ? M : K, ty ? K : M, ldy), "layout Y");
    LT(g_lib.api.MatrixLayoutCreate(&p.lc, HIP_R_32F, N, M, ldc), "layout C");
    LT(g_lib.api.MatmulPreferenceCreate(&pref), "PreferenceCreate");
    uint64_t wsb = kWorkspace;
    LT(g_lib.api.MatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb)),
       "set workspace");
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    const hipblasStatus_t st =
        g_lib.api.MatmulAlgoGetHeuristic(g_lib.handle, p.op, p.lx, p.ly, p.lc, p.lc, pref, 1, res, &found);
    if (st == HIPBLAS_STATUS_SUCCESS && found > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS &&
        res[0].workspaceSize <= kWorkspace) {
      p.algo = res[0].algo;
      p.usable = true;
    }
    return VH_OK;
  };
  const int rc = build();
  if (pref) g_lib.api.MatmulPreferenceDestroy(pref);
  if (rc != VH_OK) {
    destroy(p);
    return rc;
  }
  *out = p;
  return VH_OK;
}

}  // namespace

namespace vh_rt {

int blaslt_gemm(const vh_gemm_desc* d, bool akc, bool bkc, void* stream, bool* taken) {
  *taken = false;
  const int64_t M = d->M, N = d->N, K = d->K;
  // X = B^T [N, K]: a k-contiguous B is a stored [K, N] (column-major) to transpose.
  const int tx = bkc ? 1 : 0;
  const int64_t ldx = bkc ? (N == 1 ? K : d->b_sn) : (K == 1 ? N : d->b_sk);
  // Y = A^T [K, M]: a k-contiguous A is a stored [K, M] as is.
  const int ty = akc ? 0 : 1;
  const int64_t ldy = akc ? (M == 1 ? K : d->a_sm) : (K == 1 ? M : d->a_sk);
  const int64_t ldc = M == 1 ? N : d->c_sm;
  if (ldx < (tx ? K : N) || ldy < (ty ? M : K) || ldc < N) return VH_OK;  // not a layout it takes
  const hipStream_t s = stream_of(stream);
  std::lock_guard<std::mutex> lk(g_lib.mu);
  {
    const int rc = load_api();
    if (rc != VH_OK) return rc;
  }
  if (!g_lib.handle) LT(g_lib.api.Create(&g_lib.handle), "Create");
  void*& ws = g_lib.ws[s];
  if (!ws) {
    const hipError_t e = hipMalloc(&ws, kWorkspace);
    if (e != hipSuccess) {
      g_lib.ws.erase(s);
      return fail(VH_ERR_OOM, std::string("hipBLASLt workspace: ") + hipGetErrorString(e));
    }
  }
  const int bias = d->e ? 1 : 0;
  if (bias && !(d->e_sm == 0 && d->e_sn == 1)) return VH_OK;  // only a bias over the columns
  const Key key{M, N, K, ldx, ldy, ldc, tx, ty, bias};
  auto it = g_lib.plans.find(key);
  if (it == g_lib.plans.end()) {
    Plan p;
    const int rc = make_plan(key, &p);
    if (rc != VH_OK) return rc;
    it = g_lib.plans.emplace(key, p).first;
  }
  if (!it->second.usable) return VH_OK;  // no algorithm: the caller's kernel runs it
  const float alpha = d->alpha, beta = d->accumulate ? 1.0f : 0.0f;
  const Plan& p = it->second;
  if (bias) {
    const void* bp = d->e;
    LT(g_lib.api.MatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)),
       "set BIAS_POINTER");
  }
  LT(g_lib.api.Matmul(g_lib.handle, p.op, &alpha, d->b, p.lx, d->a, p.ly, &beta, d->c, p.lc, d->c, p.lc, &p.algo,
                     ws, kWorkspace, s),
     "Matmul");
  *taken = true;
  return VH_OK;
}

void blaslt_shutdown() {
  std::lock_guard<std::mutex> lk(g_lib.mu);
  if (!g_lib.api.so) return;  // the library was never opened: nothing of it to release
  for (auto& kv : g_lib.plans) destroy(kv.second);
  g_lib.plans.clear();
  for (auto& kv : g_lib.ws) (void)hipFree(kv.second);
  g_lib.ws.clear();
  if (g_lib.handle) g_lib.api.Destroy(g_lib.handle);
  g_lib.handle = nullptr;
}

}  // namespace vh_rt
