// Prefill GEMMs on hipBLASLt with a fixed algorithm per shape (host code only).
//
// The prefill's projections are plain bf16 GEMMs over all prompt tokens (M in the thousands):
// y[M,N] = x[M,K] . W[N,K]^T, fp32 accumulation, bf16 out -- the reference runs them through
// F.linear (engine.py:131-132 via _forward, engine.py:459-503), i.e. the BLAS library's heuristic
// choice. On MI355X hipBLASLt's first heuristic candidate is up to 25% slower than its best
// candidate for the Qwen3-4B shapes (measured at 16,223 tokens: down 788 -> 569 us, O 382 ->
// 247 us per layer). The caller names the algorithm: a hipBLASLt solution index (stable for one
// library build), chosen offline per (N, K, M range) by timing and kept in a table the host
// reads. The same solution on the same operands gives the same bits in every process; nothing
// here times, allocates device memory or synchronises.
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "api.h"

namespace dd {
namespace {

constexpr int MAX_DEV = 16;
constexpr int NCAND = 16;            // heuristic candidates listed for the tuning tool

std::mutex g_mu;
hipblasLtHandle_t g_handle[MAX_DEV] = {};

// RAII holders for a shape's descriptors (kept per shape: a prefill makes the same products
// for every layer, and creating them per call costs host time comparable to the GEMM)
struct Desc {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  ~Desc() {
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (c) hipblasLtMatrixLayoutDestroy(c);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (op) hipblasLtMatmulDescDestroy(op);
  }
};

// What a (device, M, N, K, workspace) runs: the descriptors and, per requested solution index,
// the algorithm resolved for this problem (the requested one when it supports the problem within
// the workspace, else the heuristic's first candidate).
struct Shape {
  Desc d;
  bool have_first = false;
  hipblasLtMatmulAlgo_t first;
  std::map<int, hipblasLtMatmulAlgo_t> algo;
};

int blas_err(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + (int)s; }

// Column-major view: Y^T[N,M] = W[N,K] (stored as col-major K x N, op T) . X^T (col-major K x M)
int make_desc(Desc& d, int M, int N, int K, size_t ws_bytes) {
  hipblasStatus_t s = hipblasLtMatmulDescCreate(&d.op, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (s != HIPBLAS_STATUS_SUCCESS) return blas_err(s);
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  s = hipblasLtMatmulDescSetAttribute(d.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulDescSetAttribute(d.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&d.a, HIP_R_16BF, K, N, K);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&d.b, HIP_R_16BF, K, M, K);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&d.c, HIP_R_16BF, N, M, N);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatmulPreferenceCreate(&d.pref);
  if (s == HIPBLAS_STATUS_SUCCESS) {
    const uint64_t wsb = ws_bytes;
    s = hipblasLtMatmulPreferenceSetAttribute(d.pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                              &wsb, sizeof(wsb));
  }
  return blas_err(s);
}

int run(hipblasLtHandle_t h, const Desc& d, const hipblasLtMatmulAlgo_t& algo, const void* x,
        const void* w, void* y, void* ws, size_t ws_bytes, hipStream_t stream) {
  const float alpha = 1.f, beta = 0.f;
  return blas_err(hipblasLtMatmul(h, d.op, &alpha, w, d.a, x, d.b, &beta, y, d.c, y, d.c, &algo,
                                  ws, ws_bytes, stream));
}

// The handle of the current device and the (bounded) per-shape record; g_mu held.
int shape_of(int M, int N, int K, size_t ws_bytes, hipblasLtHandle_t* h_out, Shape** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return (int)hipErrorInvalidValue;
  if (!g_handle[dev]) {
    const hipblasStatus_t s = hipblasLtCreate(&g_handle[dev]);
    if (s != HIPBLAS_STATUS_SUCCESS) return blas_err(s);
  }
  *h_out = g_handle[dev];
  static std::map<std::tuple<int, int, int, int, size_t>, Shape*> shapes;
  const auto key = std::make_tuple(dev, M, N, K, ws_bytes);
  auto it = shapes.find(key);
  if (it == shapes.end()) {
    if (shapes.size() >= 256) {              // bounded: drop them all (rebuilt on demand)
      for (auto& kv : shapes) delete kv.second;
      shapes.clear();
    }
    Shape* ns = new Shape;
    const int e = make_desc(ns->d, M, N, K, ws_bytes);
    if (e) {
      delete ns;
      return e;
    }
    it = shapes.emplace(key, ns).first;
  }
  *out = it->second;
  return 0;
}

// the heuristic's candidates for the shape (up to `max`, in its order)
int candidates(hipblasLtHandle_t h, const Desc& d, int max,
               std::vector<hipblasLtMatmulHeuristicResult_t>& cand) {
  cand.resize(max);
  int n = 0;
  const hipblasStatus_t s = hipblasLtMatmulAlgoGetHeuristic(h, d.op, d.a, d.b, d.c, d.c, d.pref,
                                                            max, cand.data(), &n);
  if (s != HIPBLAS_STATUS_SUCCESS) return blas_err(s);
  if (n < 1) return (int)hipErrorInvalidValue;
  cand.resize(n);
  return 0;
}

// The algorithm a (shape, solution) pair runs; g_mu held.
int resolve(hipblasLtHandle_t h, Shape& sh, int solution, size_t ws_bytes,
            const hipblasLtMatmulAlgo_t** out) {
  auto it = sh.algo.find(solution);
  if (it != sh.algo.end()) {
    *out = &it->second;
    return 0;
  }
  if (!sh.have_first) {
    std::vector<hipblasLtMatmulHeuristicResult_t> cand;
    const int e = candidates(h, sh.d, 1, cand);
    if (e) return e;
    sh.first = cand[0].algo;
    sh.have_first = true;
  }
  hipblasLtMatmulAlgo_t pick = sh.first;
  if (solution >= 0) {
    std::vector<int> idx{solution};
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    if (hipblaslt_ext::getAlgosFromIndex(h, idx, res) == HIPBLAS_STATUS_SUCCESS && !res.empty()) {
      const float alpha = 1.f, beta = 0.f;
      size_t need = 0;
      hipblasLtMatmulAlgo_t a = res[0].algo;
      if (hipblaslt_ext::matmulIsAlgoSupported(h, sh.d.op, &alpha, sh.d.a, sh.d.b, &beta, sh.d.c,
                                               sh.d.c, a, need) == HIPBLAS_STATUS_SUCCESS &&
          need <= ws_bytes)
        pick = a;
    }
  }
  if (sh.algo.size() >= 64) sh.algo.clear();
  *out = &sh.algo.emplace(solution, pick).first->second;
  return 0;
}

}  // namespace
}  // namespace dd

using namespace dd;

DD_API size_t dd_gemm_ws_bytes(void) { return (size_t)64 << 20; }

DD_API int dd_gemm_bf16(const void* x, const void* w, void* y, int M, int N, int K, void* ws,
                        size_t ws_bytes, int solution, hipStream_t stream) {
  DD_REQUIRE(x && w && y && M >= 1 && N >= 1 && K >= 1);
  DD_REQUIRE(ws_bytes == 0 || ws != nullptr);
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h = nullptr;
  Shape* sh = nullptr;
  int e = shape_of(M, N, K, ws_bytes, &h, &sh);
  if (e) return e;
  const hipblasLtMatmulAlgo_t* algo = nullptr;
  e = resolve(h, *sh, solution, ws_bytes, &algo);
  if (e) return e;
  return run(h, sh->d, *algo, x, w, y, ws, ws_bytes, stream);
}

DD_API int dd_gemm_bf16_supported(int M, int N, int K, size_t ws_bytes, int solution) {
  if (!(M >= 1 && N >= 1 && K >= 1 && solution >= 0)) return 0;
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h = nullptr;
  Shape* sh = nullptr;
  if (shape_of(M, N, K, ws_bytes, &h, &sh)) return 0;
  std::vector<int> idx{solution};
  std::vector<hipblasLtMatmulHeuristicResult_t> res;
  if (hipblaslt_ext::getAlgosFromIndex(h, idx, res) != HIPBLAS_STATUS_SUCCESS || res.empty()) return 0;
  const float alpha = 1.f, beta = 0.f;
  size_t need = 0;
  hipblasLtMatmulAlgo_t a = res[0].algo;
  return hipblaslt_ext::matmulIsAlgoSupported(h, sh->d.op, &alpha, sh->d.a, sh->d.b, &beta, sh->d.c,
                                              sh->d.c, a, need) == HIPBLAS_STATUS_SUCCESS &&
                 need <= ws_bytes
             ? 1
             : 0;
}

DD_API int dd_gemm_bf16_solutions(int M, int N, int K, size_t ws_bytes, int* out, int max) {
  if (!(M >= 1 && N >= 1 && K >= 1 && out && max >= 1)) return -1;
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h = nullptr;
  Shape* sh = nullptr;
  int e = shape_of(M, N, K, ws_bytes, &h, &sh);
  if (e) return -1;
  std::vector<hipblasLtMatmulHeuristicResult_t> cand;
  e = candidates(h, sh->d, max < NCAND ? max : NCAND, cand);
  if (e) return -1;
  int n = 0;
  for (auto& c : cand) {
    if (c.state != HIPBLAS_STATUS_SUCCESS || c.workspaceSize > ws_bytes) continue;
    out[n++] = hipblaslt_ext::getIndexFromAlgo(c.algo);
  }
  return n;
}
