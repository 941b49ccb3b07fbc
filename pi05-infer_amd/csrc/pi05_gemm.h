// hipBLASLt plans shared by the prefill and the vision tower (host code).
//
// C[M, N] (row-major) = A[M, K] (row-major) . W[N, K]^T (nn.Linear layout), fp32 accumulation.
// In hipBLASLt's column-major terms that is C^T (N x M) = W (stored K x N, transposed) . A^T
// (stored K x M).  Options: an fp32 bias per output column added before the one rounding
// (HIPBLASLT_EPILOGUE_BIAS; the pointer is set per call), fp32 operands, split-K batches.
#pragma once

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <string>
#include <vector>

namespace pi05 {

struct GemmPlan {
  int M = 0, N = 0, K = 0;
  bool bias = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
  std::vector<hipblasLtMatmulHeuristicResult_t> cands;  // heuristic candidates, timed by tune_plan
  float ms = 0.f;                                        // the chosen algorithm's time
};
constexpr int kGemmCandidates = 256;

inline bool lt_ok(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS; }

struct GemmOpts {
  int batch = 1;                // > 1: split-K over `batch` K-slices of width K of rows ld_k long
  int ld_k = 0;                 // row length of the A and W operands (0: K)
  hipDataType ab = HIP_R_16BF;  // operand type (HIP_R_32F for an fp32 GEMM)
  hipDataType c = HIP_R_16BF;   // output type (split-K partials: HIP_R_32F)
  bool bias = false;            // fp32 per-column bias before the rounding
};

inline bool make_plan(hipblasLtHandle_t h, int M, int N, int K, size_t ws_max, GemmPlan* p, std::string* err, GemmOpts o = GemmOpts{}) {
  const int ld_k = o.ld_k ? o.ld_k : K;
  p->M = M, p->N = N, p->K = K, p->bias = o.bias;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  const hipDataType ct = o.batch > 1 ? HIP_R_32F : o.c;
  if (!lt_ok(hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)) ||
      !lt_ok(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta))) ||
      !lt_ok(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb))) ||
      !lt_ok(hipblasLtMatrixLayoutCreate(&p->lw, o.ab, K, N, ld_k)) || !lt_ok(hipblasLtMatrixLayoutCreate(&p->la, o.ab, K, M, ld_k)) ||
      !lt_ok(hipblasLtMatrixLayoutCreate(&p->lc, ct, N, M, N))) {
    *err = "hipBLASLt descriptor creation failed";
    return false;
  }
  if (o.bias) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bt = HIP_R_32F;
    if (!lt_ok(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep))) ||
        !lt_ok(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)))) {
      *err = "hipBLASLt bias epilogue failed";
      return false;
    }
  }
  if (o.batch > 1) {
    const int32_t bc = o.batch;
    const int64_t sk = K, sc = (int64_t)N * M;
    for (hipblasLtMatrixLayout_t l : {p->lw, p->la, p->lc}) {
      const int64_t st = l == p->lc ? sc : sk;
      if (!lt_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc))) ||
          !lt_ok(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &st, sizeof(st)))) {
        *err = "hipBLASLt batch layout failed";
        return false;
      }
    }
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  if (!lt_ok(hipblasLtMatmulPreferenceCreate(&pref))) {
    *err = "hipBLASLt preference creation failed";
    return false;
  }
  uint64_t wsb = ws_max;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
  std::vector<hipblasLtMatmulHeuristicResult_t> res(kGemmCandidates);
  int n = 0;
  const hipblasStatus_t s = hipblasLtMatmulAlgoGetHeuristic(h, p->desc, p->lw, p->la, p->lc, p->lc, pref, kGemmCandidates, res.data(), &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  for (int i = 0; lt_ok(s) && i < n; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= ws_max) p->cands.push_back(res[i]);
  if (!p->cands.empty()) {
    p->algo = p->cands[0].algo;  // the heuristic's first choice until tune_plan has timed them all
    p->ws = p->cands[0].workspaceSize;
    return true;
  }
  *err = "hipBLASLt found no GEMM algorithm for M=" + std::to_string(M) + " N=" + std::to_string(N) + " K=" + std::to_string(K);
  return false;
}

// One GEMM with plan p (bias: device fp32 [N], only for plans made with a bias).
inline hipblasStatus_t run_plan(hipblasLtHandle_t h, const GemmPlan& p, const hipblasLtMatmulAlgo_t& algo, size_t ws_bytes, const void* W,
                                const void* A, void* C, const float* bias, void* ws, hipStream_t st) {
  if (p.bias) {
    const hipblasStatus_t s = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    if (!lt_ok(s)) return s;
  }
  const float alpha = 1.f, beta = 0.f;
  return hipblasLtMatmul(h, p.desc, &alpha, W, p.lw, A, p.la, &beta, C, p.lc, C, p.lc, &algo, ws, ws_bytes, st);
}

// Time every candidate algorithm on real buffers (3 runs after one warm-up; values do not affect
// the timing) and keep the fastest; candidates that fail to launch are skipped.
inline bool tune_plan(hipblasLtHandle_t h, GemmPlan* p, const void* W, const void* A, void* C, void* ws, hipStream_t st,
                      const float* bias = nullptr) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return false;
  if (hipEventCreate(&e1) != hipSuccess) {
    hipEventDestroy(e0);
    return false;
  }
  float best = 1e30f;
  for (const auto& c : p->cands) {
    bool ok = lt_ok(run_plan(h, *p, c.algo, c.workspaceSize, W, A, C, bias, ws, st));
    if (!ok) continue;
    hipEventRecord(e0, st);
    for (int r = 0; r < 3 && ok; ++r) ok = lt_ok(run_plan(h, *p, c.algo, c.workspaceSize, W, A, C, bias, ws, st));
    hipEventRecord(e1, st);
    if (hipEventSynchronize(e1) != hipSuccess) break;
    float ms = 0.f;
    if (!ok || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) continue;
    if (ms < best) {
      best = ms;
      p->algo = c.algo;
      p->ws = c.workspaceSize;
    }
  }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  p->ms = best / 3.f;
  return hipGetLastError() == hipSuccess;
}

inline void free_plan(GemmPlan* p) {
  if (p->desc) hipblasLtMatmulDescDestroy(p->desc);
  if (p->lw) hipblasLtMatrixLayoutDestroy(p->lw);
  if (p->la) hipblasLtMatrixLayoutDestroy(p->la);
  if (p->lc) hipblasLtMatrixLayoutDestroy(p->lc);
  *p = GemmPlan{};
}

}  // namespace pi05
