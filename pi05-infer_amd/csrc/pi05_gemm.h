// hipBLASLt plans shared by the prefill and the vision tower (host code).
//
// C[M, N] (row-major) = A[M, K] (row-major) . W[N, K]^T (nn.Linear layout), fp32 accumulation.
// In hipBLASLt's column-major terms that is C^T (N x M) = W (stored K x N, transposed) . A^T
// (stored K x M).  Options: an fp32 bias per output column added before the one rounding
// (HIPBLASLT_EPILOGUE_BIAS; the pointer is set per call), fp32 operands, split-K batches.
#pragma once

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <string>
#include <utility>
#include <vector>

namespace pi05 {

struct GemmPlan {
  int M = 0, N = 0, K = 0;
  bool bias = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
  std::vector<hipblasLtMatmulHeuristicResult_t> cands;  // heuristic picks + other supported solutions, timed by tune_plan
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
  int ld_c = 0;                 // row length of the output (0: N)
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
      !lt_ok(hipblasLtMatrixLayoutCreate(&p->lc, ct, N, M, o.ld_c ? o.ld_c : N))) {
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
    const int64_t sk = K, sc = (int64_t)(o.ld_c ? o.ld_c : N) * M;
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
  std::vector<int> seen;
  for (int i = 0; lt_ok(s) && i < n; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= ws_max) {
      p->cands.push_back(res[i]);
      seen.push_back(hipblaslt_ext::getIndexFromAlgo(res[i].algo));
    }
  // every other solution the library holds for this problem type that accepts this problem
  // (split-K / stream-K variants the heuristic leaves out fill the GPU at small M x N)
  std::vector<hipblasLtMatmulHeuristicResult_t> all;
  const hipDataType ct_all = ct;
  if (lt_ok(hipblaslt_ext::getAllAlgos(h, hipblaslt_ext::GemmType::HIPBLASLT_GEMM, ta, tb, o.ab, o.ab, ct_all, ct_all, HIPBLAS_COMPUTE_32F, all))) {
    const float alpha = 1.f, beta = 0.f;
    for (auto& r : all) {
      const int idx = hipblaslt_ext::getIndexFromAlgo(r.algo);
      if (std::find(seen.begin(), seen.end(), idx) != seen.end()) continue;
      size_t wsz = 0;
      if (!lt_ok(hipblaslt_ext::matmulIsAlgoSupported(h, p->desc, &alpha, p->lw, p->la, &beta, p->lc, p->lc, r.algo, wsz)) || wsz > ws_max)
        continue;
      r.workspaceSize = wsz;
      r.state = HIPBLAS_STATUS_SUCCESS;
      p->cands.push_back(r);
      seen.push_back(idx);
    }
  }
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

// Time every candidate algorithm on real buffers (2 runs after one warm-up; values do not affect
// the timing), re-time the 6 fastest and keep the best; candidates that fail to launch are skipped.  w_stride / w_count: see w_at below.
inline bool tune_plan(hipblasLtHandle_t h, GemmPlan* p, const void* W, const void* A, void* C, void* ws, hipStream_t st,
                      const float* bias = nullptr, size_t w_stride = 0, int w_count = 1) {
  // run r reads the weights at W + (r mod w_count) * w_stride: with one weight block per layer the
  // timed runs stream weights from HBM as the layer loop does, instead of re-reading a cached block
  auto w_at = [&](int r) { return static_cast<const void*>(static_cast<const char*>(W) + (size_t)(r % w_count) * w_stride); };
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return false;
  if (hipEventCreate(&e1) != hipSuccess) {
    hipEventDestroy(e0);
    return false;
  }
  auto time_algo = [&](const hipblasLtMatmulHeuristicResult_t& c, int reps, float* ms) {
    bool ok = lt_ok(run_plan(h, *p, c.algo, c.workspaceSize, w_at(w_count - 1), A, C, bias, ws, st));
    if (!ok) return false;
    hipEventRecord(e0, st);
    for (int r = 0; r < reps && ok; ++r) ok = lt_ok(run_plan(h, *p, c.algo, c.workspaceSize, w_at(r), A, C, bias, ws, st));
    hipEventRecord(e1, st);
    if (hipEventSynchronize(e1) != hipSuccess || !ok || hipEventElapsedTime(ms, e0, e1) != hipSuccess) return false;
    *ms /= (float)reps;
    return true;
  };
  std::vector<std::pair<float, size_t>> timed;
  for (size_t i = 0; i < p->cands.size(); ++i) {
    float ms = 0.f;
    if (time_algo(p->cands[i], 2, &ms)) timed.emplace_back(ms, i);
  }
  std::sort(timed.begin(), timed.end());
  // finalists: 3 interleaved rounds of 10 runs each (so clock drift hits them alike), best round kept
  const size_t nf = timed.size() < 6 ? timed.size() : 6;
  std::vector<float> score(nf, 1e30f);
  for (int round = 0; round < 3; ++round)
    for (size_t k = 0; k < nf; ++k) {
      float ms = 0.f;
      if (time_algo(p->cands[timed[k].second], 10, &ms) && ms < score[k]) score[k] = ms;
    }
  float best = 1e30f;
  for (size_t k = 0; k < nf; ++k)
    if (score[k] < best) {
      best = score[k];
      p->algo = p->cands[timed[k].second].algo;
      p->ws = p->cands[timed[k].second].workspaceSize;
    }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  p->ms = best;
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
