// The fp32 projections of the batched prefill through hipBLASLt: plain GEMMs
// C[M x N] (+)= A[M x K] . W[N x K]^T (+ bias[N]) whose only epilogues (a bias
// vector, accumulation into the residual rows) the library fuses itself.  At
// the Qwen3-4B prefill shapes (512 rows) it measured 113-137 TFLOP/s against
// 80-107 for the hand-written MFMA GEMM of gemm.hpp (which still serves the
// int8 images: their group dequantisation is fused into its LDS staging).
//
// Row-major operands map onto the library's column-major ones without copies:
// row-major C[M x N] is column-major C^T[N x M], and C^T = W . A^T with W seen
// as a column-major K x N matrix (leading dimension ldw) taken transposed and
// A as a column-major K x M matrix (leading dimension lda).  One plan (matmul
// descriptor, layouts, heuristic algorithm) is kept per shape; the bias
// pointer is set per call.
#pragma once
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <tuple>

namespace kl {

class LtGemm {
 public:
  static constexpr size_t kWorkspaceBytes = size_t(64) << 20;

  // Creates the library handle and its workspace; false if either fails.
  bool init() {
    if (hipblasLtCreate(&handle_) != HIPBLAS_STATUS_SUCCESS) {
      handle_ = nullptr;
      return false;
    }
    if (hipMalloc(&ws_, kWorkspaceBytes) != hipSuccess) {
      ws_ = nullptr;
      return false;
    }
    return true;
  }

  ~LtGemm() {
    for (auto& kv : plans_) {
      Plan& p = kv.second;
      if (p.op) hipblasLtMatmulDescDestroy(p.op);
      if (p.lw) hipblasLtMatrixLayoutDestroy(p.lw);
      if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
      if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    }
    if (ws_) (void)hipFree(ws_);
    if (scratch_) (void)hipFree(scratch_);
    if (handle_) hipblasLtDestroy(handle_);
  }

  // Whether the library has a plan for this shape (built and cached on the
  // first query; a shape without one runs the caller's own kernel).
  bool ready(int M, int N, int K, int lda, int ldw, int ldc, bool has_bias) {
    return plan(M, N, K, lda, ldw, ldc, has_bias) != nullptr;
  }

  // Two products over the same A as one strided batch, C_i = A . W_i^T for
  // i = 0, 1, where W1 and C1 lie w_stride and c_stride elements after W0
  // and C0 (both positive; no bias: the library has no per-batch bias
  // stride).  The batch fills the chip where one narrow product does not
  // (the K and V projections of a prefill).  False if there is no plan or
  // the call fails.
  bool gemm_pair(const float* A, int M, int K, int lda, const float* W0, long long w_stride, int N,
                 int ldw, float* C0, long long c_stride, int ldc, hipStream_t st) {
    if (w_stride <= 0 || c_stride <= 0) return false;
    Plan* p = plan(M, N, K, lda, ldw, ldc, false, w_stride, c_stride);
    if (!p) return false;
    const float alpha = 1.f, beta = 0.f;
    auto run = [&](const hipblasLtMatmulAlgo_t& algo) {
      return hipblasLtMatmul(handle_, p->op, &alpha, W0, p->lw, A, p->la, &beta, C0, p->lc, C0,
                             p->lc, &algo, ws_, kWorkspaceBytes, st) == HIPBLAS_STATUS_SUCCESS;
    };
    tune(p, st, run);  // C = product: the trial runs write the same result
    return run(p->algo);
  }

  // C (+)= A . W^T (+ bias) on stream st; false if the shape has no plan or
  // the call fails.
  bool gemm(const float* A, int M, int K, int lda, const float* W, int N, int ldw, float* C,
            int ldc, const float* bias, bool accumulate, hipStream_t st) {
    Plan* p = plan(M, N, K, lda, ldw, ldc, bias != nullptr);
    if (!p) return false;
    if (bias && hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                                sizeof(bias)) != HIPBLAS_STATUS_SUCCESS)
      return false;
    const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
    if (!p->tuned) {
      // Trial runs of an accumulating product go to a scratch output (C = product
      // there), so C is accumulated into exactly once.
      float* out = accumulate ? tune_scratch(static_cast<size_t>(M) * ldc) : C;
      const float b0 = 0.f;
      if (out)
        tune(p, st, [&](const hipblasLtMatmulAlgo_t& algo) {
          return hipblasLtMatmul(handle_, p->op, &alpha, W, p->lw, A, p->la, &b0, out, p->lc, out,
                                 p->lc, &algo, ws_, kWorkspaceBytes, st) == HIPBLAS_STATUS_SUCCESS;
        });
      p->tuned = true;
    }
    return hipblasLtMatmul(handle_, p->op, &alpha, W, p->lw, A, p->la, &beta, C, p->lc, C, p->lc,
                           &p->algo, ws_, kWorkspaceBytes, st) == HIPBLAS_STATUS_SUCCESS;
  }

 private:
  static constexpr int kCandidates = 16;  // at most this many heuristic algorithms per shape

  struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    hipblasLtMatmulAlgo_t cand[kCandidates]{};
    int ncand = 0;
    bool ok = false;
    bool tuned = false;
  };

  // Times each heuristic candidate of a plan once (one warm-up and three
  // timed runs of `run` on stream st, on the real operands) and keeps the
  // fastest; the library's first choice stays where timing fails.
  // KL_LT_TUNE=0 keeps the first choice without timing.
  template <class Run>
  void tune(Plan* p, hipStream_t st, Run run) {
    if (p->tuned) return;
    p->tuned = true;
    const char* env = std::getenv("KL_LT_TUNE");
    if (p->ncand < 2 || (env && std::atoi(env) == 0)) return;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
      if (e0) (void)hipEventDestroy(e0);
      return;
    }
    float best = 0.f;
    int bi = -1;
    for (int i = 0; i < p->ncand; ++i) {
      if (!run(p->cand[i])) continue;
      bool good = hipEventRecord(e0, st) == hipSuccess;
      for (int r = 0; r < 3 && good; ++r) good = run(p->cand[i]);
      float ms = 0.f;
      good = good && hipEventRecord(e1, st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
             hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
      if (good && (bi < 0 || ms < best)) {
        best = ms;
        bi = i;
      }
    }
    if (bi >= 0) p->algo = p->cand[bi];
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }

  // Scratch output of at least n floats for the trial runs (grown on demand).
  float* tune_scratch(size_t n) {
    if (n > scratch_n_) {
      if (scratch_) (void)hipFree(scratch_);
      scratch_ = nullptr;
      scratch_n_ = 0;
      if (hipMalloc(&scratch_, n * sizeof(float)) != hipSuccess) {
        scratch_ = nullptr;
        return nullptr;
      }
      scratch_n_ = n;
    }
    return scratch_;
  }
  typedef std::tuple<int, int, int, int, int, int, bool, long long, long long> Key;

  // One plan per shape; w_stride > 0 makes it a batch of two (A shared).
  Plan* plan(int M, int N, int K, int lda, int ldw, int ldc, bool has_bias,
             long long w_stride = 0, long long c_stride = 0) {
    const Key key{M, N, K, lda, ldw, ldc, has_bias, w_stride, c_stride};
    auto it = plans_.find(key);
    if (it != plans_.end()) return it->second.ok ? &it->second : nullptr;
    Plan& p = plans_[key];
    bool good = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    good = good &&
           hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
               HIPBLAS_STATUS_SUCCESS;
    if (good && has_bias) {
      const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
      const hipDataType bt = HIP_R_32F;
      good = hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ==
                 HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt,
                                             sizeof(bt)) == HIPBLAS_STATUS_SUCCESS;
    }
    good = good &&
           hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_32F, K, N, ldw) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&p.la, HIP_R_32F, K, M, lda) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, N, M, ldc) == HIPBLAS_STATUS_SUCCESS;
    if (good && w_stride > 0) {
      const int32_t two = 2;
      const int64_t sw = w_stride, sa = 0, sc = c_stride;
      auto batch = [&](hipblasLtMatrixLayout_t l, int64_t stride) {
        return hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &two,
                                                 sizeof(two)) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET,
                                                 &stride, sizeof(stride)) == HIPBLAS_STATUS_SUCCESS;
      };
      good = batch(p.lw, sw) && batch(p.la, sa) && batch(p.lc, sc);
    }
    if (good) {
      hipblasLtMatmulPreference_t pref = nullptr;
      good = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
      const uint64_t wsb = kWorkspaceBytes;
      good = good && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                           &wsb, sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS;
      hipblasLtMatmulHeuristicResult_t res[kCandidates];
      int n = 0, want = kCandidates;  // KL_LT_CANDIDATES: how many to time (1 .. kCandidates)
      if (const char* env = std::getenv("KL_LT_CANDIDATES"))
        want = std::max(1, std::min(kCandidates, std::atoi(env)));
      good = good && hipblasLtMatmulAlgoGetHeuristic(handle_, p.op, p.lw, p.la, p.lc, p.lc, pref,
                                                     want, res, &n) == HIPBLAS_STATUS_SUCCESS;
      for (int i = 0; good && i < n; ++i)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kWorkspaceBytes)
          p.cand[p.ncand++] = res[i].algo;
      good = good && p.ncand > 0;
      if (good) p.algo = p.cand[0];
      if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    }
    p.ok = good;
    return good ? &p : nullptr;
  }

  hipblasLtHandle_t handle_ = nullptr;
  void* ws_ = nullptr;
  float* scratch_ = nullptr;  // trial outputs of accumulating products
  size_t scratch_n_ = 0;
  std::map<Key, Plan> plans_;
};

}  // namespace kl
