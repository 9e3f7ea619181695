// GEMMs through hipBLASLt, the vendor library GEMM: f32, or f16 storage with f32 accumulation (and f32 output
// when asked, for the SwiGLU epilogue pass), with an optional per-column bias and either ReLU / tanh-GELU or a
// residual.
//
// The hand-written MFMA kernels (gemm.hip, f16.hip) keep the forms the library cannot express: output scales,
// activation plus residual, split-K partials for a consumer, the conv loaders, the fused SwiGLU without a
// workspace. lk_hip_gemm_f32, lk_hip_f16_gemm and the one-tap convs call bltGemm and fall back to their own kernels
// when the library has no algorithm for a shape. At the few-hundred-row sizes of ALBERT, the GPT-2 prefill and the
// Qwen3 prefill the library's kernels measured 1.1-1.5x faster than the hand-written ones.
//
// Row-major C = A B is the column-major product C^T [N, M] = B^T [N, K] A^T [K, M]: the row-major buffers are passed
// unchanged as the column-major operands (B first), and the per-column bias becomes hipBLASLt's per-row bias of D.
// A residual R [M, N] is the library's C operand with beta = 1 (D = A B + R + bias, one rounding at the output).
// f32 compute (HIPBLAS_COMPUTE_32F, no reduced-precision inner products) for both storage types. One handle per
// device and one plan per shape, cached for the process: its descriptors and the fastest of the heuristic's first
// eight algorithms, timed on the shape's first (eager) call; LK_BLASLT_NOTUNE=1 keeps the heuristic's first.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>
#include <vector>

namespace lkh {

namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
  bool ok = false;
  bool tuned = false;  // the algorithm is final: chosen on the shape's first call and never changed after
  std::vector<std::pair<hipblasLtMatmulAlgo_t, size_t>> cands;  // the heuristic's candidates (algorithm, workspace)
};

using Key = std::tuple<int, int64_t, int64_t, int64_t, bool, bool, int, bool, bool, size_t>;

std::mutex gMu;
std::map<Key, Plan> gPlans;
std::map<int, hipblasLtHandle_t> gHandles;

hipblasLtHandle_t handleFor(int dev) {
  auto it = gHandles.find(dev);
  if (it != gHandles.end()) return it->second;
  hipblasLtHandle_t h = nullptr;
  if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
  gHandles[dev] = h;
  return h;
}

Plan makePlan(hipblasLtHandle_t h, int64_t m, int64_t n, int64_t k, bool nt, bool bias, int act, bool f16,
              bool f32out, size_t wsMax) {
  Plan p;
  const hipDataType ty = f16 ? HIP_R_16F : HIP_R_32F, tyc = f32out ? HIP_R_32F : ty;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return p;
  const int32_t ta = nt ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  uint32_t epi = bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
  if (act == 1) epi = bias ? HIPBLASLT_EPILOGUE_RELU_BIAS : HIPBLASLT_EPILOGUE_RELU;
  if (act == 2) epi = bias ? HIPBLASLT_EPILOGUE_GELU_BIAS : HIPBLASLT_EPILOGUE_GELU;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
  if (bias) {
    const int32_t bty = tyc;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bty, sizeof(bty));
  }
  // column-major operands: "A" = B^T [N, K] (stored [K, N] with ld N, or [N, K] with ld K read transposed),
  // "B" = A^T [K, M] with ld K, D = C^T [N, M] with ld N
  if (nt) hipblasLtMatrixLayoutCreate(&p.la, ty, static_cast<uint64_t>(k), static_cast<uint64_t>(n), k);
  else hipblasLtMatrixLayoutCreate(&p.la, ty, static_cast<uint64_t>(n), static_cast<uint64_t>(k), n);
  hipblasLtMatrixLayoutCreate(&p.lb, ty, static_cast<uint64_t>(k), static_cast<uint64_t>(m), k);
  hipblasLtMatrixLayoutCreate(&p.lc, tyc, static_cast<uint64_t>(n), static_cast<uint64_t>(m), n);
  if (!p.la || !p.lb || !p.lc) return p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return p;
  const uint64_t wsBytes = wsMax;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsBytes, sizeof(wsBytes));
  constexpr int kCands = 8;
  hipblasLtMatmulHeuristicResult_t res[kCands];
  int got = 0;
  const hipblasStatus_t st =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, kCands, res, &got);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return p;
  for (int i = 0; i < got; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= wsMax)
      p.cands.emplace_back(res[i].algo, res[i].workspaceSize);
  if (p.cands.empty()) return p;
  p.algo = p.cands[0].first;  // the heuristic's first choice until tuned
  p.ws = p.cands[0].second;
  p.ok = true;
  return p;
}

}  // namespace

// C [M, N] = act(A [M, K] B (+ bias [N])) (+ res [M, N], only with act 0: the library's epilogue activation would
// apply after the residual); act 0 none, 1 relu, 2 gelu (tanh form). B [K, N], or [N, K] with nt; f16: A and B are
// IEEE half, and so are bias, res and C unless f32out (then they are f32: the unrounded f32 accumulations). Returns
// false (nothing launched) when no library algorithm fits the shape and the workspace.
bool bltGemm(const void* a, const void* b, const void* bias, const void* res, void* c, int64_t m, int64_t n, int64_t k,
             bool nt, int act, bool f16, bool f32out, void* ws, size_t wsBytes, hipStream_t s) {
  if (act < 0 || act > 2 || (act != 0 && res)) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  // the bias pointer lives in the shared per-shape descriptor: set it and enqueue under the lock
  std::lock_guard<std::mutex> lock(gMu);
  hipblasLtHandle_t h = handleFor(dev);
  if (!h) return false;
  const size_t wsb = ws ? wsBytes : 0;
  const Key key{dev, m, n, k, nt, bias != nullptr, act, f16, f32out && f16, wsb};
  auto it = gPlans.find(key);
  if (it == gPlans.end()) it = gPlans.emplace(key, makePlan(h, m, n, k, nt, bias != nullptr, act, f16, f32out && f16, wsb)).first;
  Plan& plan = it->second;
  if (!plan.ok) return false;
  if (bias && hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
                  HIPBLAS_STATUS_SUCCESS)
    return false;
  const float alpha = 1.0f, beta = res ? 1.0f : 0.0f;
  auto run = [&](const hipblasLtMatmulAlgo_t& algo, size_t wsz) {
    return hipblasLtMatmul(h, plan.desc, &alpha, b, plan.la, a, plan.lb, &beta, res ? res : c, plan.lc, c, plan.lc,
                           &algo, wsz ? ws : nullptr, wsz, s) == HIPBLAS_STATUS_SUCCESS;
  };
  if (!plan.tuned) {
    plan.tuned = true;
    // the shape's first call times the heuristic's candidates on these operands and keeps the fastest. Not while
    // the stream is being captured (the first choice then stays), nor when the residual is the output (each trial
    // run would add it again); the trial runs' outputs are overwritten by the call's own run below.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone;
    if (plan.cands.size() > 1 && !capturing && !(res && res == c) && !getenv("LK_BLASLT_NOTUNE")) {
      hipEvent_t e0 = nullptr, e1 = nullptr;
      if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        float best = -1.0f;
        for (const auto& cand : plan.cands) {
          if (!run(cand.first, cand.second)) continue;  // warm-up; an algorithm that fails here is skipped
          hipEventRecord(e0, s);
          bool okRun = true;
          for (int r = 0; r < 3 && okRun; ++r) okRun = run(cand.first, cand.second);
          hipEventRecord(e1, s);
          float ms = 0.0f;
          if (!okRun || hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
            continue;
          if (best < 0.0f || ms < best) {
            best = ms;
            plan.algo = cand.first;
            plan.ws = cand.second;
          }
        }
      }
      if (e0) hipEventDestroy(e0);
      if (e1) hipEventDestroy(e1);
      (void)hipGetLastError();  // a failed trial leaves no error for the caller's launch check
    }
  }
  return run(plan.algo, plan.ws);
}

}  // namespace lkh
