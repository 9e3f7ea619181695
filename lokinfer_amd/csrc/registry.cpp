// Kernel registry and the C-ABI boundary.
//
// Every GPU kernel name of the reference's compiled path is registered here with the reference's argument
// convention (include/lokinfer/runtime/kernel.h:1-11, src/runtime/executable.cpp:406-447 in lariaus/lokinfer):
// ptrs = operands then outs; ints = every operand's dims, every out's dims, then int attrs in attribute-name
// order; floats = float attrs in attribute-name order. A RunFn decodes that and calls the typed lk_hip_*
// launcher on the call's stream. Invalid shapes set ExecCtx::error (a static string) like the reference's
// kernels do; the C-ABI turns that into a nonzero status plus lk_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "lokinfer_hip.h"

namespace lkh {

namespace {

std::map<std::string, KernelEntry>& table() {
  static std::map<std::string, KernelEntry> t;
  return t;
}

std::vector<std::string>& names() {
  static std::vector<std::string> n;
  return n;
}

thread_local std::string tlsError;

}  // namespace

void setLastError(std::string msg) { tlsError = std::move(msg); }

void registerKernel(const KernelEntry& e) {
  auto& t = table();
  if (t.find(e.name) == t.end()) names().push_back(e.name);
  t[e.name] = e;
}

// ---- GEMM family ------------------------------------------------------------------------------------------

namespace {

// operands a[M, K], b[K, N] or b^T [N, K], [bias[N]], [res[M, N]]; out [M, N]
template <bool NT, bool BIAS, int ACT, bool RES>
void runGemm(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t m = it.next(), k = it.next();
  int64_t kb, n;
  if (NT) {
    n = it.next();
    kb = it.next();
  } else {
    kb = it.next();
    n = it.next();
  }
  LK_REQUIRE(ctx, kb == k, "gemm: inner dimensions differ");
  int idx = 2;
  const float* bias = BIAS ? P<float>(a, idx++) : nullptr;
  const float* res = RES ? P<float>(a, idx++) : nullptr;
  float* out = P<float>(a, idx);
  if (NT && m <= 8 && !BIAS && !RES && ACT == 0 && k % 4 == 0) {
    status(ctx, lk_hip_rowdot_f32(P<float>(a, 1), P<float>(a, 0), nullptr, 0, out, n, k, static_cast<int>(m), n,
                                  ctx.stream),
           "gemm_nt: launch failed");
    return;
  }
  status(ctx, lk_hip_gemm_f32(P<float>(a, 0), P<float>(a, 1), bias, res, out, m, n, k, NT ? 1 : 0, ACT, 1.0f,
                              ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream),
         "gemm: launch failed");
}

// gemv4 / gemv: x[1, K], w[K, N], [b[N]], [r[1, N]] -> out[1, N]
template <bool BIAS, int ACT, bool RES>
void runGemv(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  LK_REQUIRE(ctx, it.next() == 1, "gemv: x must be f32[1, K]");
  const int64_t k = it.next();
  LK_REQUIRE(ctx, it.next() == k, "gemv: w must be f32[K, N]");
  const int64_t n = it.next();
  int idx = 2;
  const float* bias = BIAS ? P<float>(a, idx++) : nullptr;
  const float* res = RES ? P<float>(a, idx++) : nullptr;
  status(ctx,
         lk_hip_gemv_f32(P<float>(a, 0), P<float>(a, 1), bias, res, P<float>(a, idx), n, k, ACT, ctx.workspace,
                         ctx.workspaceBytes, ctx.stream),
         "gemv: launch failed");
}

// gemv_rows: x[1, K] . rows of w[N, K] -> [1, N]
void runGemvRows(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  LK_REQUIRE(ctx, it.next() == 1, "gemv_rows: x must be f32[1, K]");
  const int64_t k = it.next(), n = it.next();
  LK_REQUIRE(ctx, it.next() == k && k % 4 == 0, "gemv_rows: w must be f32[N, K], K % 4 == 0");
  status(ctx, lk_hip_rowdot_f32(P<float>(a, 1), P<float>(a, 0), nullptr, 0, P<float>(a, 2), n, k, 1, n, ctx.stream),
         "gemv_rows: launch failed");
}

// gemv1_bias: x[R, K] . w[K, 1] + b[1] -> [R, 1]
void runGemv1Bias(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), k = it.next();
  LK_REQUIRE(ctx, it.next() == k && it.next() == 1 && k % 4 == 0, "gemv1_bias: w must be f32[K, 1], K % 4 == 0");
  status(ctx, lk_hip_rowdot_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), 0, P<float>(a, 3), r, k, 1, r,
                                ctx.stream),
         "gemv1_bias: launch failed");
}

// conv1d_lc: x[L, Ci], w[Co, K, Ci], b[Co], [res[Lo, Co]]; attrs dilation, [oscale], padding, stride
template <bool RES>
void runConvLc(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), ci = it.next();
  const int64_t co = it.next(), kw = it.next();
  LK_REQUIRE(ctx, it.next() == ci, "conv1d_lc: w must be f32[Co, K, Ci]");
  it.skip(1);               // b
  if (RES) it.skip(2);      // res
  it.skip(2);               // out
  const int dil = static_cast<int>(it.next()), pad = static_cast<int>(it.next()), str = static_cast<int>(it.next());
  const float scale = RES ? F(a, 0, 1.0f) : 1.0f;
  LK_REQUIRE(ctx, ci % 16 == 0, "conv1d_lc: Ci must be a multiple of 16");
  const float* res = RES ? P<float>(a, 3) : nullptr;
  float* out = P<float>(a, RES ? 4 : 3);
  status(ctx, lk_hip_conv1d_lc_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), res, out, l, ci, co, kw, str, pad,
                                   dil, scale, nullptr, nullptr, 0, 0.0f, nullptr, ctx.workspace,
                                   static_cast<int64_t>(ctx.workspaceBytes), ctx.stream),
         "conv1d_lc: invalid configuration");
}

// conv1d_act_lc[_res][_stats] (this backend's fused prologue conv): x[L, Ci], w[Co, K, Ci], b[Co], affine[3, Ci],
// alpha[Ci], [res[Lo, Co]] -> out[Lo, Co] [, stats[ceil(Lo / 128), Co, 2]]; ints attrs: act (0 affine only,
// 1 snake, 2 leaky), dilation, padding, stride; floats: oscale, slope
template <bool RES, bool STATS>
void runConvActLc(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), ci = it.next();
  const int64_t co = it.next(), kw = it.next();
  LK_REQUIRE(ctx, it.next() == ci, "conv1d_act_lc: w must be f32[Co, K, Ci]");
  it.skip(1 + 2 + 1);  // b, affine, alpha
  if (RES) it.skip(2);
  const int64_t lo = it.next();
  it.skip(1);
  if (STATS) {
    LK_REQUIRE(ctx, it.next() == (lo + 127) / 128 && it.next() == co && it.next() == 2,
               "conv1d_act_lc_stats: stats must be f32[ceil(Lo / 128), Co, 2]");
  }
  const int act = static_cast<int>(it.next());
  const int dil = static_cast<int>(it.next()), pad = static_cast<int>(it.next()), str = static_cast<int>(it.next());
  const float scale = F(a, 0, 1.0f), slope = F(a, 1, 0.0f);
  LK_REQUIRE(ctx, ci % 16 == 0, "conv1d_act_lc: Ci must be a multiple of 16");
  const float* res = RES ? P<float>(a, 5) : nullptr;
  float* out = P<float>(a, RES ? 6 : 5);
  float* stats = STATS ? P<float>(a, RES ? 7 : 6) : nullptr;
  status(ctx, lk_hip_conv1d_lc_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), res, out, l, ci, co, kw, str, pad,
                                   dil, scale, P<float>(a, 3), P<float>(a, 4), act, slope, stats, ctx.workspace,
                                   static_cast<int64_t>(ctx.workspaceBytes), ctx.stream),
         "conv1d_act_lc: invalid configuration");
}

}  // namespace

void registerGemmKernels() {
  const Device G = Device::Gpu;
  registerKernel({"gemm_f32_gpu_mps", G, runGemm<false, false, 0, false>, 2, 1});
  registerKernel({"gemm_nt_f32_gpu_mps", G, runGemm<true, false, 0, false>, 2, 1});
  registerKernel({"gemm_f32_gpu", G, runGemm<false, false, 0, false>, 2, 1});
  registerKernel({"gemm_bias_f32_gpu", G, runGemm<false, true, 0, false>, 3, 1});
  registerKernel({"gemm_bias_relu_f32_gpu", G, runGemm<false, true, 1, false>, 3, 1});
  registerKernel({"gemm_steel_f32_gpu", G, runGemm<false, false, 0, false>, 2, 1});
  registerKernel({"gemm_steel_bias_f32_gpu", G, runGemm<false, true, 0, false>, 3, 1});
  registerKernel({"gemm_steel_bias_relu_f32_gpu", G, runGemm<false, true, 1, false>, 3, 1});
  registerKernel({"gemm_steel_bias_gelu_f32_gpu", G, runGemm<false, true, 2, false>, 3, 1});
  registerKernel({"gemm_steel_bias_res_f32_gpu", G, runGemm<false, true, 0, true>, 4, 1});
  registerKernel({"gemm_nt_steel_f32_gpu", G, runGemm<true, false, 0, false>, 2, 1});
  registerKernel({"gemv4_f32_gpu", G, runGemv<false, 0, false>, 2, 1});
  registerKernel({"gemv4_bias_f32_gpu", G, runGemv<true, 0, false>, 3, 1});
  registerKernel({"gemv4_bias_gelu_f32_gpu", G, runGemv<true, 2, false>, 3, 1});
  registerKernel({"gemv4_bias_res_f32_gpu", G, runGemv<true, 0, true>, 4, 1});
  registerKernel({"gemv_f32_gpu", G, runGemv<false, 0, false>, 2, 1});
  registerKernel({"gemv_bias_f32_gpu", G, runGemv<true, 0, false>, 3, 1});
  registerKernel({"gemv_bias_gelu_f32_gpu", G, runGemv<true, 2, false>, 3, 1});
  registerKernel({"gemv_rows_f32_gpu", G, runGemvRows, 2, 1});
  registerKernel({"gemv1_bias_f32_gpu", G, runGemv1Bias, 3, 1});
  registerKernel({"conv1d_lc_f32_gpu", G, runConvLc<false>, 3, 1});
  registerKernel({"conv1d_lc_res_f32_gpu", G, runConvLc<true>, 4, 1});
  registerKernel({"conv1d_act_lc_f32_gpu", G, runConvActLc<false, false>, 5, 1});
  registerKernel({"conv1d_act_lc_res_f32_gpu", G, runConvActLc<true, false>, 6, 1});
  registerKernel({"conv1d_act_lc_stats_f32_gpu", G, runConvActLc<false, true>, 5, 2});
  registerKernel({"conv1d_act_lc_res_stats_f32_gpu", G, runConvActLc<true, true>, 6, 2});
}

// ---- transformer ------------------------------------------------------------------------------------------

namespace {

// layernorm: x[R, C], gamma[C], beta[C]; float eps
void runLayerNorm(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), c = it.next();
  LK_REQUIRE(ctx, c <= 2048, "layernorm: C must be <= 2048");
  status(ctx, lk_hip_layernorm_f32(P<float>(a, 0), nullptr, nullptr, P<float>(a, 1), P<float>(a, 2), nullptr,
                                   P<float>(a, 3), r, c, F(a, 0, 1e-5f), 0, ctx.stream),
         "layernorm: launch failed");
}

// add_bias_layernorm[2]: a[R, C], bias[C], r[R, C], gamma, beta -> out (LN) or (sum, LN)
template <bool TWO>
void runAddBiasLn(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), c = it.next();
  LK_REQUIRE(ctx, c <= 2048, "add_bias_layernorm: C must be <= 2048");
  float* sum = TWO ? P<float>(a, 5) : nullptr;
  float* out = P<float>(a, TWO ? 6 : 5);
  status(ctx, lk_hip_layernorm_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), P<float>(a, 4), sum,
                                   out, r, c, F(a, 0, TWO ? 1e-5f : 1e-12f), TWO ? 2 : 1, ctx.stream),
         "add_bias_layernorm: launch failed");
}

void runBiasGelu(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), c = it.next();
  status(ctx, lk_hip_bias_gelu_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), r, c, ctx.stream),
         "bias_gelu: launch failed");
}

// attention_qkv[_sg][_causal]: qkv[T, 3D], bias[3D]; attrs heads[, nsg]
template <bool CAUSAL>
void runAttnQkv(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d3 = it.next();
  it.skip(1 + 2);  // bias, out
  const int heads = static_cast<int>(it.next());
  LK_REQUIRE(ctx, heads > 0 && d3 == 3 * 64 * heads, "attention_qkv: qkv must be f32[T, 3D] with head_dim 64");
  status(ctx, lk_hip_attention_qkv_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), t, heads, CAUSAL ? 1 : 0,
                                       ctx.stream),
         "attention_qkv: launch failed");
}

// attention_decode_split / _kvw / plain: qkv[1, 3D], kc[cap, D], vc[cap, D], pos[1] (device i64), bias[3D];
// attrs heads[, nsg, single, splits]. kvw / split variants write row pos of both caches.
template <bool WRITE, bool SPLITATTRS>
void runAttnDecode(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  LK_REQUIRE(ctx, it.next() == 1, "attention_decode: qkv must be f32[1, 3D]");
  const int64_t d3 = it.next();
  const int64_t cap = it.next(), d = it.next();
  it.skip(2 + 1 + 1 + 2);  // vc, pos, bias, out
  const int heads = static_cast<int>(it.next());
  int splitsAttr = 0;
  if (SPLITATTRS) {
    it.skip(2);  // nsg, single (Metal launch shapes; no meaning on CDNA4)
    splitsAttr = static_cast<int>(it.next());
  }
  LK_REQUIRE(ctx, d3 == 3 * d && d == 64 * heads, "attention_decode: head_dim must be 64, qkv f32[1, 3D]");
  // The splits attr (reference: Metal key-split count, 0 = auto) has no meaning here: the CDNA4 kernel always
  // uses 64-key chunks (one wave each) and a merge launch.
  (void)splitsAttr;
  const int rc = lk_hip_attention_decode_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                             P<float>(a, 4), P<float>(a, 5), cap, heads, cap, WRITE ? 1 : 0,
                                             ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream);
  status(ctx, rc, rc == 3 ? "attention_decode: workspace too small" : "attention_decode: launch failed");
}

// kv_write_f32_gpu (inout kc, vc): kc[cap, D], vc[cap, D], qkv[1, 3D], pos[1], bias[3D]; no outs
void runKvWrite(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t cap = it.next(), d = it.next();
  status(ctx, lk_hip_kv_write_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3), P<float>(a, 4),
                                  d, cap, ctx.stream),
         "kv_write: launch failed");
}

// kv_write_rows_f32_gpu (inout kc, vc): kc[cap, D], vc[cap, D], qkv[T, 3D], pos[1], bias[3D]; no outs. Rows past
// the cache are dropped on the device (the reference's host check "pos + T exceeds the cache" needs pos on the host).
void runKvWriteRows(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t cap = it.next(), d = it.next();
  it.skip(2);
  const int64_t t = it.next(), d3 = it.next();
  LK_REQUIRE(ctx, d3 == 3 * d && d % 4 == 0, "kv_write_rows: qkv must be f32[T, 3D] over caches f32[P, D]");
  status(ctx, lk_hip_kv_write_rows_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                       P<float>(a, 4), t, d, cap, ctx.stream),
         "kv_write_rows: launch failed");
}

// attention_cache[_sg]_f32_gpu: qkv[T, 3D], kc[cap, D], vc[cap, D], pos[1], bias[3D] -> out[T, D]; attrs heads[, nsg]
void runAttnCache(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d3 = it.next(), cap = it.next(), d = it.next();
  it.skip(2 + 1 + 1 + 2);  // vc, pos, bias, out
  const int heads = static_cast<int>(it.next());
  LK_REQUIRE(ctx, d3 == 3 * d && d == 64 * heads, "attention_cache: head_dim must be 64, qkv f32[T, 3D]");
  status(ctx, lk_hip_attention_cache_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                         P<float>(a, 4), P<float>(a, 5), t, heads, cap, ctx.stream),
         "attention_cache: launch failed");
}

// attention_gen[2]_f32_gpu (inout kc, vc): same operands as attention_cache. T = 1 -> the split-key decode attention
// that also writes row pos; T > 1 -> kv_write_rows, then the flash attention over the cache.
void runAttnGen(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d3 = it.next(), cap = it.next(), d = it.next();
  it.skip(2 + 1 + 1 + 2);
  const int heads = static_cast<int>(it.next());
  LK_REQUIRE(ctx, d3 == 3 * d && d == 64 * heads && d % 4 == 0, "attention_gen: head_dim must be 64");
  if (t == 1) {
    const int rc = lk_hip_attention_decode_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                               P<float>(a, 4), P<float>(a, 5), cap, heads, cap, 1, ctx.workspace,
                                               static_cast<int64_t>(ctx.workspaceBytes), ctx.stream);
    status(ctx, rc, rc == 3 ? "attention_gen: workspace too small" : "attention_gen: launch failed");
    return;
  }
  status(ctx, lk_hip_kv_write_rows_f32(P<float>(a, 1), P<float>(a, 2), P<float>(a, 0), P<int64_t>(a, 3),
                                       P<float>(a, 4), t, d, cap, ctx.stream),
         "attention_gen: kv_write_rows failed");
  if (ctx.error) return;
  status(ctx, lk_hip_attention_cache_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                         P<float>(a, 4), P<float>(a, 5), t, heads, cap, ctx.stream),
         "attention_gen: attention_cache failed");
}

// Split-K pays while the 64 x 64 output tiles leave most of the 256 CUs idle; above that (and for M = 1, where the
// work is one GEMV) the producer writes one plane and the consumer reads one. The rule is shared by
// gemm_splitk / gemm_auto_sk and add_bias_layernorm2_sk (reference splitKEffective, transformer_gpu.cpp:253-268,
// whose threshold is tuned for its own GPU).
constexpr int64_t kSplitKMaxTiles = 64;
int64_t splitKPlanes(int64_t m, int64_t n, int64_t splits) {
  return m > 1 && ((m + 63) / 64) * ((n + 63) / 64) < kSplitKMaxTiles ? splits : 1;
}

// gemm_splitk / gemm_auto_sk: a[M, K], b[K, N] -> out[S, M, N]; attrs splits, tile. Planes past splitKPlanes are
// not written (their consumer does not read them).
template <bool AUTO>
void runGemmSplitK(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t m = it.next(), k = it.next();
  LK_REQUIRE(ctx, it.next() == k, "gemm_splitk: inner dimensions differ");
  const int64_t n = it.next();
  it.skip(3);
  const int64_t splits = it.next(), tile = it.next();
  LK_REQUIRE(ctx, splits >= 1 && k % (16 * splits) == 0, "gemm_splitk: K must be divisible by 16*splits");
  LK_REQUIRE(ctx, tile == 32 || tile == 64, "gemm_splitk: tile must be 32 or 64");
  const int64_t planes = splitKPlanes(m, n, splits);
  if (planes == 1) {
    if (AUTO && m == 1)
      status(ctx, lk_hip_gemv_f32(P<float>(a, 0), P<float>(a, 1), nullptr, nullptr, P<float>(a, 2), n, k, 0,
                                  ctx.workspace, ctx.workspaceBytes, ctx.stream),
             "gemm_auto_sk: launch failed");
    else
      status(ctx, lk_hip_gemm_f32(P<float>(a, 0), P<float>(a, 1), nullptr, nullptr, P<float>(a, 2), m, n, k, 0, 0,
                                  1.0f, ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream),
             "gemm_splitk: launch failed");
    return;
  }
  status(ctx, lk_hip_gemm_splitk_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), m, n, k,
                                     static_cast<int>(planes), ctx.stream),
         "gemm_splitk: launch failed (K, N % 4 and 16-byte aligned operands needed)");
}

// add_bias_layernorm2_sk: parts[S, R, C], bias[C], r[R, C], gamma, beta -> (sum, LN); float eps
void runAddBiasLnSk(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t s = it.next(), r = it.next(), c = it.next();
  LK_REQUIRE(ctx, c <= 2048, "add_bias_layernorm2_sk: C must be <= 2048");
  status(ctx, lk_hip_add_bias_ln_sk_f32(P<float>(a, 0), splitKPlanes(r, c, s), P<float>(a, 1), P<float>(a, 2),
                                        P<float>(a, 3), P<float>(a, 4), P<float>(a, 5), P<float>(a, 6), r, c,
                                        F(a, 0, 1e-5f), ctx.stream),
         "add_bias_layernorm2_sk: launch failed");
}

// gemm_auto[_bias_gelu]: x[M, K], w[K, N][, bias[N]] -> [M, N]; M = 1 -> GEMV, else the MFMA GEMM
template <bool GELU>
void runGemmAuto(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t m = it.next(), k = it.next();
  LK_REQUIRE(ctx, it.next() == k, "gemm_auto: inner dimensions differ");
  const int64_t n = it.next();
  const float* bias = GELU ? P<float>(a, 2) : nullptr;
  float* out = P<float>(a, GELU ? 3 : 2);
  if (m == 1)
    status(ctx, lk_hip_gemv_f32(P<float>(a, 0), P<float>(a, 1), bias, nullptr, out, n, k, GELU ? 2 : 0, ctx.workspace,
                                ctx.workspaceBytes, ctx.stream),
           "gemm_auto: launch failed");
  else
    status(ctx, lk_hip_gemm_f32(P<float>(a, 0), P<float>(a, 1), bias, nullptr, out, m, n, k, 0, GELU ? 2 : 0, 1.0f,
                                ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream),
           "gemm_auto: launch failed");
}

}  // namespace

void registerTransformerKernels() {
  const Device G = Device::Gpu;
  registerKernel({"layernorm_f32_gpu", G, runLayerNorm, 3, 1});
  registerKernel({"add_bias_layernorm_f32_gpu", G, runAddBiasLn<false>, 5, 1});
  registerKernel({"add_bias_layernorm2_f32_gpu", G, runAddBiasLn<true>, 5, 2});
  registerKernel({"bias_gelu_f32_gpu", G, runBiasGelu, 2, 1});
  registerKernel({"attention_qkv_f32_gpu", G, runAttnQkv<false>, 2, 1});
  registerKernel({"attention_qkv_causal_f32_gpu", G, runAttnQkv<true>, 2, 1});
  registerKernel({"attention_qkv_sg_f32_gpu", G, runAttnQkv<false>, 2, 1});
  registerKernel({"attention_qkv_sg_causal_f32_gpu", G, runAttnQkv<true>, 2, 1});
  registerKernel({"attention_decode_split_f32_gpu", G, runAttnDecode<true, true>, 5, 1});
  registerKernel({"attention_decode_kvw_f32_gpu", G, runAttnDecode<true, false>, 5, 1});
  registerKernel({"attention_decode_f32_gpu", G, runAttnDecode<false, false>, 5, 1});
  registerKernel({"kv_write_f32_gpu", G, runKvWrite, 5, 0});
  registerKernel({"kv_write_rows_f32_gpu", G, runKvWriteRows, 5, 0});
  registerKernel({"attention_cache_f32_gpu", G, runAttnCache, 5, 1});
  registerKernel({"attention_cache_sg_f32_gpu", G, runAttnCache, 5, 1});
  registerKernel({"attention_gen_f32_gpu", G, runAttnGen, 5, 1});
  registerKernel({"attention_gen2_f32_gpu", G, runAttnGen, 5, 1});
  registerKernel({"gemm_splitk_f32_gpu", G, runGemmSplitK<false>, 2, 1});
  registerKernel({"gemm_auto_sk_f32_gpu", G, runGemmSplitK<true>, 2, 1});
  registerKernel({"add_bias_layernorm2_sk_f32_gpu", G, runAddBiasLnSk, 5, 2});
  registerKernel({"gemm_auto_f32_gpu", G, runGemmAuto<false>, 2, 1});
  registerKernel({"gemm_auto_bias_gelu_f32_gpu", G, runGemmAuto<true>, 3, 1});
}

// ---- Kokoro frame-rate ------------------------------------------------------------------------------------

namespace {

void runStats(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), c = it.next();
  status(ctx, lk_hip_channel_stats_lc_f32(P<float>(a, 0), P<float>(a, 1), l, c, ctx.stream), "channel_stats: failed");
}

// adain_affine_lc: stats[S, C, 2], gb[2 Creal]; attrs length (int), eps (float)
void runAdainAffine(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t s = it.next(), c = it.next();
  it.skip(1);
  const int64_t g2 = it.next();
  it.skip(2);
  const int64_t length = it.next();
  LK_REQUIRE(ctx, s == (length + 127) / 128 && g2 % 2 == 0 && g2 / 2 <= c, "adain_affine_lc: bad stats / gb");
  status(ctx, lk_hip_adain_affine_lc_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), length, c, g2 / 2,
                                         F(a, 0, 1e-5f), ctx.stream),
         "adain_affine_lc: failed");
}

// snake_affine_lc(x, affine, alpha); leaky_affine_lc(x, affine; slope); leaky_lc(x; slope)
template <int ACT, bool AFF>
void runAct(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), c = it.next();
  const float* af = AFF ? P<float>(a, 1) : nullptr;
  const float* alpha = ACT == 1 ? P<float>(a, 2) : nullptr;
  const int outIdx = ACT == 1 ? 3 : (AFF ? 2 : 1);
  status(ctx, lk_hip_act_lc_f32(P<float>(a, 0), af, alpha, P<float>(a, outIdx), l, c, ACT, F(a, 0), ctx.stream),
         "act_lc: failed");
}

// convt_gather_lc[_add]: y[Lin, K*Co], b[Co], [add[Lout, Co]]; attrs kernel, padding, reflect_left, stride
template <bool ADD>
void runConvtGather(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t lin = it.next(), kco = it.next();
  const int64_t co = it.next();
  if (ADD) it.skip(2);
  const int64_t lout = it.next();
  it.skip(1);
  const int k = static_cast<int>(it.next()), pad = static_cast<int>(it.next());
  const int refl = static_cast<int>(it.next()), str = static_cast<int>(it.next());
  LK_REQUIRE(ctx, kco == k * co && lout == (lin - 1) * str - 2 * pad + k + refl, "convt_gather_lc: bad shapes");
  status(ctx, lk_hip_convt_gather_lc_f32(P<float>(a, 0), P<float>(a, 1), ADD ? P<float>(a, 2) : nullptr,
                                         P<float>(a, ADD ? 3 : 2), lin, lout, co, k, str, pad, refl, ctx.stream),
         "convt_gather_lc: failed");
}

// dwconvt_lc: x[Lin, C], w[C, K], b[C]; attrs padding, stride
void runDwConvt(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t lin = it.next(), c = it.next();
  it.skip(1);
  const int k = static_cast<int>(it.next());
  it.skip(1);
  const int64_t lout = it.next();
  it.skip(1);
  const int pad = static_cast<int>(it.next()), str = static_cast<int>(it.next());
  status(ctx, lk_hip_dwconvt_lc_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), lin, lout, c, k,
                                    str, pad, ctx.stream),
         "dwconvt_lc: failed");
}

void runUpsample2(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), c = it.next();
  status(ctx, lk_hip_upsample2_lc_f32(P<float>(a, 0), P<float>(a, 1), l, c, ctx.stream), "upsample2_lc: failed");
}

// concat_pad_lc(a, b; cout) / pad_cols_lc(a; cout)
template <bool TWO>
void runConcatPad(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), ca = it.next();
  int64_t cb = 0;
  if (TWO) {
    LK_REQUIRE(ctx, it.next() == l, "concat_pad_lc: row counts differ");
    cb = it.next();
  }
  it.skip(2);
  const int64_t cout = it.next();
  status(ctx, lk_hip_concat_pad_lc_f32(P<float>(a, 0), TWO ? P<float>(a, 1) : nullptr, P<float>(a, TWO ? 2 : 1), l, ca,
                                       cb, cout, ctx.stream),
         "concat_pad_lc: failed");
}

// lc_to_cf(x[L, Cpad]; channels) -> [channels, L]
void runLcToCf(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), cpad = it.next();
  it.skip(2);
  const int64_t ch = it.next();
  LK_REQUIRE(ctx, ch <= cpad, "lc_to_cf: channels exceeds the padded width");
  status(ctx, lk_hip_transpose_f32(P<float>(a, 0), P<float>(a, 1), l, ch, cpad, ctx.stream), "lc_to_cf: failed");
}

void runTranspose(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), c = it.next();
  status(ctx, lk_hip_transpose_f32(P<float>(a, 0), P<float>(a, 1), r, c, c, ctx.stream), "transpose: failed");
}

int64_t numel(const KernelArgs& a, uint32_t rank) {
  int64_t n = 1;
  for (uint32_t i = 0; i < rank; ++i) n *= a.ints[i];
  return n;
}

// add / mul / add3_scale over any shape: the element count is the product of operand 0's dims, whose rank is
// (numInts - attrs) / (operands + 1).
template <int OP>
void runElementwise(ExecCtx& ctx, const KernelArgs& a) {
  const uint32_t nOperands = OP == 2 ? 3 : 2;
  const uint32_t rank = a.numInts / (nOperands + 1);
  const int64_t n = numel(a, rank);
  status(ctx, lk_hip_elementwise_f32(P<float>(a, 0), P<float>(a, 1), OP == 2 ? P<float>(a, 2) : nullptr,
                                     P<float>(a, nOperands), n, OP, OP == 2 ? F(a, 0, 1.0f) : 1.0f, ctx.stream),
         "elementwise: failed");
}

// istft_logits_lc(x[L, Cpad]; hop, n_fft) -> [hop (L - 1)]
void runIstft(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t l = it.next(), cpad = it.next();
  it.skip(1);
  const int hop = static_cast<int>(it.next()), nfft = static_cast<int>(it.next());
  status(ctx, lk_hip_istft_lc_f32(P<float>(a, 0), P<float>(a, 1), l, cpad, nfft, hop, ctx.stream),
         "istft_logits_lc: invalid configuration");
}

}  // namespace

void registerKokoroKernels() {
  const Device G = Device::Gpu;
  registerKernel({"channel_stats_lc_f32_gpu", G, runStats, 1, 1});
  registerKernel({"adain_affine_lc_f32_gpu", G, runAdainAffine, 2, 1});
  registerKernel({"snake_affine_lc_f32_gpu", G, runAct<1, true>, 3, 1});
  registerKernel({"leaky_affine_lc_f32_gpu", G, runAct<2, true>, 2, 1});
  registerKernel({"leaky_lc_f32_gpu", G, runAct<2, false>, 1, 1});
  registerKernel({"convt_gather_lc_f32_gpu", G, runConvtGather<false>, 2, 1});
  registerKernel({"convt_gather_add_lc_f32_gpu", G, runConvtGather<true>, 3, 1});
  registerKernel({"dwconvt_lc_f32_gpu", G, runDwConvt, 3, 1});
  registerKernel({"upsample2_lc_f32_gpu", G, runUpsample2, 1, 1});
  registerKernel({"concat_pad_lc_f32_gpu", G, runConcatPad<true>, 2, 1});
  registerKernel({"pad_cols_lc_f32_gpu", G, runConcatPad<false>, 1, 1});
  registerKernel({"lc_to_cf_f32_gpu", G, runLcToCf, 1, 1});
  registerKernel({"transpose_f32_gpu", G, runTranspose, 1, 1});
  registerKernel({"add_f32_gpu", G, runElementwise<0>, 2, 1});
  registerKernel({"mul_f32_gpu", G, runElementwise<1>, 2, 1});
  registerKernel({"add3_scale_f32_gpu", G, runElementwise<2>, 3, 1});
  registerKernel({"istft_logits_lc_f32_gpu", G, runIstft, 1, 1});
}

static void registerAll() {
  static std::once_flag once;
  std::call_once(once, [] {
    registerGemmKernels();
    registerTransformerKernels();
    registerKokoroKernels();
    registerFrontendKernels();
    registerSequenceKernels();
    registerSignalKernels();
    registerDecodeFusedKernels();
    registerWinogradKernels();
    registerF16Kernels();
    std::sort(names().begin(), names().end());
  });
}

}  // namespace lkh

namespace lkh {
const KernelEntry* findKernel(const std::string& name) {
  registerAll();
  auto it = table().find(name);
  return it == table().end() ? nullptr : &it->second;
}
}  // namespace lkh

// ---- C-ABI --------------------------------------------------------------------------------------------------
extern "C" {

int lk_init(void) {
  lkh::registerAll();
  return 0;
}

int lk_num_kernels(void) {
  lkh::registerAll();
  return static_cast<int>(lkh::names().size());
}

const char* lk_kernel_name_at(int i) {
  lkh::registerAll();
  if (i < 0 || i >= static_cast<int>(lkh::names().size())) return nullptr;
  return lkh::names()[i].c_str();
}

const lk_kernel* lk_find_kernel(const char* name) {
  lkh::registerAll();
  auto it = lkh::table().find(name ? name : "");
  return it == lkh::table().end() ? nullptr : reinterpret_cast<const lk_kernel*>(&it->second);
}

int lk_kernel_is_gpu(const lk_kernel* k) {
  return k ? (reinterpret_cast<const lkh::KernelEntry*>(k)->device == lkh::Device::Gpu ? 1 : 0) : -1;
}

int lk_kernel_arity(const lk_kernel* k, int* numOperands, int* numOuts) {
  if (!k) return 1;
  const auto* e = reinterpret_cast<const lkh::KernelEntry*>(k);
  if (numOperands) *numOperands = e->numOperands;
  if (numOuts) *numOuts = e->numOuts;
  return 0;
}

int lk_run_kernel(const lk_kernel* k, void* const* ptrs, uint32_t numPtrs, const int64_t* ints, uint32_t numInts,
                  const double* floats, uint32_t numFloats, void* workspace, uint64_t workspaceBytes, void* stream) {
  if (!k) {
    lkh::tlsError = "lk_run_kernel: null kernel";
    return 1;
  }
  const auto* e = reinterpret_cast<const lkh::KernelEntry*>(k);
  if (e->numOperands >= 0 && numPtrs != static_cast<uint32_t>(e->numOperands + e->numOuts)) {
    lkh::tlsError = std::string(e->name) + ": wrong number of operands";
    return 1;
  }
  // Runners index ints / floats by position. A caller's short arrays are copied into zero-padded ones, so a
  // missing dim or attribute reads as 0 (which every runner's shape checks reject) instead of past the array.
  constexpr uint32_t kMaxInts = 256, kMaxFloats = 32;
  if (numInts > kMaxInts || numFloats > kMaxFloats || (numInts && !ints) || (numFloats && !floats)) {
    lkh::tlsError = std::string(e->name) + ": too many (or missing) int / float arguments";
    return 1;
  }
  int64_t iv[kMaxInts] = {};
  double fv[kMaxFloats] = {};
  if (numInts) std::memcpy(iv, ints, numInts * sizeof(int64_t));
  if (numFloats) std::memcpy(fv, floats, numFloats * sizeof(double));
  lkh::KernelArgs args{ptrs, nullptr, iv, fv, nullptr, numPtrs, numInts, numFloats};
  lkh::ExecCtx ctx;
  ctx.stream = static_cast<hipStream_t>(stream);
  ctx.workspace = workspace;
  ctx.workspaceBytes = workspaceBytes;
  e->run(ctx, args);
  if (ctx.error) {
    lkh::tlsError = std::string(e->name) + ": " + ctx.error;
    return 1;
  }
  return 0;
}

const char* lk_last_error(void) { return lkh::tlsError.c_str(); }

}  // extern "C"
