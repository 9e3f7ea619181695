// Token-rate transformer kernels, row-major [T, D] (ALBERT in Kokoro, GPT-2 decode).
//
//   lk_hip_layernorm_f32         LN rows (reference layernorm_f32_gpu, kokoro_tok.metal:169-204)
//   lk_hip_add_bias_ln_f32       LN(a + bias + r) [+ the sum]  (add_bias_layernorm[2]_f32_gpu, kokoro_tok.metal:36-117)
//   lk_hip_bias_gelu_f32         gelu_tanh(x + bias)            (bias_gelu_f32_gpu, kokoro_tok.metal:25-34)
//   lk_hip_attention_qkv_f32     SDPA over a fused QKV [T, 3D]  (attention_qkv[_sg][_causal]_f32_gpu,
//                                transformer_gpu.cpp:72-86, kokoro_tok.metal:465-601)
//   lk_hip_kv_write_f32          k, v (+ bias) into row pos of the caches (kv_write_f32_gpu, kokoro_lc.cpp:826-872)
//
// Rows are reduced by a whole workgroup with wave64 shuffles; statistics use the reference's two-pass form
// (mean, then the centred sum of squares) with the biased variance.
#include "common.h"

namespace lkd {

constexpr int kLnThreads = 256;
constexpr int kLnMaxPerThread = 8;  // C <= 2048

__device__ __forceinline__ float blockSum256(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = waveSum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// mode 0: out = LN(x); mode 1: out = LN(a + bias + r); mode 2: sum = a + bias + r, out = LN(sum).
__global__ __launch_bounds__(kLnThreads) void lnRowsKernel(const float* a, const float* bias, const float* r,
                                                         const float* gamma, const float* beta, float* sumOut,
                                                         float* out, int64_t cols, float eps, int mode) {
  __shared__ float scratch[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
  float v[kLnMaxPerThread];
  float s = 0.0f;
  int n = 0;
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads, ++n) {
    float x = a[base + c];
    if (mode != 0) x = x + bias[c] + r[base + c];
    v[n] = x;
    s += x;
  }
  const float mean = blockSum256(s, scratch) / static_cast<float>(cols);
  float q = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  const float var = blockSum256(q, scratch) / static_cast<float>(cols);
  const float rstd = 1.0f / sqrtf(var + eps);
  n = 0;
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads, ++n) {
    if (mode == 2) sumOut[base + c] = v[n];
    out[base + c] = (v[n] - mean) * rstd * gamma[c] + beta[c];
  }
}

__global__ void biasGeluKernel(const float* x, const float* bias, float* out, int64_t n, int64_t cols) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = geluTanh(x[i] + bias[i % cols]);
}

// Flash attention over a fused QKV projection, head_dim 64. One wave per (head, 64-query tile), one query per
// lane: q (+ q-bias, * 1/8) in registers, 64-key K/V tiles staged in LDS, online softmax in base e. The k-bias
// cancels in softmax and is dropped; the v-bias is added once at the end (softmax weights sum to 1), as in the
// reference kernel.
__global__ __launch_bounds__(64) void attnQkvKernel(const float* __restrict__ qkv, const float* __restrict__ bias,
                                                    float* __restrict__ out, int64_t t, int heads, int causal) {
  constexpr int HD = 64, KT = 64;
  __shared__ float ks[KT][HD + 1];
  __shared__ float vs[KT][HD];
  const int h = blockIdx.y, lane = threadIdx.x;
  const int64_t D = static_cast<int64_t>(heads) * HD, ld = 3 * D;
  const int64_t qi = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool active = qi < t;
  float q[HD], acc[HD];
  const float* qr = qkv + (active ? qi : 0) * ld + h * HD;
#pragma unroll
  for (int d = 0; d < HD; ++d) {
    q[d] = (qr[d] + bias[h * HD + d]) * 0.125f;
    acc[d] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const int64_t kEnd = causal ? min<int64_t>(t, static_cast<int64_t>(blockIdx.x) * 64 + 64) : t;
  for (int64_t k0 = 0; k0 < kEnd; k0 += KT) {
    __syncthreads();
    for (int i = lane; i < KT * HD; i += 64) {
      const int kr = i / HD, d = i % HD;
      const int64_t j = k0 + kr;
      ks[kr][d] = j < t ? qkv[j * ld + D + h * HD + d] : 0.0f;
      vs[kr][d] = j < t ? qkv[j * ld + 2 * D + h * HD + d] : 0.0f;
    }
    __syncthreads();
    const int nk = static_cast<int>(min<int64_t>(KT, kEnd - k0));
    for (int j = 0; j < nk; ++j) {
      if (causal && k0 + j > qi) break;
      float sc = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; ++d) sc += q[d] * ks[j][d];
      const float mn = fmaxf(m, sc);
      const float corr = expf(m - mn), p = expf(sc - mn);
      l = l * corr + p;
#pragma unroll
      for (int d = 0; d < HD; ++d) acc[d] = acc[d] * corr + p * vs[j][d];
      m = mn;
    }
  }
  if (!active) return;
  const float inv = 1.0f / l;
  float* o = out + qi * D + h * HD;
#pragma unroll
  for (int d = 0; d < HD; ++d) o[d] = acc[d] * inv + bias[2 * D + h * HD + d];
}

// Flash attention on f32 MFMA (32x32x2), head_dim 64. A workgroup = 4 waves = 128 queries of one head; each wave
// owns 32 queries and walks the keys in 32-key tiles shared through LDS:
//   S = Q K^T   32 MFMAs over the 64 dims (Q pre-scaled by 1/8 and + q-bias, held in 32 registers per lane)
//   online softmax per query row on the accumulator layout (a row's 32 keys sit in 32 lanes of one half-wave)
//   O += P V    P goes through LDS to the A-operand layout; 2 x 16 MFMAs for the 64 output dims
// The k-bias cancels in softmax and is dropped; the v-bias is added once at the end.
typedef float v16f_t __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void attnMfmaKernel(const float* __restrict__ qkv, const float* __restrict__ bias,
                                                      float* __restrict__ out, int64_t t, int heads, int causal) {
  constexpr int HD = 64, KT = 32, LDK = HD + 1, LDV = HD + 4, LDP = KT + 1;
  __shared__ float ks[KT][LDK];
  __shared__ float vs[KT][LDV];
  __shared__ float ps[4][32][LDP];
  const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t D = static_cast<int64_t>(heads) * HD, ld = 3 * D;
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * 128 + wave * 32;
  const int lr = lane & 31, lh = lane >> 5;
  // Q operand: lane holds Q[q0 + lr][2 s + lh] for s = 0..31
  float qa[32];
  {
    const int64_t qi = min<int64_t>(q0 + lr, t - 1);
    const float* qr = qkv + qi * ld + h * HD;
#pragma unroll
    for (int s = 0; s < 32; ++s) qa[s] = (qr[2 * s + lh] + bias[h * HD + 2 * s + lh]) * 0.125f;
  }
  v16f_t o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;
  float mrow[16], lrow[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    mrow[r] = -INFINITY;
    lrow[r] = 0.0f;
  }
  const int64_t blockQmax = min<int64_t>(t, static_cast<int64_t>(blockIdx.x) * 128 + 128);
  const int64_t kEnd = causal ? blockQmax : t;
  for (int64_t k0 = 0; k0 < kEnd; k0 += KT) {
    __syncthreads();
    for (int i = tid; i < KT * HD; i += 256) {
      const int kr = i / HD, d = i % HD;
      const int64_t j = k0 + kr;
      ks[kr][d] = j < t ? qkv[j * ld + D + h * HD + d] : 0.0f;
      vs[kr][d] = j < t ? qkv[j * ld + 2 * D + h * HD + d] : 0.0f;
    }
    __syncthreads();
    // S tile: rows = queries, cols = keys
    v16f_t sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; ++s) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[s], ks[lr][2 * s + lh], sacc, 0, 0, 0);
    // online softmax: register r holds row 8 (r / 4) + 4 lh + r % 4, column (key) lr
    const int64_t key = k0 + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t qrow = q0 + 8 * (r >> 2) + 4 * lh + (r & 3);
      float sv = sacc[r];
      if (key >= t || (causal && key > qrow)) sv = -INFINITY;
      float mx = sv;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      const float mn = fmaxf(mrow[r], mx);
      const float p = mn == -INFINITY ? 0.0f : expf(sv - mn);
      const float corr = mn == -INFINITY ? 1.0f : expf(mrow[r] - mn);
      float ps_ = p;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) ps_ += __shfl_xor(ps_, o, 64);
      lrow[r] = lrow[r] * corr + ps_;
      mrow[r] = mn;
      o0[r] *= corr;
      o1[r] *= corr;
      ps[wave][8 * (r >> 2) + 4 * lh + (r & 3)][lr] = p;
    }
    __syncthreads();
    // O += P V: A = P[q = lr][key = 2 s + lh], B = V[key][dim]
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const float pa = ps[wave][lr][2 * s + lh];
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa, vs[2 * s + lh][lr], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa, vs[2 * s + lh][32 + lr], o1, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t qrow = q0 + 8 * (r >> 2) + 4 * lh + (r & 3);
    if (qrow < t) {
      const float inv = 1.0f / lrow[r];
      float* o = out + qrow * D + h * HD;
      o[lr] = o0[r] * inv + bias[2 * D + h * HD + lr];
      o[32 + lr] = o1[r] * inv + bias[2 * D + h * HD + 32 + lr];
    }
  }
}

__global__ void kvWriteKernel(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias,
                              int64_t d) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= d) return;
  const int64_t p = *pos;
  kc[p * d + i] = qkv[d + i] + bias[d + i];
  vc[p * d + i] = qkv[2 * d + i] + bias[2 * d + i];
}

}  // namespace lkd

extern "C" {

// mode 0: out = LN(a); 1: out = LN(a + bias + r); 2: also writes sum = a + bias + r. cols <= 2048.
int lk_hip_layernorm_f32(const float* a, const float* bias, const float* r, const float* gamma, const float* beta,
                         float* sum, float* out, int64_t rows, int64_t cols, float eps, int mode, void* stream) {
  if (cols > lkd::kLnThreads * lkd::kLnMaxPerThread || cols <= 0) return 1;
  if (rows <= 0) return rows == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::lnRowsKernel, dim3(static_cast<unsigned>(rows)), dim3(lkd::kLnThreads), 0,
                     static_cast<hipStream_t>(stream), a, bias, r, gamma, beta, sum, out, cols, eps, mode);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_bias_gelu_f32(const float* x, const float* bias, float* out, int64_t rows, int64_t cols, void* stream) {
  const int64_t n = rows * cols;
  if (n <= 0) return n == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::biasGeluKernel, dim3(lkh::ceilDiv(n, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, bias, out, n, cols);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_attention_qkv_f32(const float* qkv, const float* bias, float* out, int64_t t, int heads, int causal,
                             void* stream) {
  if (t <= 0) return t == 0 ? 0 : 1;
  dim3 grid(lkh::ceilDiv(t, 128), static_cast<unsigned>(heads));
  hipLaunchKernelGGL(lkd::attnMfmaKernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), qkv, bias, out, t,
                     heads, causal);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_kv_write_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias, int64_t d,
                        void* stream) {
  hipLaunchKernelGGL(lkd::kvWriteKernel, dim3(lkh::ceilDiv(d, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), kc, vc, qkv, pos, bias, d);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
