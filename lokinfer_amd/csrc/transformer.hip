// Token-rate transformer kernels, row-major [T, D] (ALBERT in Kokoro, GPT-2 decode).
//
//   lk_hip_layernorm_f32         LN rows (reference layernorm_f32_gpu, kokoro_tok.metal:169-204)
//   lk_hip_add_bias_ln_f32       LN(a + bias + r) [+ the sum]  (add_bias_layernorm[2]_f32_gpu, kokoro_tok.metal:36-117)
//   lk_hip_bias_gelu_f32         gelu_tanh(x + bias)            (bias_gelu_f32_gpu, kokoro_tok.metal:25-34)
//   lk_hip_attention_qkv_f32     SDPA over a fused QKV [T, 3D]  (attention_qkv[_sg][_causal]_f32_gpu,
//                                transformer_gpu.cpp:72-86, kokoro_tok.metal:465-601)
//   lk_hip_kv_write_f32          k, v (+ bias) into row pos of the caches (kv_write_f32_gpu, kokoro_lc.cpp:826-872)
//   lk_hip_kv_write_rows_f32     the same for the T rows of a chunk at pos..pos+T-1 (kv_write_rows_f32_gpu,
//                                python/lokinfer/ops/transformer.py:239-242)
//   lk_hip_attention_cache_f32   causal SDPA of a chunk's T queries over cache rows 0..pos+i (attention_cache[_sg]_f32_gpu,
//                                python/lokinfer/ops/transformer.py:255-268, 348-351)
//   lk_hip_add_bias_ln_sk_f32    LN(sum of split-K partials + bias + r) and the sum (add_bias_layernorm2_sk_f32_gpu,
//                                python/lokinfer/ops/transformer.py:458-472)
//
// Rows are reduced by a whole workgroup with wave64 shuffles; statistics use the reference's two-pass form
// (mean, then the centred sum of squares) with the biased variance.
#include <algorithm>

#include "common.h"
#include "lokinfer_hip.h"

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

// mode 0: out = LN(x); mode 1: out = LN(a + bias + r); mode 2: sum = a + bias + r, out = LN(sum). With parts > 1,
// a is the sum of `parts` planes of partStride floats (split-K partials).
__global__ __launch_bounds__(kLnThreads) void lnRowsKernel(const float* a, const float* bias, const float* r,
                                                         const float* gamma, const float* beta, float* sumOut,
                                                         float* out, int64_t cols, float eps, int mode, int parts,
                                                         int64_t partStride) {
  __shared__ float scratch[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
  float v[kLnMaxPerThread];
  float s = 0.0f;
  int n = 0;
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads, ++n) {
    float x = a[base + c];
    for (int q = 1; q < parts; ++q) x += a[q * partStride + base + c];  // split-K partials, summed in order
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

// Flash attention on f32 MFMA (32x32x2) over a fused QKV projection, head_dim 64, in the transposed form: a wave
// computes S^T = K Q^T for 32 queries x 32 keys, so each lane's accumulator column is ONE query (16 of its 32 keys
// in this lane, the other 16 in lane ^ 32):
//   * the online-softmax max / sum of a query is 15 in-lane operations and one shuffle;
//   * P^T sits in registers exactly as the B operand of O^T = V^T P^T: MFMA step s, lane half h reads key
//     8 (s / 4) + 4 h + s % 4, which is accumulator register s of that lane; P never goes through LDS.
// The 64 dims are consumed in the order 32 h + s (lane half h, step s), so a lane's share of a Q or K row is 32
// contiguous floats (eight 16-byte loads, straight into registers, no LDS); V^T is read as 32-float rows per
// key. Q is pre-scaled by log2(e) / 8 (+ q-bias) so that softmax uses exp2. The k-bias cancels in softmax and is
// dropped; the v-bias is added once at the end (softmax weights sum to 1), as in the reference kernel.
// A workgroup = NW waves = one head's 32-query block; wave w takes key tiles w, w + NW, ... (prefetched one tile
// ahead into registers) and the NW partial (max, sum, O) states merge through LDS at the end. Grid =
// ceil(T / 32) x heads. NW = 8: a block holds few key tiles (16 at 512 tokens), so more waves per block keep more
// tiles in flight (GPT-2 512-token prefill 1.609 -> 1.586 ms against 4).
// CACHE: the chunk form. Query i of qkv sits at position pos + i (pos read from the device) and attends causally to
// rows 0..pos+i of the K / V caches [cap, D] (row stride D), which already hold the chunk's rows with their biases
// (so no v-bias is added at the end). Key tiles start at row 0, not at the query block, so a wave can own a tile
// that lies wholly past some of its queries; its max stays -inf there and the exp2 reference is taken as 0. Keys
// stop at cap; a query at position >= cap has no cache row and gets NaN.
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

template <bool CACHE, int NW = 4>
__global__ __launch_bounds__(64 * NW) void attnMfmaKernel(const float* __restrict__ qkv, const float* __restrict__ bias,
                                                      const float* __restrict__ kc, const float* __restrict__ vc,
                                                      const int64_t* __restrict__ pos, int64_t cap,
                                                      float* __restrict__ out, int64_t t, int heads, int causal,
                                                      unsigned long long* err) {
  constexpr int HD = 64, KT = 32;
  __shared__ float mS[NW][32], lS[NW][32];
  __shared__ float oS[NW][32][HD + 1];
  const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t D = static_cast<int64_t>(heads) * HD, ld = 3 * D;
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t qi = q0 + lr;  // this lane's query (accumulator column)
  // chunk start, key count, key row stride and bases
  const int64_t p0 = CACHE ? *pos : 0;
  const int64_t nk = CACHE ? (p0 < 0 ? 0 : min<int64_t>(p0 + t, cap)) : t;
  const int64_t kld = CACHE ? D : ld;
  const float* kbase = CACHE ? kc : qkv + D;
  const float* vbase = CACHE ? vc : qkv + 2 * D;
  const int64_t qpos = p0 + qi;  // this lane's query position
  // B operand of S^T: Q[q][32 lh + s] * log2(e) / 8
  float qb[32];
  {
    const float* qr = qkv + min<int64_t>(qi, t - 1) * ld + h * HD + 32 * lh;
    const float* br = bias + h * HD + 32 * lh;
    constexpr float kScale = 0.125f * 1.44269504088896341f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const v4f_t x = *reinterpret_cast<const v4f_t*>(qr + 4 * v), bb = *reinterpret_cast<const v4f_t*>(br + 4 * v);
#pragma unroll
      for (int c = 0; c < 4; ++c) qb[4 * v + c] = (x[c] + bb[c]) * kScale;
    }
  }
  const int64_t kEnd = causal ? min<int64_t>(nk, p0 + q0 + 32) : nk;
  const int tiles = kEnd > 0 ? static_cast<int>((kEnd + KT - 1) / KT) : 0;
  // A operands of one key tile: K[k0 + lr][32 lh + s] (32 floats) and V[k0 + key(s, lh)][32 b + lr] (2 x 16)
  v4f_t kr[8];
  float vr[32];
  auto loadTile = [&](int tile) {
    const int64_t k0 = static_cast<int64_t>(tile) * KT;
    const float* kp = kbase + min<int64_t>(k0 + lr, nk - 1) * kld + h * HD + 32 * lh;
#pragma unroll
    for (int v = 0; v < 8; ++v) kr[v] = *reinterpret_cast<const v4f_t*>(kp + 4 * v);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int64_t key = min<int64_t>(k0 + 8 * (s >> 2) + 4 * lh + (s & 3), nk - 1);
      const float* vp = vbase + key * kld + h * HD + lr;
      vr[s] = vp[0];
      vr[16 + s] = vp[32];
    }
  };
  v16f_t o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  if (wave < tiles) loadTile(wave);
  for (int tile = wave; tile < tiles; tile += NW) {
    const int64_t k0 = static_cast<int64_t>(tile) * KT;
    float ka[32], va[32];
#pragma unroll
    for (int v = 0; v < 8; ++v)
#pragma unroll
      for (int c = 0; c < 4; ++c) ka[4 * v + c] = kr[v][c];
#pragma unroll
    for (int s = 0; s < 32; ++s) va[s] = vr[s];
    if (tile + NW < tiles) loadTile(tile + NW);
    v16f_t sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; ++s) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[s], qb[s], sacc, 0, 0, 0);
    // accumulator r: key k0 + 8 (r / 4) + 4 lh + r % 4, query qi
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
      if (key >= nk || (causal && key > qpos)) sacc[r] = -INFINITY;
      mt = fmaxf(mt, sacc[r]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mx = fmaxf(m, mt);  // without CACHE finite: every tile holds a key <= qi (causal) or < t
    const float mn = CACHE && mx == -INFINITY ? 0.0f : mx;
    const float corr = __builtin_amdgcn_exp2f(m - mn);
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = __builtin_amdgcn_exp2f(sacc[r] - mn);
      ls += sacc[r];
    }
    ls += __shfl_xor(ls, 32, 64);
    l = l * corr + ls;
    m = mx;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o0[r] *= corr;
      o1[r] *= corr;
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(va[s], sacc[s], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(va[16 + s], sacc[s], o1, 0, 0, 0);
    }
  }
  // merge the four waves: O^T accumulator r of block b is dim 32 b + 8 (r / 4) + 4 lh + r % 4 of query lr
  if (lh == 0) {
    mS[wave][lr] = m;
    lS[wave][lr] = l;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = 8 * (r >> 2) + 4 * lh + (r & 3);
    oS[wave][lr][d] = o0[r];
    oS[wave][lr][32 + d] = o1[r];
  }
  __syncthreads();
  constexpr int TPQ = 2 * NW, DPT = HD / TPQ;  // threads per query, dims per thread
  const int q = tid / TPQ, d0 = (tid % TPQ) * DPT;
  const int64_t qrow = q0 + q;
  if (qrow >= t) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) mx = fmaxf(mx, mS[w][q]);
  float wsum = 0.0f, sc[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    sc[w] = lS[w][q] > 0.0f ? __builtin_amdgcn_exp2f(mS[w][q] - mx) : 0.0f;
    wsum += sc[w] * lS[w][q];
  }
  const float inv = 1.0f / wsum;
  float* o = out + qrow * D + h * HD;
  const float* bv = bias + 2 * D + h * HD;
  const bool noRow = CACHE && p0 + qrow >= cap;
#pragma unroll
  for (int d = d0; d < d0 + DPT; ++d) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) acc += sc[w] * oS[w][q][d];
    o[d] = noRow ? __builtin_nanf("") : CACHE ? acc * inv : acc * inv + bv[d];
  }
  // recorded once, by the thread of head 0 that owns the first query without a cache row
  if (noRow && d0 == 0 && h == 0 && qrow == (p0 < 0 ? 0 : cap - p0)) raiseDeviceError(err, LK_DEVERR_POSITION, p0 + qrow);
}

// a position outside [0, cap) writes nothing and is recorded in the GPU's error record
__global__ void kvWriteKernel(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias,
                              int64_t d, int64_t cap, unsigned long long* err) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= d) return;
  const int64_t p = *pos;
  if (p < 0 || p >= cap) {
    if (i == 0) raiseDeviceError(err, LK_DEVERR_POSITION, p);
    return;
  }
  kc[p * d + i] = qkv[d + i] + bias[d + i];
  vc[p * d + i] = qkv[2 * d + i] + bias[2 * d + i];
}

// rows pos..pos+T-1 of the caches = k / v of qkv [T, 3D] + bias, float4 per thread; rows outside the cache are
// dropped and recorded in the GPU's error record
__global__ void kvWriteRowsKernel(float* __restrict__ kc, float* __restrict__ vc, const float* __restrict__ qkv,
                                  const int64_t* __restrict__ pos, const float* __restrict__ bias, int64_t t,
                                  int64_t d, int64_t cap, unsigned long long* err) {
  const int64_t p0 = *pos, d4 = d / 4, total = t * d4;
  if ((p0 < 0 || p0 + t > cap) && blockIdx.x == 0 && threadIdx.x == 0)
    raiseDeviceError(err, LK_DEVERR_POSITION, p0 < 0 ? p0 : p0 + t - 1);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d4, c = (i - r * d4) * 4, row = p0 + r;
    if (row < 0 || row >= cap) continue;
    const float* q = qkv + r * 3 * d;
    const v4f_t k = *reinterpret_cast<const v4f_t*>(q + d + c) + *reinterpret_cast<const v4f_t*>(bias + d + c);
    const v4f_t v = *reinterpret_cast<const v4f_t*>(q + 2 * d + c) + *reinterpret_cast<const v4f_t*>(bias + 2 * d + c);
    *reinterpret_cast<v4f_t*>(kc + row * d + c) = k;
    *reinterpret_cast<v4f_t*>(vc + row * d + c) = v;
  }
}

}  // namespace lkd

extern "C" {

// mode 0: out = LN(a); 1: out = LN(a + bias + r); 2: also writes sum = a + bias + r. cols <= 2048.
int lk_hip_layernorm_f32(const float* a, const float* bias, const float* r, const float* gamma, const float* beta,
                         float* sum, float* out, int64_t rows, int64_t cols, float eps, int mode, void* stream) {
  if (cols > lkd::kLnThreads * lkd::kLnMaxPerThread || cols <= 0) return 1;
  if (rows <= 0) return rows == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::lnRowsKernel, dim3(static_cast<unsigned>(rows)), dim3(lkd::kLnThreads), 0,
                     static_cast<hipStream_t>(stream), a, bias, r, gamma, beta, sum, out, cols, eps, mode, 1,
                     int64_t{0});
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// sum = parts[0] + ... + parts[S-1] + bias + r, out = LN(sum); parts [S, rows, cols], cols <= 2048.
int lk_hip_add_bias_ln_sk_f32(const float* parts, int64_t splits, const float* bias, const float* r,
                              const float* gamma, const float* beta, float* sum, float* out, int64_t rows,
                              int64_t cols, float eps, void* stream) {
  if (cols > lkd::kLnThreads * lkd::kLnMaxPerThread || cols <= 0 || splits < 1 || splits > (1 << 20)) return 1;
  if (rows <= 0) return rows == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::lnRowsKernel, dim3(static_cast<unsigned>(rows)), dim3(lkd::kLnThreads), 0,
                     static_cast<hipStream_t>(stream), parts, bias, r, gamma, beta, sum, out, cols, eps, 2,
                     static_cast<int>(splits), rows * cols);
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
  dim3 grid(lkh::ceilDiv(t, 32), static_cast<unsigned>(heads));
  hipLaunchKernelGGL((lkd::attnMfmaKernel<false, 8>), grid, dim3(512), 0, static_cast<hipStream_t>(stream), qkv,
                     bias, nullptr, nullptr, nullptr, int64_t{0}, out, t, heads, causal, nullptr);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_attention_cache_f32(const float* qkv, const float* kc, const float* vc, const int64_t* pos,
                               const float* bias, float* out, int64_t t, int heads, int64_t cap, void* stream) {
  if (t <= 0 || heads <= 0 || cap <= 0) return t == 0 ? 0 : 1;
  dim3 grid(lkh::ceilDiv(t, 32), static_cast<unsigned>(heads));
  hipLaunchKernelGGL((lkd::attnMfmaKernel<true, 8>), grid, dim3(512), 0, static_cast<hipStream_t>(stream), qkv, bias,
                     kc, vc, pos, cap, out, t, heads, 1, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_kv_write_rows_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias,
                             int64_t t, int64_t d, int64_t cap, void* stream) {
  const int64_t total = t * d;
  if (t <= 0 || d <= 0 || d % 4 != 0) return t == 0 ? 0 : 1;
  if (((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc) | reinterpret_cast<uintptr_t>(qkv) |
        reinterpret_cast<uintptr_t>(bias)) & 15) != 0)
    return 1;
  const int64_t blocks = std::min<int64_t>((total / 4 + 255) / 256, 4096);
  hipLaunchKernelGGL(lkd::kvWriteRowsKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), kc, vc, qkv, pos, bias, t, d, cap, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_kv_write_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias, int64_t d,
                        int64_t cap, void* stream) {
  if (d <= 0 || cap <= 0) return 1;
  hipLaunchKernelGGL(lkd::kvWriteKernel, dim3(lkh::ceilDiv(d, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), kc, vc, qkv, pos, bias, d, cap, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
