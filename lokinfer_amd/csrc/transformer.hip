// Token-rate transformer kernels, row-major [T, D] (ALBERT in Kokoro, GPT-2 decode).
//
//   lk_hip_layernorm_f32         LN rows (reference layernorm_f32_gpu, kokoro_tok.metal:169-204)
//   lk_hip_add_bias_ln_f32       LN(a + bias + r) [+ the sum]  (add_bias_layernorm[2]_f32_gpu, kokoro_tok.metal:36-117)
//   lk_hip_bias_gelu_f32         gelu_tanh(x + bias)            (bias_gelu_f32_gpu, kokoro_tok.metal:25-34)
//   lk_hip_attention_qkv_f32     SDPA over a fused QKV [T, 3D]  (attention_qkv[_sg][_causal]_f32_gpu,
//                                transformer_gpu.cpp:72-86, kokoro_tok.metal:465-601)
//   lk_hip_attention_decode_f32  fused KV write + one-query attention over rows 0..pos, split over keys with an
//                                in-kernel combine (attention_decode_split_f32_gpu, transformer_gpu.cpp:122-222,
//                                kokoro_tok.metal:637-876)
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

// Decode attention, one wave per (head, key split): lane j scores key kb + j against q (q = (q + bq) / 8),
// then p = exp(s - m_split), acc[d] = sum p v[d] with lane = d. Row `pos` comes from qkv + bias (and the block
// owning it writes it to both caches). Partials (m, l, acc[64]) go to the workspace; the last split of a head
// (atomic ticket) merges them in split order.
struct DecodeParams {
  const float* qkv;
  float* kc;
  float* vc;
  const int64_t* pos;
  const float* bias;
  float* out;
  float* partial;     // [heads, splits, 66]
  unsigned* tickets;  // [heads]
  int64_t cap;
  int heads;
  int keysPerSplit;
  int splits;
  int writeKv;
};

__global__ __launch_bounds__(64) void decodeAttnKernel(DecodeParams p) {
  constexpr int HD = 64;
  __shared__ bool last;
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int64_t D = static_cast<int64_t>(p.heads) * HD;
  const int64_t pos = *p.pos;
  if (pos < 0 || pos >= p.cap) {  // out-of-range position: no cache write, NaN output (every block exits here)
    if (s == 0) p.out[h * HD + lane] = __builtin_nanf("");
    return;
  }
  const int64_t kb = static_cast<int64_t>(s) * p.keysPerSplit;
  const int64_t ke = min<int64_t>(pos + 1, kb + p.keysPerSplit);
  const float* qrow = p.qkv + h * HD;
  // New key / value row (bias added), lane = dim.
  const float knew = p.qkv[D + h * HD + lane] + p.bias[D + h * HD + lane];
  const float vnew = p.qkv[2 * D + h * HD + lane] + p.bias[2 * D + h * HD + lane];
  if (p.writeKv && pos >= kb && pos < kb + p.keysPerSplit) {
    p.kc[pos * D + h * HD + lane] = knew;
    p.vc[pos * D + h * HD + lane] = vnew;
  }
  float q[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) q[d] = (qrow[d] + p.bias[h * HD + d]) * 0.125f;
  // Score of the new key (row pos), computed by the whole wave: lane d holds q[d] and k_new[d].
  const float snew = waveSum((qrow[lane] + p.bias[h * HD + lane]) * 0.125f * knew);
  float m = -INFINITY, l = 0.0f, acc = 0.0f;
  for (int64_t c0 = kb; c0 < ke; c0 += 64) {
    const int64_t j = c0 + lane;
    float sc = -INFINITY;
    if (j < ke) {
      float dot = snew;
      if (j != pos) {
        dot = 0.0f;
        const float4* kr = reinterpret_cast<const float4*>(p.kc + j * D + h * HD);
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; ++d4) {
          const float4 kv = kr[d4];
          dot += q[4 * d4] * kv.x + q[4 * d4 + 1] * kv.y + q[4 * d4 + 2] * kv.z + q[4 * d4 + 3] * kv.w;
        }
      }
      sc = dot;
    }
    const float cm = waveMax(sc);
    const float mn = fmaxf(m, cm);
    const float pj = j < ke ? expf(sc - mn) : 0.0f;
    const float corr = expf(m - mn);
    l = l * corr + waveSum(pj);
    acc *= corr;
    const int nk = static_cast<int>(min<int64_t>(64, ke - c0));
    for (int jj = 0; jj < nk; ++jj) {
      const float pw = __shfl(pj, jj, 64);
      const int64_t row = c0 + jj;
      const float vv = row == pos ? vnew : p.vc[row * D + h * HD + lane];
      acc += pw * vv;
    }
    m = mn;
  }
  if (p.splits == 1) {
    p.out[h * HD + lane] = acc / l;
    return;
  }
  float* part = p.partial + (static_cast<int64_t>(h) * p.splits + s) * (HD + 2);
  part[2 + lane] = acc;
  if (lane == 0) {
    part[0] = m;
    part[1] = l;
  }
  __threadfence();
  __syncthreads();
  if (lane == 0) last = atomicAdd(&p.tickets[h], 1u) == static_cast<unsigned>(p.splits - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  float M = -INFINITY;
  for (int i = 0; i < p.splits; ++i) {
    const float* pi = p.partial + (static_cast<int64_t>(h) * p.splits + i) * (HD + 2);
    M = fmaxf(M, __hip_atomic_load(pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
  float L = 0.0f, A = 0.0f;
  for (int i = 0; i < p.splits; ++i) {
    const float* pi = p.partial + (static_cast<int64_t>(h) * p.splits + i) * (HD + 2);
    const float mi = __hip_atomic_load(pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float li = __hip_atomic_load(pi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float ai = __hip_atomic_load(pi + 2 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float w = li > 0.0f ? expf(mi - M) : 0.0f;
    L += li * w;
    A += ai * w;
  }
  p.out[h * HD + lane] = A / L;
  if (lane == 0) p.tickets[h] = 0u;
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
  dim3 grid(lkh::ceilDiv(t, 64), static_cast<unsigned>(heads));
  hipLaunchKernelGGL(lkd::attnQkvKernel, grid, dim3(64), 0, static_cast<hipStream_t>(stream), qkv, bias, out, t,
                     heads, causal);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int64_t lk_hip_attention_decode_workspace_bytes(int heads, int64_t cap) {
  const int64_t splits = (cap + 31) / 32;
  return 65536 + static_cast<int64_t>(heads) * splits * 66 * 4;
}

// qkv [1, 3D] (before bias), kc / vc [cap, D] (rows 0..pos-1 valid; row pos written when writeKv), pos device
// i64[1], bias [3D] -> out [1, D]. keysPerSplit 0 = auto. The caller guarantees pos < cap (checked on the host
// by the registry entry, which reads nothing from the device; the kernel clamps nothing).
int lk_hip_attention_decode_f32(const float* qkv, float* kc, float* vc, const int64_t* pos, const float* bias,
                                float* out, int64_t cap, int heads, int64_t maxKeys, int keysPerSplit, int writeKv,
                                void* workspace, int64_t workspaceBytes, void* stream) {
  if (keysPerSplit <= 0) keysPerSplit = 32;
  lkd::DecodeParams p{};
  p.qkv = qkv;
  p.kc = kc;
  p.vc = vc;
  p.pos = pos;
  p.bias = bias;
  p.out = out;
  p.cap = cap;
  p.heads = heads;
  p.keysPerSplit = keysPerSplit;
  p.writeKv = writeKv;
  // maxKeys bounds pos + 1 for the grid; splits beyond the live keys exit after contributing l = 0.
  int64_t splits = (maxKeys + keysPerSplit - 1) / keysPerSplit;
  if (splits < 1) splits = 1;
  if (splits > 1) {
    const int64_t need = 65536 + static_cast<int64_t>(heads) * splits * 66 * 4;
    if (!workspace || workspaceBytes < need) return 3;
  }
  p.splits = static_cast<int>(splits);
  p.tickets = static_cast<unsigned*>(workspace);
  p.partial = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + 65536) : nullptr;
  dim3 grid(static_cast<unsigned>(heads), static_cast<unsigned>(splits));
  hipLaunchKernelGGL(lkd::decodeAttnKernel, grid, dim3(64), 0, static_cast<hipStream_t>(stream), p);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_kv_write_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias, int64_t d,
                        void* stream) {
  hipLaunchKernelGGL(lkd::kvWriteKernel, dim3(lkh::ceilDiv(d, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), kc, vc, qkv, pos, bias, d);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
