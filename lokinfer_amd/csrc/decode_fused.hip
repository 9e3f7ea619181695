// Fused decode-step kernels (batch-1 transformer decode, e.g. GPT-2 124M): the GEMV split in two launches
// (partial sums, then a reduction) is kept, but each reduction is folded into the kernel that consumes it, so a
// layer is 5 launches instead of 13. At decode sizes every launch costs a few microseconds whatever it does, so
// the step time follows the launch count.
//
//   lk_hip_gemv_partial_f32    part[S, N] of x[1, K] . W[K, N], S = ceil(K / (4 rpw)) row slices; the input x is
//                              (mode 0) a vector, (mode 1) gelu(sum of a previous partial + bias), (mode 2)
//                              the merge of decode-attention chunk partials (one head per 64 rows), or (mode 3)
//                              LayerNorm(sum of a previous partial + bias + residual), the sum also written out
//   lk_hip_attention_decode_part_f32
//                              decode attention whose q, k, v come as GEMV partials (+ bias): writes row pos of
//                              both caches and the per-(head, 64-key chunk) partials (m, l, acc[64])
//   lk_hip_reduce_ln_f32       sum = sum_s part[s] + bias + res; ln = LayerNorm(sum) (one workgroup)
//
// They replace the reference's gemv4*_f32_gpu / attention_decode_split_f32_gpu / add_bias_layernorm2_f32_gpu
// sequence (transformer_gpu.cpp:122-251, kokoro_tok.metal:36-117, 637-924 in lariaus/lokinfer) for one layer,
// with the same arithmetic per element: the sums over K are split into row slices and added in a fixed order
// (deterministic), softmax is base e on q / 8, LayerNorm is two-pass with the biased variance.
#include "common.h"
#include "lokinfer_hip.h"

#include <cstdint>

namespace lkd {

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kDecHd = 64;     // head dim
constexpr int kDecChunk = 64;  // keys per decode chunk
constexpr int kPartStride = kDecHd + 2;

// rows per wave of the partial GEMV: 16 for K <= 1024, else 64 (12 slices at K = 768 and at K = 3072)
inline int64_t gemvRowsPerWave(int64_t k) { return k <= 1024 ? 16 : 64; }

#ifndef LK_GEMV_MIN_WGS
#define LK_GEMV_MIN_WGS 256
#endif
// Column block of the partial GEMV: the widest of 256 / 128 / 64 columns whose grid still has LK_GEMV_MIN_WGS
// workgroups, else 64.
inline int gemvColBlock(int64_t n, int64_t slices) {
  for (int cb = 256; cb > 64; cb /= 2)
    if (lkh::ceilDiv(n, cb) * slices >= LK_GEMV_MIN_WGS) return cb;
  return 64;
}

// Workgroup = 4 waves over CB columns and 4 * RPW rows; wave w owns rows r0 + w RPW .. + RPW - 1. A wave row of
// CB / 4 lanes (float4 each) spans the CB columns, so a wave holds RS = 256 / CB such rows: lane subgroup q sums
// rows q, q + RS, q + 2 RS, ... of the wave's RPW. The subgroups combine by permlane swaps ((q0 + q1) + (q2 + q3)),
// the four wave sums in LDS as (w0 + w1) + (w2 + w3), and the workgroup writes slice blockIdx.y. Narrow column
// blocks multiply the workgroups of a small-N GEMV (N = 768: 36 at CB = 256, 144 at CB = 64) without adding row
// slices for the consumer to sum. The workgroup's slice of x is first formed in LDS according to XMODE.
struct LnIn {  // mode 3: x = LayerNorm(sum of xpart slices + xbias + res), workgroup (0, 0) writes the sum
  const float* res;
  const float* gamma;
  const float* beta;
  float* sumOut;
  float eps;
};

// Sum of v over the RS lane subgroups of a wave (subgroup = 64 / RS consecutive lanes), in every subgroup.
template <int RS>
__device__ __forceinline__ float subgroupSum(float v) {
  if constexpr (RS == 1) {
    return v;
  } else {
    float r = v;
    if constexpr (RS == 4) {
      const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
      r = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
  }
}

template <int XMODE, int RPW, int CB>
__global__ __launch_bounds__(256) void gemvPartXKernel(const float* __restrict__ x, const float* __restrict__ xpart,
                                                      const float* __restrict__ xbias, int64_t xslices, int chunks,
                                                      LnIn ln, const float* __restrict__ w, float* __restrict__ part,
                                                      int64_t n, int64_t k) {
  constexpr int ROWS = 4 * RPW;
  __shared__ float xs[ROWS];
  constexpr int RS = 256 / CB, CL = CB / 4, LPW = RPW / RS;  // row subgroups, lanes per row, loads per lane
  static_assert(RPW % RS == 0, "rows per wave must split over the lane subgroups");
  __shared__ f4v wsum[4][CL];
  __shared__ float mrg[4][kDecHd];
  __shared__ float cw[64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t rBase = static_cast<int64_t>(blockIdx.y) * ROWS;
  // The weight loads do not depend on x: the first batch is issued before x is formed, so its latency overlaps
  // the prologue's own loads and reductions.
  constexpr int B0 = LPW < 32 ? LPW : 32;
  const int cl = lane % CL, q = lane / CL;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * CB + 4 * cl;
  const int64_t r0 = rBase + static_cast<int64_t>(wv) * RPW + q;  // this lane's rows r0 + RS i
  const int64_t colc = min<int64_t>(col, n - 4);  // columns past N compute on a valid column, never stored
  f4v wr[B0];
#pragma unroll
  for (int i = 0; i < B0; ++i)
    wr[i] = __builtin_nontemporal_load(
        reinterpret_cast<const f4v*>(w + min<int64_t>(r0 + RS * i, k - 1) * n + colc));
  if constexpr (XMODE == 0) {
    for (int t = tid; t < ROWS; t += 256) xs[t] = rBase + t < k ? x[rBase + t] : 0.0f;
  } else if constexpr (XMODE == 1) {
    // x[r] = gelu(sum_s xpart[s, r] + xbias[r]), slices in order
    for (int t = tid; t < ROWS; t += 256) {
      const int64_t r = rBase + t;
      float v = 0.0f;
      if (r < k) {
        float s = 0.0f;
#pragma unroll 12
        for (int64_t sl = 0; sl < xslices; ++sl) s += xpart[sl * k + r];
        v = geluTanh(s + xbias[r]);
      }
      xs[t] = v;
    }
  } else if constexpr (XMODE == 3) {
    // the whole row (K <= 1024): sum = slices in order + xbias + res, two-pass LayerNorm (biased variance)
    __shared__ float lnrow[1024];
    __shared__ float scr[4];
    float v[4];
    float s1 = 0.0f;
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = tid + 256 * j;
      float xv = 0.0f;
      if (c < k) {
        float sp = 0.0f;
#pragma unroll 12
        for (int64_t sl = 0; sl < xslices; ++sl) sp += xpart[sl * k + c];
        xv = sp + (xbias ? xbias[c] : 0.0f) + ln.res[c];
        if (writer) ln.sumOut[c] = xv;
      }
      v[j] = xv;
      s1 += xv;
    }
    s1 = waveSum(s1);
    if (lane == 0) scr[wv] = s1;
    __syncthreads();
    const float mean = ((scr[0] + scr[1]) + (scr[2] + scr[3])) / static_cast<float>(k);
    __syncthreads();
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = v[j] - mean;
      if (tid + 256 * j < k) s2 += d * d;
    }
    s2 = waveSum(s2);
    if (lane == 0) scr[wv] = s2;
    __syncthreads();
    const float var = ((scr[0] + scr[1]) + (scr[2] + scr[3])) / static_cast<float>(k);
    const float rstd = 1.0f / sqrtf(var + ln.eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = tid + 256 * j;
      if (c < k) lnrow[c] = (v[j] - mean) * rstd * ln.gamma[c] + ln.beta[c];
    }
    __syncthreads();
    for (int t = tid; t < ROWS; t += 256) xs[t] = rBase + t < k ? lnrow[rBase + t] : 0.0f;
  } else {
    // rows rBase .. rBase + 63 are head blockIdx.y: merge its chunk partials (m, l, acc) in chunk order,
    // M = max m_c, out[d] = sum_c e^{m_c - M} acc_c[d] / sum_c e^{m_c - M} l_c
    static_assert(XMODE != 2 || ROWS == kDecHd, "attention merge needs 64 rows per workgroup");
    const float* base = xpart + static_cast<int64_t>(blockIdx.y) * chunks * kPartStride;
    // chunk weights (chunks <= 64): lane c of wave 0 holds chunk c's (m, l)
    if (wv == 0) {
      const float mc = lane < chunks ? base[lane * kPartStride] : -INFINITY;
      const float lc = lane < chunks ? base[lane * kPartStride + 1] : 0.0f;
      const float M = waveMax(mc);
      const float wc = lc > 0.0f ? expf(mc - M) : 0.0f;
      cw[lane] = wc;
      const float L = waveSum(lc * wc);
      if (lane == 0) xs[0] = L;  // xs doubles as a scratch slot until the merge below
    }
    __syncthreads();
    // thread (d = lane, chunk group wv) sums chunks wv, wv + 4, ... for dim d; groups combine in order
    float a = 0.0f;
    for (int c = wv; c < chunks; c += 4) a += cw[c] * base[c * kPartStride + 2 + lane];
    mrg[wv][lane] = a;
    const float L = xs[0];
    __syncthreads();
    if (wv == 0) xs[lane] = ((mrg[0][lane] + mrg[1][lane]) + (mrg[2][lane] + mrg[3][lane])) / L;
    // NaN when the chunk kernel flagged an invalid position
  }
  __syncthreads();
  f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < B0; ++i) acc += xs[wv * RPW + q + RS * i] * wr[i];  // xs is 0 past K
#pragma unroll
  for (int b = B0; b < LPW; b += 32) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      wr[i] = __builtin_nontemporal_load(
          reinterpret_cast<const f4v*>(w + min<int64_t>(r0 + RS * (b + i), k - 1) * n + colc));
#pragma unroll
    for (int i = 0; i < 32; ++i) acc += xs[wv * RPW + q + RS * (b + i)] * wr[i];
  }
  acc.x = subgroupSum<RS>(acc.x);
  acc.y = subgroupSum<RS>(acc.y);
  acc.z = subgroupSum<RS>(acc.z);
  acc.w = subgroupSum<RS>(acc.w);
  if (q == 0) wsum[wv][cl] = acc;
  __syncthreads();
  if (wv == 0 && q == 0 && col < n)
    *reinterpret_cast<f4v*>(part + static_cast<int64_t>(blockIdx.y) * n + col) =
        (wsum[0][cl] + wsum[1][cl]) + (wsum[2][cl] + wsum[3][cl]);
}

// One wave per (head, 64-key chunk), as the split decode kernel, but q / k / v of this step are the fixed-order
// sums of `slices` GEMV partial rows (+ bias). An invalid position writes NaN partials (no cache write) and is
// recorded in the GPU's error record.
__global__ __launch_bounds__(64) void decodeChunkPartKernel(const float* __restrict__ qpart, int64_t slices,
                                                           float* kc, float* vc, const int64_t* pos,
                                                           const float* __restrict__ bias, float* __restrict__ cpart,
                                                           int64_t cap, int heads, int chunks,
                                                           unsigned long long* err) {
  __shared__ float qs[kDecHd], vs[kDecHd];
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int64_t D = static_cast<int64_t>(heads) * kDecHd, ld = 3 * D;
  float* part = cpart + (static_cast<int64_t>(h) * chunks + s) * kPartStride;
  const int64_t ps = *pos;
  if (ps < 0 || ps >= cap) {
    if (h == 0 && s == 0 && lane == 0) raiseDeviceError(err, LK_DEVERR_POSITION, ps);
    if (lane == 0) {
      part[0] = __builtin_nanf("");
      part[1] = 1.0f;
    }
    part[2 + lane] = __builtin_nanf("");
    return;
  }
  const int64_t kb = static_cast<int64_t>(s) * kDecChunk;
  const int64_t ke = min<int64_t>(ps + 1, kb + kDecChunk);
  if (kb >= ke) {  // chunk past the live keys
    if (lane == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    part[2 + lane] = 0.0f;
    return;
  }
  // this lane's dim of q, k, v: fixed-order sums of the partial rows
  const int64_t cq = h * kDecHd + lane;
  float sq = 0.0f, sk = 0.0f, sv = 0.0f;
#pragma unroll 12
  for (int64_t sl = 0; sl < slices; ++sl) {
    const float* row = qpart + sl * ld;
    sq += row[cq];
    sk += row[D + cq];
    sv += row[2 * D + cq];
  }
  const float qd = (sq + bias[cq]) * 0.125f;
  const float knew = sk + bias[D + cq];
  const float vnew = sv + bias[2 * D + cq];
  if (ps >= kb && ps < kb + kDecChunk) {
    kc[ps * D + cq] = knew;
    vc[ps * D + cq] = vnew;
  }
  qs[lane] = qd;
  vs[lane] = vnew;
  const float snew = waveSum(qd * knew);
  __syncthreads();
  float q[kDecHd];
#pragma unroll
  for (int d = 0; d < kDecHd; ++d) q[d] = qs[d];

  const int64_t j = kb + lane;
  float sc = -INFINITY;
  if (j < ke) {
    if (j == ps) {
      sc = snew;
    } else {
      const f4v* kr = reinterpret_cast<const f4v*>(kc + j * D + h * kDecHd);
      f4v kv[kDecHd / 4];
#pragma unroll
      for (int d4 = 0; d4 < kDecHd / 4; ++d4) kv[d4] = kr[d4];
      float dot = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < kDecHd / 4; ++d4)
        dot += q[4 * d4] * kv[d4].x + q[4 * d4 + 1] * kv[d4].y + q[4 * d4 + 2] * kv[d4].z + q[4 * d4 + 3] * kv[d4].w;
      sc = dot;
    }
  }
  const float m = waveMax(sc);
  const float pj = j < ke ? expf(sc - m) : 0.0f;
  const float l = waveSum(pj);

  // P.V: lane = (g, d4); keys kb + g + 4 i, i = 0..15
  const int g = lane >> 4, d4 = lane & 15;
  f4v vv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = kb + g + 4 * i;
    if (row < ke && row != ps) {
      vv[i] = reinterpret_cast<const f4v*>(vc + row * D + h * kDecHd)[d4];
    } else if (row == ps) {
      vv[i] = f4v{vs[4 * d4], vs[4 * d4 + 1], vs[4 * d4 + 2], vs[4 * d4 + 3]};
    } else {
      vv[i] = f4v{0.f, 0.f, 0.f, 0.f};
    }
  }
  f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 16; ++i) acc += __shfl(pj, g + 4 * i, 64) * vv[i];
#pragma unroll
  for (int o = 16; o < 64; o <<= 1) {
    acc.x += __shfl_xor(acc.x, o, 64);
    acc.y += __shfl_xor(acc.y, o, 64);
    acc.z += __shfl_xor(acc.z, o, 64);
    acc.w += __shfl_xor(acc.w, o, 64);
  }
  if (lane == 0) {
    part[0] = m;
    part[1] = l;
  }
  if (g == 0) reinterpret_cast<f4v*>(part + 2)[d4] = acc;
}

constexpr int kRedMaxPerThread = 4;  // N <= 1024

__device__ __forceinline__ float blockSum1024(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  v = waveSum(v);
  __syncthreads();
  if (lane == 0) scratch[wv] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += scratch[i];
  return t;
}

// One 1024-thread workgroup: thread (c, q) sums slices q, q + 4, ... of columns c + 256 j; the quarter sums
// combine as (q0 + q1) + (q2 + q3); then sum = . + bias + res is written and LayerNorm'ed (two-pass, biased).
__global__ __launch_bounds__(1024) void reduceLnKernel(const float* __restrict__ part, int64_t slices,
                                                      const float* __restrict__ bias, const float* __restrict__ res,
                                                      const float* __restrict__ gamma, const float* __restrict__ beta,
                                                      float* __restrict__ sumOut, float* __restrict__ lnOut, int64_t n,
                                                      float eps) {
  __shared__ float red[4][256 * kRedMaxPerThread];
  __shared__ float scratch[16];
  const int tid = threadIdx.x, c = tid & 255, q = tid >> 8;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const int64_t col = c + 256 * j;
    float s = 0.0f;
    if (col < n) {
#pragma unroll 4
      for (int64_t sl = q; sl < slices; sl += 4) s += part[sl * n + col];
    }
    red[q][c + 256 * j] = s;
  }
  __syncthreads();
  // threads q == 0 own the columns; the others contribute zeros to the block sums
  float v[kRedMaxPerThread];
  float s1 = 0.0f;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const int64_t col = c + 256 * j;
    float x = 0.0f;
    if (q == 0 && col < n) {
      const int o = c + 256 * j;
      x = ((red[0][o] + red[1][o]) + (red[2][o] + red[3][o])) + bias[col] + res[col];
      sumOut[col] = x;
    }
    v[j] = x;
    s1 += x;
  }
  const float mean = blockSum1024(s1, scratch) / static_cast<float>(n);
  float s2 = 0.0f;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const float d = v[j] - mean;
    if (q == 0 && c + 256 * j < n) s2 += d * d;
  }
  const float var = blockSum1024(s2, scratch) / static_cast<float>(n);
  const float rstd = 1.0f / sqrtf(var + eps);
  if (q == 0) {
#pragma unroll
    for (int j = 0; j < kRedMaxPerThread; ++j) {
      const int64_t col = c + 256 * j;
      if (col < n) lnOut[col] = (v[j] - mean) * rstd * gamma[col] + beta[col];
    }
  }
}

}  // namespace lkd

extern "C" {

int64_t lk_hip_gemv_partial_slices(int64_t k) {
  const int64_t rpw = lkd::gemvRowsPerWave(k);
  return (k + 4 * rpw - 1) / (4 * rpw);
}

int lk_hip_gemv_partial_f32(int xmode, const float* x, const float* xpart, const float* xbias, int64_t xslices,
                            int chunks, const float* res, const float* gamma, const float* beta, float* sum_out,
                            float eps, const float* w, float* part, int64_t n, int64_t k, void* stream) {
  if (n <= 0 || k <= 0 || n % 4 != 0) return 1;
  const lkd::LnIn ln{res, gamma, beta, sum_out, eps};
  if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(part)) & 15) != 0) return 1;
  const int64_t rpw = lkd::gemvRowsPerWave(k);
  const int64_t slices = (k + 4 * rpw - 1) / (4 * rpw);
  const int cb = lkd::gemvColBlock(n, slices);
  const dim3 grid(lkh::ceilDiv(n, cb), static_cast<unsigned>(slices));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LK_GP_CB(MODE, R, CB) \
  hipLaunchKernelGGL((lkd::gemvPartXKernel<MODE, R, CB>), grid, dim3(256), 0, s, x, xpart, xbias, xslices, chunks, ln, \
                     w, part, n, k)
#define LK_GP(MODE, R)                    \
  do {                                    \
    if (cb == 256) LK_GP_CB(MODE, R, 256); \
    else if (cb == 128) LK_GP_CB(MODE, R, 128); \
    else LK_GP_CB(MODE, R, 64);           \
  } while (0)
  if (xmode == 0) {
    if (rpw == 16) LK_GP(0, 16);
    else LK_GP(0, 64);
  } else if (xmode == 1) {
    if (rpw == 16) LK_GP(1, 16);
    else LK_GP(1, 64);
  } else if (xmode == 2) {
    if (rpw != 16 || k % lkd::kDecHd != 0 || chunks <= 0 || chunks > 64) return 1;
    LK_GP(2, 16);
  } else if (xmode == 3) {
    if (k > 1024 || !res || !gamma || !beta || !sum_out || (xslices > 0 && !xpart)) return 1;
    LK_GP(3, 16);
  } else {
    return 1;
  }
#undef LK_GP
#undef LK_GP_CB
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_attention_decode_part_f32(const float* qkv_part, int64_t slices, float* kc, float* vc, const int64_t* pos,
                                     const float* bias, float* chunk_part, int64_t cap, int heads, void* stream) {
  if (heads <= 0 || cap <= 0 || slices <= 0) return 1;
  const int chunks = static_cast<int>((cap + lkd::kDecChunk - 1) / lkd::kDecChunk);
  hipLaunchKernelGGL(lkd::decodeChunkPartKernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(chunks)),
                     dim3(64), 0, static_cast<hipStream_t>(stream), qkv_part, slices, kc, vc, pos, bias, chunk_part,
                     cap, heads, chunks, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_reduce_ln_f32(const float* part, int64_t slices, const float* bias, const float* res, const float* gamma,
                         const float* beta, float* sum_out, float* ln_out, int64_t n, float eps, void* stream) {
  if (n <= 0 || n > 256 * lkd::kRedMaxPerThread || slices <= 0) return 1;
  hipLaunchKernelGGL(lkd::reduceLnKernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), part, slices,
                     bias, res, gamma, beta, sum_out, ln_out, n, eps);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// gemv_partial_f32_gpu(x[1, K], w[K, N]) -> part[S, N]
void runGemvPartial(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t k = a.ints[1], n = a.ints[3];
  LK_REQUIRE(ctx, a.ints[0] == 1 && a.ints[2] == k && a.ints[4] == lk_hip_gemv_partial_slices(k) && a.ints[5] == n,
             "gemv_partial: expected x [1, K], w [K, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(0, P<float>(a, 0), nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, nullptr, 0.0f,
                              P<float>(a, 1), P<float>(a, 2), n, k, ctx.stream))
    ctx.error = "gemv_partial: N % 4 != 0 or unaligned operands";
}

// gemv_partial_gelu_f32_gpu(xpart[Sx, K], xbias[K], w[K, N]) -> part[S, N], x = gelu(sum xpart + xbias)
void runGemvPartialGelu(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t sx = a.ints[0], k = a.ints[1], n = a.ints[4];
  LK_REQUIRE(ctx, a.ints[2] == k && a.ints[3] == k && a.ints[5] == lk_hip_gemv_partial_slices(k) && a.ints[6] == n,
             "gemv_partial_gelu: expected xpart [Sx, K], xbias [K], w [K, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(1, nullptr, P<float>(a, 0), P<float>(a, 1), sx, 0, nullptr, nullptr, nullptr, nullptr,
                              0.0f, P<float>(a, 2), P<float>(a, 3), n, k, ctx.stream))
    ctx.error = "gemv_partial_gelu: N % 4 != 0 or unaligned operands";
}

// gemv_partial_attn_f32_gpu(chunks[H, C, 66], w[64 H, N]) -> part[S, N], x = merged decode attention
void runGemvPartialAttn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t h = a.ints[0], c = a.ints[1], k = a.ints[3], n = a.ints[4];
  LK_REQUIRE(ctx, a.ints[2] == lkd::kPartStride && k == 64 * h && a.ints[5] == lk_hip_gemv_partial_slices(k) &&
                      a.ints[6] == n,
             "gemv_partial_attn: expected chunks [H, C, 66], w [64 H, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(2, nullptr, P<float>(a, 0), nullptr, 0, static_cast<int>(c), nullptr, nullptr, nullptr,
                              nullptr, 0.0f, P<float>(a, 1), P<float>(a, 2), n, k, ctx.stream))
    ctx.error = "gemv_partial_attn: invalid configuration";
}

// gemv_partial_res_ln_f32_gpu(xpart[Sx, K], xbias[K], res[1, K], gamma[K], beta[K], w[K, N]; eps)
//   -> (part[S, N], sum[1, K]); x = LN(sum), sum = slices of xpart + xbias + res
void runGemvPartialResLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t sx = a.ints[0], k = a.ints[1], n = a.ints[8];
  LK_REQUIRE(ctx, a.ints[2] == k && a.ints[3] == 1 && a.ints[4] == k && a.ints[5] == k && a.ints[6] == k &&
                      a.ints[7] == k && a.ints[9] == lk_hip_gemv_partial_slices(k) && a.ints[10] == n &&
                      a.ints[11] == 1 && a.ints[12] == k,
             "gemv_partial_res_ln: expected xpart [Sx, K], xbias [K], res [1, K], gamma [K], beta [K], w [K, N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_gemv_partial_f32(3, nullptr, P<float>(a, 0), P<float>(a, 1), sx, 0, P<float>(a, 2), P<float>(a, 3),
                              P<float>(a, 4), P<float>(a, 7), eps, P<float>(a, 5), P<float>(a, 6), n, k, ctx.stream))
    ctx.error = "gemv_partial_res_ln: K > 1024, N % 4 != 0 or unaligned operands";
}

// gemv_partial_ln_f32_gpu(x[1, K], gamma[K], beta[K], w[K, N]; eps) -> (part[S, N], copy of x [1, K]); x' = LN(x)
void runGemvPartialLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t k = a.ints[1], n = a.ints[5];
  LK_REQUIRE(ctx, a.ints[0] == 1 && a.ints[2] == k && a.ints[3] == k && a.ints[4] == k &&
                      a.ints[6] == lk_hip_gemv_partial_slices(k) && a.ints[7] == n && a.ints[8] == 1 &&
                      a.ints[9] == k,
             "gemv_partial_ln: expected x [1, K], gamma [K], beta [K], w [K, N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_gemv_partial_f32(3, nullptr, nullptr, nullptr, 0, 0, P<float>(a, 0), P<float>(a, 1), P<float>(a, 2),
                              P<float>(a, 5), eps, P<float>(a, 3), P<float>(a, 4), n, k, ctx.stream))
    ctx.error = "gemv_partial_ln: K > 1024, N % 4 != 0 or unaligned operands";
}

// attention_decode_part_f32_gpu(qkv_part[S, 3D], kc[cap, D], vc[cap, D], pos[1], bias[3D]; heads)
//   -> chunks[heads, ceil(cap / 64), 66]; writes row pos of kc, vc
void runAttnDecodePart(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], d3 = a.ints[1], cap = a.ints[2], d = a.ints[3];
  const int heads = static_cast<int>(a.ints[11]);
  LK_REQUIRE(ctx, d3 == 3 * d && d == 64 * heads && a.ints[4] == cap && a.ints[5] == d && a.ints[6] == 1 &&
                      a.ints[7] == d3 && a.ints[8] == heads && a.ints[9] == (cap + 63) / 64 && a.ints[10] == 66,
             "attention_decode_part: expected qkv_part [S, 3D], kc/vc [cap, D], pos [1], bias [3D], D = 64 heads");
  if (lk_hip_attention_decode_part_f32(P<float>(a, 0), s, P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                       P<float>(a, 4), P<float>(a, 5), cap, heads, ctx.stream))
    ctx.error = "attention_decode_part: launch failed";
}

// reduce_bias_res_ln2_f32_gpu(part[S, N], bias[N], res[1, N], gamma[N], beta[N]; eps) -> (sum[1, N], ln[1, N])
void runReduceLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], n = a.ints[1];
  LK_REQUIRE(ctx, a.ints[2] == n && a.ints[3] == 1 && a.ints[4] == n && a.ints[5] == n && a.ints[6] == n,
             "reduce_bias_res_ln2: expected part [S, N], bias [N], res [1, N], gamma [N], beta [N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_reduce_ln_f32(P<float>(a, 0), s, P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), P<float>(a, 4),
                           P<float>(a, 5), P<float>(a, 6), n, eps, ctx.stream))
    ctx.error = "reduce_bias_res_ln2: N > 1024";
}

}  // namespace

void registerDecodeFusedKernels() {
  const Device G = Device::Gpu;
  registerKernel({"gemv_partial_f32_gpu", G, runGemvPartial, 2, 1});
  registerKernel({"gemv_partial_gelu_f32_gpu", G, runGemvPartialGelu, 3, 1});
  registerKernel({"gemv_partial_attn_f32_gpu", G, runGemvPartialAttn, 2, 1});
  registerKernel({"gemv_partial_res_ln_f32_gpu", G, runGemvPartialResLn, 6, 2});
  registerKernel({"gemv_partial_ln_f32_gpu", G, runGemvPartialLn, 4, 2});
  registerKernel({"attention_decode_part_f32_gpu", G, runAttnDecodePart, 5, 1});
  registerKernel({"reduce_bias_res_ln2_f32_gpu", G, runReduceLn, 5, 2});
}

}  // namespace lkh
