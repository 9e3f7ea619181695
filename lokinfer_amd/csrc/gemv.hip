// Bandwidth-bound matrix-vector kernels (decode-time GEMVs, tied LM head, one-column projections).
//
//   lk_hip_gemv_f32   out[1, N] = act(x[1, K] . W[K, N] + b) + res     (reference gemv4*_f32_gpu,
//                     transformer_gpu.cpp:233-251; kokoro_tok.metal:878-924)
//   lk_hip_rowdot_f32 out[m, r] = vec[m, :] . mat[r, :] (+ bias)        (reference gemm_nt_f32_gpu_mps at M = 1
//                     for the GPT-2 LM head, gemv_rows_f32_gpu kokoro_lc.cpp:227-254, gemv1_bias_f32_gpu
//                     kokoro_lc.cpp:257-267 / vision.metal:266-284)
//
// gemv: one 1024-thread workgroup (16 waves) owns a 16-column slab of W over the whole K: 4 lanes x float4
// cover the 16 columns (64 contiguous bytes of a row) and the 256 row slots stride K, so every thread has
// K / 256 independent loads in flight. The 256 partial sums per column are reduced in LDS in a fixed order:
// no cross-workgroup communication, deterministic results, one launch. N / 16 workgroups (48 at N = 768,
// 192 at N = 3072) each stream K x 64 B.
#include "common.h"

#include <algorithm>

namespace lkd {

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ntLoad4(const float* p) {
  const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

constexpr int kGemvCols = 16;
constexpr int kGemvThreads = 1024;
constexpr int kGemvSlots = kGemvThreads / (kGemvCols / 4);  // 256

struct GemvParams {
  const float* x;
  const float* w;
  const float* bias;
  const float* res;
  float* out;
  int64_t n, k;
  int act;  // 0 none, 2 gelu_tanh
};

__global__ __launch_bounds__(kGemvThreads) void gemvKernel(GemvParams p) {
  __shared__ float4 red[kGemvSlots][kGemvCols / 4];
  const int tid = threadIdx.x;
  const int cl = tid & 3, slot = tid >> 2;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kGemvCols + cl * 4;
  const bool vec = (p.n & 3) == 0 && col + 3 < p.n;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (col < p.n) {
#pragma unroll 4
    for (int64_t k = slot; k < p.k; k += kGemvSlots) {
      const float xv = p.x[k];
      const float* wr = p.w + k * p.n + col;
      float4 wv;
      if (vec) {
        wv = ntLoad4(wr);
      } else {
        wv.x = wr[0];
        wv.y = col + 1 < p.n ? wr[1] : 0.f;
        wv.z = col + 2 < p.n ? wr[2] : 0.f;
        wv.w = col + 3 < p.n ? wr[3] : 0.f;
      }
      acc.x += xv * wv.x;
      acc.y += xv * wv.y;
      acc.z += xv * wv.z;
      acc.w += xv * wv.w;
    }
  }
  red[slot][cl] = acc;
  __syncthreads();
  // Tree over the 256 slots: 8 halvings, each step adds slot s + half into s.
  for (int half = kGemvSlots / 2; half > 0; half >>= 1) {
    if (slot < half) {
      const float4 o = red[slot + half][cl];
      float4 v = red[slot][cl];
      v.x += o.x;
      v.y += o.y;
      v.z += o.z;
      v.w += o.w;
      red[slot][cl] = v;
    }
    __syncthreads();
  }
  if (slot == 0) {
    const float4 v = red[0][cl];
    const float vv[4] = {v.x, v.y, v.z, v.w};
    for (int q = 0; q < 4; ++q) {
      const int64_t c = col + q;
      if (c >= p.n) break;
      float o = vv[q];
      if (p.bias) o += p.bias[c];
      if (p.act == 2) o = geluTanh(o);
      if (p.res) o += p.res[c];
      p.out[c] = o;
    }
  }
}

// One wave per matrix row: out[m * ldo + r] = sum_k vec[m, k] mat[r, k] (+ bias). K % 4 == 0 (float4 loads).
template <int MV>
__global__ __launch_bounds__(256) void rowdotKernel(const float* __restrict__ mat, const float* __restrict__ vec,
                                                    const float* bias, int biasPerRow, float* out, int64_t rows,
                                                    int64_t k, int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int64_t wavesTotal = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); r < rows; r += wavesTotal) {
    float acc[MV];
#pragma unroll
    for (int m = 0; m < MV; ++m) acc[m] = 0.f;
    const float* mr = mat + r * k;
    for (int64_t q = lane; q < k / 4; q += 64) {
      const float4 a = ntLoad4(mr + 4 * q);
#pragma unroll
      for (int m = 0; m < MV; ++m) {
        const float4 v = reinterpret_cast<const float4*>(vec + m * k)[q];
        acc[m] += a.x * v.x + a.y * v.y + a.z * v.z + a.w * v.w;
      }
    }
#pragma unroll
    for (int m = 0; m < MV; ++m) {
      float s = waveSum(acc[m]);
      if (lane == 0) {
        if (bias) s += biasPerRow ? bias[r] : bias[0];
        out[m * ldo + r] = s;
      }
    }
  }
}

}  // namespace lkd

extern "C" {

int lk_hip_gemv_f32(const float* x, const float* w, const float* bias, const float* res, float* out, int64_t n,
                    int64_t k, int act, void* stream) {
  if (n <= 0 || k < 0) return n == 0 ? 0 : 1;
  lkd::GemvParams p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.res = res;
  p.out = out;
  p.n = n;
  p.k = k;
  p.act = act;
  const unsigned blocks = lkh::ceilDiv(n, lkd::kGemvCols);
  hipLaunchKernelGGL(lkd::gemvKernel, dim3(blocks), dim3(lkd::kGemvThreads), 0, static_cast<hipStream_t>(stream), p);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// out[m, r] (row stride ldo) = vec[m, :K] . mat[r, :K] (+ bias[r] or + bias[0]); m < nvec <= 8, K % 4 == 0.
int lk_hip_rowdot_f32(const float* mat, const float* vec, const float* bias, int biasPerRow, float* out,
                      int64_t rows, int64_t k, int nvec, int64_t ldo, void* stream) {
  if (rows <= 0) return rows == 0 ? 0 : 1;
  if (k % 4 != 0 || nvec < 1 || nvec > 8) return 1;
  const int64_t blocks = std::min<int64_t>((rows + 3) / 4, 8192);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 g(static_cast<unsigned>(blocks)), b(256);
  switch (nvec) {
#define LK_CASE(M) \
  case M: hipLaunchKernelGGL(lkd::rowdotKernel<M>, g, b, 0, s, mat, vec, bias, biasPerRow, out, rows, k, ldo); break;
    LK_CASE(1) LK_CASE(2) LK_CASE(3) LK_CASE(4) LK_CASE(5) LK_CASE(6) LK_CASE(7) LK_CASE(8)
#undef LK_CASE
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
