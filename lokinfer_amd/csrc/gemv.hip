// Bandwidth-bound matrix-vector kernels (decode-time GEMVs, tied LM head, one-column projections).
//
//   lk_hip_gemv_f32   out[1, N] = act(x[1, K] . W[K, N] + b) + res     (reference gemv4*_f32_gpu,
//                     transformer_gpu.cpp:233-251; kokoro_tok.metal:878-924)
//   lk_hip_rowdot_f32 out[m, r] = vec[m, :] . mat[r, :] (+ bias)        (reference gemm_nt_f32_gpu_mps at M = 1
//                     for the GPT-2 LM head, gemv_rows_f32_gpu kokoro_lc.cpp:227-254, gemv1_bias_f32_gpu
//                     kokoro_lc.cpp:257-267 / vision.metal:266-284)
//
// gemv, two launches (the default when a workspace is given): at decode sizes (2-10 MB per matrix) the
// stream is latency-bound unless nearly the whole matrix is in flight at once, so
//   1. gemvPartialKernel: a wave covers 256 columns (64 lanes x float4, 1 KB of a row) x 16 rows and issues its
//      16 loads back to back; grid = ceil(N / 256) x ceil(K / 64) workgroups of 4 waves. Each wave writes its
//      16-row partial sums (summed in row order) to the workspace as slice s = 4 * blockIdx.y + wave;
//   2. gemvReduceKernel: per column, the K / 16 slices are summed in a fixed order (4 interleaved chains, then
//      (c0 + c1) + (c2 + c3)) and the epilogue (bias, gelu, residual) applied.
// Deterministic; no cross-workgroup communication inside a launch.
// gemv without a workspace (or N % 4 != 0): one 1024-thread workgroup (16 waves) owns a 16-column slab of W over
// the whole K: 4 lanes x float4 cover the 16 columns and the 256 row slots stride K; the 256 partial sums per
// column are reduced in LDS in a fixed order.
#include "common.h"

#include <algorithm>
#include <cstdint>

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

constexpr int kGemvRowsPerWave = 16;

__global__ __launch_bounds__(256) void gemvPartialKernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        float* __restrict__ part, int64_t n, int64_t k) {
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + 4 * lane;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64 + kGemvRowsPerWave * wv;
  const int64_t slice = static_cast<int64_t>(blockIdx.y) * 4 + wv;
  if (col >= n) return;
  f4v wr[kGemvRowsPerWave];
#pragma unroll
  for (int i = 0; i < kGemvRowsPerWave; ++i)
    wr[i] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(w + min<int64_t>(r0 + i, k - 1) * n + col));
  f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kGemvRowsPerWave; ++i) {
    const float xv = r0 + i < k ? x[r0 + i] : 0.0f;
    acc += xv * wr[i];
  }
  *reinterpret_cast<f4v*>(part + slice * n + col) = acc;
}

__global__ __launch_bounds__(256) void gemvReduceKernel(const float* __restrict__ part, GemvParams p,
                                                       int64_t slices) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 64 + c;
  float s = 0.0f;
  if (col < p.n) {
#pragma unroll 8
    for (int64_t sl = q; sl < slices; sl += 4) s += part[sl * p.n + col];
  }
  red[q][c] = s;
  __syncthreads();
  if (q == 0 && col < p.n) {
    float o = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
    if (p.bias) o += p.bias[col];
    if (p.act == 2) o = geluTanh(o);
    if (p.res) o += p.res[col];
    p.out[col] = o;
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
                    int64_t k, int act, void* workspace, int64_t workspaceBytes, void* stream) {
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t kBlocks = (k + 63) / 64, slices = 4 * kBlocks;
  const bool aligned = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(workspace)) & 15) == 0;
  if (k > 0 && n % 4 == 0 && aligned && workspace && workspaceBytes >= slices * n * 4 && kBlocks < 65536) {
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(lkd::gemvPartialKernel, dim3(lkh::ceilDiv(n, 256), static_cast<unsigned>(kBlocks)), dim3(256),
                       0, s, x, w, part, n, k);
    hipLaunchKernelGGL(lkd::gemvReduceKernel, dim3(lkh::ceilDiv(n, 64)), dim3(256), 0, s, part, p, slices);
  } else {
    const unsigned blocks = lkh::ceilDiv(n, lkd::kGemvCols);
    hipLaunchKernelGGL(lkd::gemvKernel, dim3(blocks), dim3(lkd::kGemvThreads), 0, s, p);
  }
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
