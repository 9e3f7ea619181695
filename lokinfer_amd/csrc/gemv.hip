// Bandwidth-bound matrix-vector kernels (decode-time GEMVs, tied LM head, one-column projections).
//
//   lk_hip_gemv_f32   out[1, N] = act(x[1, K] . W[K, N] + b) + res     (reference gemv4*_f32_gpu,
//                     transformer_gpu.cpp:233-251; kokoro_tok.metal:878-924)
//   lk_hip_rowdot_f32 out[m, r] = vec[m, :] . mat[r, :] (+ bias)        (reference gemm_nt_f32_gpu_mps at M = 1
//                     for the GPT-2 LM head, gemv_rows_f32_gpu kokoro_lc.cpp:227-254, gemv1_bias_f32_gpu
//                     kokoro_lc.cpp:257-267 / vision.metal:266-284)
//
// gemv: each 256-thread workgroup owns 64 columns (16 lanes x float4) and a K-chunk (16 row slots); the K
// split makes enough workgroups to keep HBM busy at N = 768. Partials land in the caller's workspace and the
// last workgroup of a column group (atomic ticket) sums them in fixed split order, so results are
// deterministic and the op stays one launch. The ticket counters are restored to 0 by that last workgroup.
#include "common.h"

#include <algorithm>

namespace lkd {

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ntLoad4(const float* p) {
  const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

struct GemvParams {
  const float* x;
  const float* w;
  const float* bias;
  const float* res;
  float* out;
  float* partial;       // [splits, N]
  unsigned* tickets;    // [ceil(N / 64)], zero between calls
  int64_t n, k;
  int splits;
  int64_t kChunk;
  int act;  // 0 none, 2 gelu_tanh
};

__global__ __launch_bounds__(256) void gemvKernel(GemvParams p) {
  __shared__ float4 red[16][17];
  __shared__ bool last;
  const int tid = threadIdx.x;
  const int cl = tid & 15, slot = tid >> 4;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 64 + cl * 4;
  const int s = blockIdx.y;
  const int64_t kb = s * p.kChunk, ke = min(p.k, kb + p.kChunk);
  const bool vec = (p.n & 3) == 0 && col + 3 < p.n;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t k = kb + slot; k < ke; k += 16) {
    const float xv = p.x[k];
    const float* wr = p.w + k * p.n + col;
    float4 wv;
    if (vec) {
      wv = ntLoad4(wr);
    } else {
      wv.x = col < p.n ? wr[0] : 0.f;
      wv.y = col + 1 < p.n ? wr[1] : 0.f;
      wv.z = col + 2 < p.n ? wr[2] : 0.f;
      wv.w = col + 3 < p.n ? wr[3] : 0.f;
    }
    acc.x += xv * wv.x;
    acc.y += xv * wv.y;
    acc.z += xv * wv.z;
    acc.w += xv * wv.w;
  }
  red[slot][cl] = acc;
  __syncthreads();
  float4 tot = make_float4(0.f, 0.f, 0.f, 0.f);
  if (slot == 0) {
    for (int j = 0; j < 16; ++j) {
      const float4 v = red[j][cl];
      tot.x += v.x;
      tot.y += v.y;
      tot.z += v.z;
      tot.w += v.w;
    }
  }
  auto finish = [&](float4 v) {
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
  };
  if (p.splits == 1) {
    if (slot == 0) finish(tot);
    return;
  }
  if (slot == 0) {
    const float tv[4] = {tot.x, tot.y, tot.z, tot.w};
    for (int q = 0; q < 4; ++q)
      if (col + q < p.n) p.partial[static_cast<int64_t>(s) * p.n + col + q] = tv[q];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned t = atomicAdd(&p.tickets[blockIdx.x], 1u);
    last = (t == static_cast<unsigned>(p.splits - 1));
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (slot == 0) {
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < p.splits; ++j) {
      const float* pr = p.partial + static_cast<int64_t>(j) * p.n + col;
      // Device-coherent reads: the partials were written by other workgroups (possibly other XCDs).
      sum.x += col < p.n ? __hip_atomic_load(pr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      sum.y += col + 1 < p.n ? __hip_atomic_load(pr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      sum.z += col + 2 < p.n ? __hip_atomic_load(pr + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      sum.w += col + 3 < p.n ? __hip_atomic_load(pr + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
    finish(sum);
  }
  if (tid == 0) p.tickets[blockIdx.x] = 0u;
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
    const float4* mr = reinterpret_cast<const float4*>(mat + r * k);
    for (int64_t q = lane; q < k / 4; q += 64) {
      const float4 a = ntLoad4(reinterpret_cast<const float*>(mr + q));
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

// Workspace bytes gemv needs: tickets (64 KiB, zero-initialised once by the owner) + partials.
int64_t lk_hip_gemv_workspace_bytes(int64_t n, int64_t k) {
  (void)k;
  return 65536 + 64 * n * static_cast<int64_t>(sizeof(float));
}

int lk_hip_gemv_f32(const float* x, const float* w, const float* bias, const float* res, float* out, int64_t n,
                    int64_t k, int act, void* workspace, int64_t workspaceBytes, void* stream) {
  if (n <= 0) return n == 0 ? 0 : 1;
  lkd::GemvParams p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.res = res;
  p.out = out;
  p.n = n;
  p.k = k;
  p.act = act;
  const int64_t colGroups = (n + 63) / 64;
  // Aim for ~1024 workgroups; each split covers at least 32 rows.
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>((1024 + colGroups - 1) / colGroups, (k + 31) / 32));
  splits = std::min<int64_t>(splits, 64);
  if (splits > 1 && (workspace == nullptr || colGroups > 16384 ||
                     workspaceBytes < 65536 + splits * n * static_cast<int64_t>(sizeof(float))))
    splits = 1;
  p.splits = static_cast<int>(splits);
  p.kChunk = (k + splits - 1) / splits;
  p.tickets = static_cast<unsigned*>(workspace);
  p.partial = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + 65536) : nullptr;
  dim3 grid(static_cast<unsigned>(colGroups), static_cast<unsigned>(splits));
  hipLaunchKernelGGL(lkd::gemvKernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), p);
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
