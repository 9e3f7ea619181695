// Token-rate front-end kernels on the GPU. The reference runs these as host CPU kernels inside its GPU graphs
// (embedding_f32_cpu, kernels/cpu/kokoro_norm.cpp; argmax in Python, models/gpt2.py:348-359); here they stay
// on the device so that a decode step or a forward is one captured graph with no host round trips.
//
//   lk_hip_embedding_f32   out[i] = table[ids[i]] (+ table2[ids2[i]])   ids out of range -> row of NaN
//   lk_hip_argmax_f32      per row: index of the first maximum (int64)
#include "common.h"

namespace lkd {

__global__ void embeddingKernel(const float* __restrict__ table, const int64_t* __restrict__ ids,
                                const float* __restrict__ table2, const int64_t* __restrict__ ids2,
                                float* __restrict__ out, int64_t n, int64_t d, int64_t rows, int64_t rows2) {
  const int64_t total = n * d;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d, c = i - r * d;
    const int64_t id = ids[r];
    float v = (id >= 0 && id < rows) ? table[id * d + c] : __builtin_nanf("");
    if (table2) {
      const int64_t id2 = ids2[r];
      v += (id2 >= 0 && id2 < rows2) ? table2[id2 * d + c] : __builtin_nanf("");
    }
    out[i] = v;
  }
}

// One workgroup per row: (value, index) max with ties to the lower index (numpy / torch argmax semantics).
__global__ __launch_bounds__(256) void argmaxKernel(const float* __restrict__ x, int64_t* __restrict__ out,
                                                   int64_t n) {
  __shared__ float sv[4];
  __shared__ int64_t si[4];
  const float* row = x + static_cast<int64_t>(blockIdx.x) * n;
  float best = -INFINITY;
  int64_t bi = n;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float v = row[i];
    if (v > best || (bi == n && !(v < best))) {  // first element (also -inf / NaN rows) seeds the index
      best = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
        best = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi < n ? bi : 0;
  }
}

}  // namespace lkd

extern "C" {

int lk_hip_embedding_f32(const float* table, const int64_t* ids, const float* table2, const int64_t* ids2, float* out,
                         int64_t n, int64_t d, int64_t rows, int64_t rows2, void* stream) {
  const int64_t total = n * d;
  if (total <= 0) return total == 0 ? 0 : 1;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(lkd::embeddingKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), table, ids, table2, ids2, out, n, d, rows, rows2);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_argmax_f32(const float* x, int64_t* out, int64_t rows, int64_t n, void* stream) {
  if (rows <= 0 || n <= 0) return 1;
  hipLaunchKernelGGL(lkd::argmaxKernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, out, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// embedding_f32_gpu(table[V, D], ids i64[N]) -> [N, D]
void runEmbedding(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t v = a.ints[0], d = a.ints[1], n = a.ints[2];
  if (lk_hip_embedding_f32(P<float>(a, 0), P<int64_t>(a, 1), nullptr, nullptr, P<float>(a, 2), n, d, v, 0,
                           ctx.stream))
    ctx.error = "embedding: launch failed";
}

// embedding2_add_f32_gpu(table[V, D], ids i64[N], table2[V2, D], ids2 i64[N]) -> [N, D] (token + position)
void runEmbedding2(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t v = a.ints[0], d = a.ints[1], n = a.ints[2], v2 = a.ints[3];
  LK_REQUIRE(ctx, a.ints[4] == d && a.ints[5] == n, "embedding2_add: shape mismatch");
  if (lk_hip_embedding_f32(P<float>(a, 0), P<int64_t>(a, 1), P<float>(a, 2), P<int64_t>(a, 3), P<float>(a, 4), n, d,
                           v, v2, ctx.stream))
    ctx.error = "embedding2_add: launch failed";
}

// argmax_f32_gpu(x[R, N]) -> i64[R]
void runArgmax(ExecCtx& ctx, const KernelArgs& a) {
  if (lk_hip_argmax_f32(P<float>(a, 0), P<int64_t>(a, 1), a.ints[0], a.ints[1], ctx.stream))
    ctx.error = "argmax: launch failed";
}

}  // namespace

void registerFrontendKernels() {
  const Device G = Device::Gpu;
  registerKernel({"embedding_f32_gpu", G, runEmbedding, 2, 1});
  registerKernel({"embedding2_add_f32_gpu", G, runEmbedding2, 4, 1});
  registerKernel({"argmax_f32_gpu", G, runArgmax, 1, 1});
}

}  // namespace lkh
