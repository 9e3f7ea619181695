// Token-rate front-end kernels on the GPU. The reference runs these as host CPU kernels inside its GPU graphs
// (embedding_f32_cpu, kernels/cpu/kokoro_norm.cpp; argmax in Python, models/gpt2.py:348-359); here they stay
// on the device so that a decode step or a forward is one captured graph with no host round trips.
//
//   lk_hip_embedding_f32   out[i] = table[ids[i]] (+ table2[ids2[i]])   ids out of range -> row of NaN, and the
//                          GPU's error record gets LK_DEVERR_INDEX with the id
//   lk_hip_argmax_f32      per row: index of the first maximum (int64)
//   lk_hip_arange_offset_i64  out[i] = pos[0] + i (position ids of a chunk of new tokens; reference host kernel
//                          arange_offset_i64_cpu, kernels/cpu/decode.cpp:221, python/lokinfer/ops/transformer.py:272-282)
#include "common.h"
#include "lokinfer_hip.h"

namespace lkd {

__global__ void embeddingKernel(const float* __restrict__ table, const int64_t* __restrict__ ids,
                                const float* __restrict__ table2, const int64_t* __restrict__ ids2,
                                float* __restrict__ out, int64_t n, int64_t d, int64_t rows, int64_t rows2,
                                unsigned long long* err) {
  const int64_t total = n * d;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d, c = i - r * d;
    const int64_t id = ids[r];
    const bool ok = id >= 0 && id < rows;
    float v = ok ? table[id * d + c] : __builtin_nanf("");
    if (!ok && c == 0) raiseDeviceError(err, LK_DEVERR_INDEX, id);
    if (table2) {
      const int64_t id2 = ids2[r];
      const bool ok2 = id2 >= 0 && id2 < rows2;
      v += ok2 ? table2[id2 * d + c] : __builtin_nanf("");
      if (!ok2 && c == 0) raiseDeviceError(err, LK_DEVERR_INDEX, id2);
    }
    out[i] = v;
  }
}

// Two launches: workgroup (c, r) reduces chunk c of row r to (value, index) with ties to the lower index
// (numpy / torch argmax semantics) into the workspace; then one workgroup per row reduces the chunks in order.
// mode 0: x is the row data (chunked); mode 1: x is the [rows][chunks] partial values, idx the partial indices.
__global__ __launch_bounds__(256) void argmaxKernel(const float* __restrict__ x, const int64_t* __restrict__ idxIn,
                                                   float* __restrict__ pv, int64_t* __restrict__ pi,
                                                   int64_t* __restrict__ out, int64_t n, int64_t chunk) {
  __shared__ float sv[4];
  __shared__ int64_t si[4];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t c1 = min<int64_t>(n, c0 + chunk);
  const float* row = x + static_cast<int64_t>(blockIdx.y) * n;
  const int64_t* irow = idxIn ? idxIn + static_cast<int64_t>(blockIdx.y) * n : nullptr;
  float best = -INFINITY;
  int64_t bi = INT64_MAX;
  for (int64_t i = c0 + threadIdx.x; i < c1; i += 256) {
    const float v = row[i];
    const int64_t gi = irow ? irow[i] : i;
    if (v > best || (!(v < best) && gi < bi)) {
      best = v;
      bi = gi;
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
    if (out) {
      out[blockIdx.y] = bi == INT64_MAX ? 0 : bi;
    } else {
      pv[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = best;
      pi[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = bi;
    }
  }
}

__global__ void arangeOffsetKernel(const int64_t* __restrict__ pos, int64_t* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = *pos + i;
}

}  // namespace lkd

extern "C" {

int lk_hip_arange_offset_i64(const int64_t* pos, int64_t* out, int64_t n, void* stream) {
  if (n <= 0) return n == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::arangeOffsetKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), pos, out, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_embedding_f32(const float* table, const int64_t* ids, const float* table2, const int64_t* ids2, float* out,
                         int64_t n, int64_t d, int64_t rows, int64_t rows2, void* stream) {
  const int64_t total = n * d;
  if (total <= 0) return total == 0 ? 0 : 1;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(lkd::embeddingKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), table, ids, table2, ids2, out, n, d, rows, rows2,
                     lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_argmax_pairs_f32(const float* values, const int64_t* indices, int64_t* out, int64_t n, void* stream) {
  if (n <= 0) return 1;
  hipLaunchKernelGGL(lkd::argmaxKernel, dim3(1, 1), dim3(256), 0, static_cast<hipStream_t>(stream), values, indices,
                     nullptr, nullptr, out, n, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_argmax_f32(const float* x, int64_t* out, int64_t rows, int64_t n, void* workspace,
                      int64_t workspaceBytes, void* stream) {
  if (rows <= 0 || n <= 0) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t chunk = 2048;
  const int64_t chunks = (n + chunk - 1) / chunk;
  if (chunks == 1 || !workspace || workspaceBytes < rows * chunks * 16) {
    hipLaunchKernelGGL(lkd::argmaxKernel, dim3(1, static_cast<unsigned>(rows)), dim3(256), 0, s, x, nullptr, nullptr,
                       nullptr, out, n, n);
    return hipGetLastError() == hipSuccess ? 0 : 2;
  }
  float* pv = static_cast<float*>(workspace);
  int64_t* pi = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + ((rows * chunks * 4 + 255) / 256) * 256);
  hipLaunchKernelGGL(lkd::argmaxKernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), dim3(256), 0,
                     s, x, nullptr, pv, pi, nullptr, n, chunk);
  hipLaunchKernelGGL(lkd::argmaxKernel, dim3(1, static_cast<unsigned>(rows)), dim3(256), 0, s, pv, pi, nullptr,
                     nullptr, out, chunks, chunks);
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
  if (lk_hip_argmax_f32(P<float>(a, 0), P<int64_t>(a, 1), a.ints[0], a.ints[1], ctx.workspace,
                        static_cast<int64_t>(ctx.workspaceBytes), ctx.stream))
    ctx.error = "argmax: launch failed";
}

// arange_offset_i64_gpu(pos i64[1]) -> i64[length]; attr length
void runArangeOffset(ExecCtx& ctx, const KernelArgs& a) {
  LK_REQUIRE(ctx, a.ints[0] == 1, "arange_offset: pos must be i64[1]");
  if (lk_hip_arange_offset_i64(P<int64_t>(a, 0), P<int64_t>(a, 1), a.ints[1], ctx.stream))
    ctx.error = "arange_offset: launch failed";
}

}  // namespace

void registerFrontendKernels() {
  const Device G = Device::Gpu;
  registerKernel({"embedding_f32_gpu", G, runEmbedding, 2, 1});
  registerKernel({"embedding2_add_f32_gpu", G, runEmbedding2, 4, 1});
  registerKernel({"argmax_f32_gpu", G, runArgmax, 1, 1});
  registerKernel({"arange_offset_i64_gpu", G, runArangeOffset, 1, 1});
}

}  // namespace lkh
