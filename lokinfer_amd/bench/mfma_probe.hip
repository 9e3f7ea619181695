// Bench-only measurement kernel, built into its own library (lokinfer_amd/bench/libmfma_probe.so), not into the
// product library or its registry. No counterpart in the reference: the register-only f32 MFMA rate of this GPU under load, the
// ceiling the roofline fraction of an MFMA-bound kernel is read against (the published peak assumes the full
// 2.4 GHz clock, which a chip-wide MFMA load does not hold).
//
//   lk_hip_mfma_f32_probe   each wave runs `iters` rounds of 8 independent 32x32x2 f32 MFMA chains on register data
//                           (8 x 4096 FLOP per round), then writes one sum per lane so nothing is eliminated
#include <hip/hip_runtime.h>

namespace lkd {

typedef float p16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfmaProbeKernel(float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  const float a = 1.0f + 1e-7f * static_cast<float>(lane), b = 1.0f - 1e-7f * static_cast<float>(lane);
  p16f acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  out[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = s;
}

}  // namespace lkd

extern "C" {

// out f32[workgroups * 256]; FLOPs = workgroups * 4 waves * iters * 8 * 4096
int lk_hip_mfma_f32_probe(float* out, int iters, int workgroups, void* stream) {
  if (iters <= 0 || workgroups <= 0) return 1;
  hipLaunchKernelGGL(lkd::mfmaProbeKernel, dim3(static_cast<unsigned>(workgroups)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, iters);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
