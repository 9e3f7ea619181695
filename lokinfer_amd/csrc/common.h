// Shared definitions for the gfx950 kernels and the kernel registry.
//
// Kernel ABI (the same argument convention as the reference's registry,
// include/lokinfer/runtime/kernel.h:1-11 in lariaus/lokinfer):
//   ptrs   : operands in order, then outs in order (device pointers)
//   ints   : every operand's shape dims, then every out's shape dims, then
//            int/bool/int-list attrs in attribute-name order
//   floats : float attrs in attribute-name order
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstddef>

namespace lkh {

// Reference: BufRef {void* mtlBuffer; uint64_t offset} (kernel.h:26-29); on HIP
// the buffer is a plain device pointer.
struct BufRef {
  void* devPtr;
  uint64_t offset;
};

struct KernelArgs {
  void* const* ptrs;
  const BufRef* bufs;  // may be null: ptrs already carry the offset
  const int64_t* ints;
  const double* floats;
  const void* state;
  uint32_t numPtrs;
  uint32_t numInts;
  uint32_t numFloats;
};

// Per-call execution context (reference ExecCtx, kernel.h:41-47): the HIP stream
// every kernel of the call is enqueued on, a caller-owned device workspace for
// kernels that need partial results, and a static error string a kernel sets on
// invalid input instead of producing garbage.
struct ExecCtx {
  hipStream_t stream = nullptr;
  void* workspace = nullptr;
  size_t workspaceBytes = 0;
  const char* error = nullptr;
};

enum class Device : uint8_t { Cpu = 0, Gpu = 1 };

using RunFn = void (*)(ExecCtx&, const KernelArgs&);

struct KernelEntry {
  const char* name;
  Device device;
  RunFn run;
  int numOperands;  // -1: variadic / checked by the kernel
  int numOuts;
};

void registerKernel(const KernelEntry& e);

// Each kernel family registers its entries from one of these (explicit, no
// static constructors).
void registerGemmKernels();
void registerTransformerKernels();
void registerKokoroKernels();
void registerFrontendKernels();
void registerSequenceKernels();
void registerSignalKernels();
void registerDecodeFusedKernels();
void registerWinogradKernels();

inline unsigned ceilDiv(int64_t a, int64_t b) { return static_cast<unsigned>((a + b - 1) / b); }

template <typename T>
inline T* P(const KernelArgs& a, int i) {
  return static_cast<T*>(a.ptrs[i]);
}

// Sets ctx.error if a launch failed (invalid configuration etc.).
inline void checkLaunch(ExecCtx& ctx) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess && !ctx.error) ctx.error = hipGetErrorString(e);
}

#define LK_REQUIRE(ctx, cond, msg) \
  do {                             \
    if (!(cond)) {                 \
      (ctx).error = (msg);         \
      return;                      \
    }                              \
  } while (0)

}  // namespace lkh

// ---- device helpers ---------------------------------------------------------------------------------------
namespace lkd {

__device__ __forceinline__ float waveSum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float waveMax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// torch's gelu(approximate="tanh") in torch's op order: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
// sin(y)^2 for the Snake activation x + sin(a x)^2 / a. sin^2 has period pi, so y is reduced to
// r = y - n pi, |r| <= pi / 2, by Cody-Waite with pi split into its nearest float and the remainder
// (pi - 3.14159274f = -8.74227766e-8f), each product formed by one fma; sin(r) then comes from the hardware
// sine (argument in revolutions), whose absolute error on |r| <= pi / 2 is a few 1e-7. About 7 VALU
// instructions instead of the general-range sinf.
__device__ __forceinline__ float snakeSinSq(float y) {
  const float n = rintf(y * 0.318309886183790672f);
  float r = fmaf(-n, 3.14159274101257324f, y);
  r = fmaf(-n, -8.74227766e-8f, r);
  const float sn = __builtin_amdgcn_sinf(r * 0.159154943091895336f);
  return sn * sn;
}

__device__ __forceinline__ float geluTanh(float v) {
  const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.0f + tanhf(inner));
}

}  // namespace lkd
