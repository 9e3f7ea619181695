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

#include <cstddef>
#include <cstdint>
#include <string>

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
// nullptr when no kernel has this name
const KernelEntry* findKernel(const std::string& name);
// sets the message lk_last_error() returns on this thread
void setLastError(std::string msg);
// device address of the current GPU's error record {code, detail} (nullptr if it cannot be resolved)
unsigned long long* deviceErrorRecord();

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
void registerF16Kernels();

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

// Sequential reader over KernelArgs::ints (operand dims, out dims, then int attrs).
struct Ints {
  const KernelArgs& a;
  uint32_t i = 0;
  explicit Ints(const KernelArgs& args) : a(args) {}
  int64_t next() { return i < a.numInts ? a.ints[i++] : 0; }
  void skip(int n) { i += n; }
};

// float attr i (attribute-name order), or dflt when absent
inline float F(const KernelArgs& a, uint32_t i, float dflt = 0.0f) {
  return i < a.numFloats ? static_cast<float>(a.floats[i]) : dflt;
}

// records a launcher's nonzero return code as the kernel's error (the first one wins)
inline void status(ExecCtx& ctx, int rc, const char* what) {
  if (rc != 0 && !ctx.error) ctx.error = what;
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

// Records a data error in the GPU's error record (lkh::deviceErrorRecord); the first error of a run is kept.
__device__ __forceinline__ void raiseDeviceError(unsigned long long* rec, unsigned code, long long detail) {
  if (rec && atomicCAS(rec, 0ull, static_cast<unsigned long long>(code)) == 0ull)
    rec[1] = static_cast<unsigned long long>(detail);
}

constexpr float kLog2e = 1.44269504088896341f;

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

// Reductions over a row of 16 lanes by DPP moves (no LDS round trip): quad xor 1, quad xor 2, half-row mirror
// (quads 0 <-> 1, 2 <-> 3), row mirror (half-rows). Each step adds a lane's value to its partner's, so every lane of
// the row ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dppMov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rowSum16(float v) {
  v += dppMov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dppMov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dppMov<0x141>(v);  // row_half_mirror
  v += dppMov<0x140>(v);  // row_mirror
  return v;
}
// Combines the 4 rows of a wave, (r0 + r1) + (r2 + r3) in every lane, by the permlane swaps of rows and halves.
__device__ __forceinline__ float crossRowSum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}
__device__ __forceinline__ float crossRowMax(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

// Wave-wide sum / max with the same bits in every lane, by DPP and permlane swaps.
__device__ __forceinline__ float waveSumDpp(float v) { return crossRowSum(rowSum16(v)); }
__device__ __forceinline__ float waveMaxDpp(float v) {
  v = fmaxf(v, dppMov<0xB1>(v));
  v = fmaxf(v, dppMov<0x4E>(v));
  v = fmaxf(v, dppMov<0x141>(v));
  v = fmaxf(v, dppMov<0x140>(v));
  return crossRowMax(v);
}

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

// torch's gelu(approximate="tanh") in torch's op order: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float geluTanh(float v) {
  const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.0f + tanhf(inner));
}

// Work item (x, y, z) of this workgroup in an XCD-aware order. Workgroups go to the 8 XCDs round-robin by linear
// id L, so L runs on XCD L % 8 as that XCD's (L / 8)-th workgroup. Here XCD c owns the contiguous range of work
// items [c per + min(c, rem), ...) (per = total / 8, rem = total % 8; a bijection on 0 .. total - 1) with work
// item w = x + gx (y + gy z): neighbouring x (the column blocks that read the same input rows) share one L2.
struct GridItem {
  int x, y, z;
};
__device__ __forceinline__ GridItem xcdOrder() {
  const unsigned gx = gridDim.x, gy = gridDim.y;
  const unsigned total = gx * gy * gridDim.z;
  const unsigned l = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const unsigned per = total / 8, rem = total % 8, xcd = l % 8, k = l / 8;
  const unsigned w = xcd * per + min(xcd, rem) + k;
  return GridItem{static_cast<int>(w % gx), static_cast<int>((w / gx) % gy), static_cast<int>(w / (gx * gy))};
}
// The same with y fastest (w = y + gy (x + gx z)): neighbouring row blocks, which read the same B columns, share
// one L2. The better order for a GEMM whose B is larger than its A.
__device__ __forceinline__ GridItem xcdOrderYFast() {
  const unsigned gx = gridDim.x, gy = gridDim.y;
  const unsigned total = gx * gy * gridDim.z;
  const unsigned l = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const unsigned per = total / 8, rem = total % 8, xcd = l % 8, k = l / 8;
  const unsigned w = xcd * per + min(xcd, rem) + k;
  return GridItem{static_cast<int>((w / gy) % gx), static_cast<int>(w % gy), static_cast<int>(w / (gx * gy))};
}

// AdaIN affine af [3, C] = (mean, (1 + g) / sqrt(var + eps), b) from per-chunk (mean, M2) statistics st [S, C, 2]
// of an L-row tensor; gb [2 creal]; channels >= creal get 0. Chunk i = (rho, y) = (i / chunks, i % chunks) holds
// the rows of residue class rho of the dilation d from 128 y on: n_i = clamp(ceil((L - rho) / d) - 128 y, 0, 128)
// rows (d = 1: the plain 128-row chunks; chunks with no rows are never read). Instance norm with a biased
// variance, combined in one pass in double around a shift K (the channel's first chunk mean, so the sums carry
// deviations, not the mean's magnitude): S1 = sum n_i (m_i - K), S2 = sum (M2_i + n_i (m_i - K)^2);
// mean = K + S1 / L, M2 = S2 - S1^2 / L, var = M2 / L.
// Workgroup of 256 = 4 channels x 64 chunk slices. The workgroup is kept small on purpose: the kernel sits on the
// dependency chain between two convs while long conv kernels of other branches hold most of the chip, and a
// workgroup only starts once a CU has its resources free; 256 threads fit in the slot a retiring conv workgroup
// leaves (a 1024-thread form waited for up to 0.9 ms there). A slice's chunk loads are independent and issued in
// batches of 12, so a slice takes a few load round trips even at the generator's ~2300 chunks per channel. The 64
// slices combine by wave shuffles (16 per wave), then the 4 wave partials in LDS, in a fixed order.
constexpr int kAffineCh = 4;
constexpr int kAffineThreads = 256;
__device__ __forceinline__ void adainAffineSlices(const float* __restrict__ st, const float* __restrict__ gb,
                                                  float* __restrict__ af, int64_t l, int64_t c, int d,
                                                  int64_t chunks, int64_t creal, float eps) {
  constexpr int SL = kAffineThreads / kAffineCh;  // 64 slices
  constexpr int B = 12;                           // loads in flight per thread
  __shared__ double red[2][kAffineThreads / 64][kAffineCh];
  const int cl = threadIdx.x % kAffineCh, sl = threadIdx.x / kAffineCh, wave = threadIdx.x >> 6;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * kAffineCh + cl;
  const bool live = ch < creal && ch < c;
  const int total = static_cast<int>(static_cast<int64_t>(d) * chunks);
  const int ichunks = static_cast<int>(chunks);
  const float2* sp = reinterpret_cast<const float2*>(st) + (live ? ch : 0);
  const double shift = live ? static_cast<double>(sp[0].x) : 0.0;
  double s1 = 0.0, s2 = 0.0;
  if (live) {
    for (int i0 = sl; i0 < total; i0 += SL * B) {
      float2 v[B];
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * SL;
        v[b] = i < total ? sp[static_cast<int64_t>(i) * c] : make_float2(0.0f, 0.0f);
      }
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * SL;
        const int rho = i / ichunks, yy = i - rho * ichunks;
        const int64_t lr = rho < l ? (l - rho + d - 1) / d : 0;
        const int64_t n = min<int64_t>(max<int64_t>(lr - static_cast<int64_t>(yy) * 128, 0), 128);
        if (i < total && n > 0) {
          const double dn = static_cast<double>(n), dm = static_cast<double>(v[b].x) - shift;
          s1 += dn * dm;
          s2 += static_cast<double>(v[b].y) + dn * dm * dm;
        }
      }
    }
  }
  // the wave's 16 slices of each channel: lanes cl + 4 k
#pragma unroll
  for (int off = kAffineCh; off < 64; off <<= 1) {
    s1 += __shfl_xor(s1, off, 64);
    s2 += __shfl_xor(s2, off, 64);
  }
  if ((threadIdx.x & 63) < kAffineCh) {
    red[0][wave][cl] = s1;
    red[1][wave][cl] = s2;
  }
  __syncthreads();
  if (threadIdx.x < kAffineCh && ch < c) {
    if (!live) {
      af[ch] = af[c + ch] = af[2 * c + ch] = 0.0f;
    } else {
      double t1 = 0.0, t2 = 0.0;
      for (int w = 0; w < kAffineThreads / 64; ++w) {
        t1 += red[0][w][cl];
        t2 += red[1][w][cl];
      }
      const double dl = static_cast<double>(l);
      const double m2 = t2 - t1 * t1 / dl;
      const float var = static_cast<float>(max(m2, 0.0) / dl);
      af[ch] = static_cast<float>(shift + t1 / dl);
      af[c + ch] = (1.0f + gb[ch]) / sqrtf(var + eps);
      af[2 * c + ch] = gb[creal + ch];
    }
  }
}

}  // namespace lkd
