// f16 kernels of the Qwen3(-ASR) language model: the reference's f16 GPU op family (kernels/gpu/f16_gpu.cpp:1011-1050,
// op contracts python/lokinfer/ops/f16.py and f16_gpu.py in lariaus/lokinfer). f16 storage, f32 math and
// accumulation, one rounding to f16 at each op's output (the contract's "basic" roundings where an op is a fused
// composition: rmsnorm rounds h = x·r, then g·h).
//
//   lk_hip_f16_gemm              x f16[M, K] @ W (packed W^T f16[N', K]) with epilogues: plain, + bias, + residual,
//                                SwiGLU over [gate | up] (gemm[_bias]_f16_gpu, gemm[_add|_swiglu]_opt_f16_gpu).
//                                M = 1: a bandwidth-bound GEMV (two weight rows per wave); M > 1: f16 MFMA
//                                (32x32x16) tiles of 64 x 128, split-K across workgroups when the grid is small.
//   lk_hip_f16_rms_gemm          rmsnorm(x, g) @ W [+ SwiGLU] (rmsnorm_gemm[_swiglu]_opt_f16_gpu): M = 1 one GEMV
//                                whose waves normalize the row themselves; M > 1 the row kernel into the workspace
//                                operand, then the GEMM.
//   lk_hip_f16_lm_head           x[T-1] @ table f16[V, D]^T -> f32[1, V] (lm_head_last[_opt]_f16_gpu)
//   lk_hip_f16_rmsnorm           rows or heads (rmsnorm[_heads]_f16_gpu)
//   lk_hip_f16_rope              rotate_half RoPE per 128-wide head at positions pos + i (rope_f16_gpu)
//   lk_hip_f16_qknorm_rope_kv    QK-norm + RoPE of q and k, k and v into the caches (qknorm_rope_kv_opt_f16_gpu)
//   lk_hip_f16_attention_gqa     causal GQA over the caches (attention_gqa[_opt]_f16_gpu): T = 1 key-split chunks +
//                                merge; T > 1 flash tiles on MFMA (f16 operands for q.k, P split into two f16 parts
//                                for P.V so the softmax weights keep f32 precision)
//   lk_hip_f16_kv_write, lk_hip_f16_embedding, lk_hip_f16_scatter_audio, lk_hip_f16_elementwise (add, silu_mul),
//   lk_hip_f16_transpose (weight packing)
//
// Every kernel that normalizes a row reduces its sum of squares in one order (rowSumSq: a wave, lane l taking the
// 8-value chunks l, l + 64, ..., then a butterfly), so the fused GEMV prologue, the row kernel and the QK-norm give
// identical bits.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "common.h"
#include "lokinfer_hip.h"

// No fp contraction in this file (every intended fma below is an explicit fmaf).
#pragma clang fp contract(off)

namespace lkd {

typedef _Float16 h16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));


// The contract's output rounding: the f32 result, then f16. The empty asm makes the f32 value opaque, so the compiler
// cannot fold the operation producing it and the conversion into one mixed-precision instruction (v_fma_mix*),
// which rounds once, straight to f16, and differs near f16 midpoints; fused ops and their compositions then round
// alike.
__device__ __forceinline__ h16 toH16(float v) {
  asm volatile("" : "+v"(v));
  return static_cast<h16>(v);
}

__device__ __forceinline__ half8 ld8(const h16* p) { return *reinterpret_cast<const half8*>(p); }
// weight rows streamed once per call (decode GEMVs: gigabytes per token, far above the last-level cache)
__device__ __forceinline__ half8 ldStream8(const h16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const half8*>(p));
}
__device__ __forceinline__ void st8(h16* p, half8 v) { *reinterpret_cast<half8*>(p) = v; }

// Sum of squares of a row of k values (k % 8 == 0, 16-byte aligned) over one wave.
__device__ __forceinline__ float rowSumSq(const h16* x, int64_t k, int lane) {
  float s = 0.0f;
  for (int64_t c = lane; c < k / 8; c += 64) {
    const half8 v = ld8(x + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf(static_cast<float>(v[e]), static_cast<float>(v[e]), s);
  }
  return waveSum(s);
}

__device__ __forceinline__ float rmsFactor(float sumSq, int64_t k, float eps) {
  return 1.0f / sqrtf(sumSq / static_cast<float>(k) + eps);
}

// HF Qwen3RMSNorm with the contract's roundings: h = f16(x r), y = f16(g h)
__device__ __forceinline__ h16 rmsElem(h16 x, h16 g, float r) {
  const h16 h = toH16(static_cast<float>(x) * r);
  return toH16(static_cast<float>(g) * static_cast<float>(h));
}

// ---- RMSNorm over groups of `width` values (rows, or heads), one wave per group ----------------------------
template <int W>  // W > 0: width == W, the lane's W / 512 chunks of x and g loaded once, in rowSumSq's order
__global__ __launch_bounds__(256) void rmsGroupsKernel(const h16* __restrict__ x, const h16* __restrict__ g,
                                                       h16* __restrict__ out, int64_t groups, int64_t width,
                                                       float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grp >= groups) return;
  const h16* xr = x + grp * width;
  h16* o = out + grp * width;
  if constexpr (W > 0) {
    constexpr int C = W / 512;
    half8 v[C], gv[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      v[i] = ld8(xr + 8 * (lane + 64 * i));
      gv[i] = ld8(g + 8 * (lane + 64 * i));
    }
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < C; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) sq = fmaf(static_cast<float>(v[i][e]), static_cast<float>(v[i][e]), sq);
    const float r = rmsFactor(waveSum(sq), W, eps);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      half8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = rmsElem(v[i][e], gv[i][e], r);
      st8(o + 8 * (lane + 64 * i), y);
    }
  } else {
    const float r = rmsFactor(rowSumSq(xr, width, lane), width, eps);
    for (int64_t c = lane; c < width / 8; c += 64) {
      const half8 v = ld8(xr + 8 * c), gv = ld8(g + 8 * c);
      half8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = rmsElem(v[e], gv[e], r);
      st8(o + 8 * c, y);
    }
  }
}

// ---- RoPE: angle = f32(p) * invFreq[j] (f32 product), cos / sin of it in double, rounded to f32 ------------
struct RopeTable {
  float invf[64];
};

__device__ __forceinline__ void ropePair(float lo, float hi, int64_t p, float invf, h16& olo, h16& ohi) {
  const float ang = static_cast<float>(p) * invf;
  double sd, cd;
  sincos(static_cast<double>(ang), &sd, &cd);  // one routine in every kernel (the compiler may merge sin + cos)
  const float c = static_cast<float>(cd), s = static_cast<float>(sd);
  // explicit fma forms: every kernel that rotates computes the same bits (no contraction choice left to the
  // compiler, which could fuse either product)
  olo = toH16(fmaf(lo, c, -(hi * s)));
  ohi = toH16(fmaf(hi, c, lo * s));
}

// one wave per (row, 128-wide head); lane j rotates the pair (j, j + 64)
__global__ __launch_bounds__(256) void ropeKernel(const h16* __restrict__ x, const int64_t* __restrict__ pos,
                                                  h16* __restrict__ out, int64_t t, int64_t c, RopeTable tab) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t heads = c / 128;
  if (item >= t * heads) return;
  const int64_t row = item / heads, h0 = (item - row * heads) * 128;
  const int64_t p0 = *pos;
  const h16* xr = x + row * c + h0;
  h16* o = out + row * c + h0;
  h16 a, b;
  ropePair(static_cast<float>(xr[lane]), static_cast<float>(xr[lane + 64]), p0 + row, tab.invf[lane], a, b);
  o[lane] = a;
  o[lane + 64] = b;
}

// ---- QK-norm + RoPE + KV write: one wave per (row, head slot). Slots 0..qh-1: q heads (normalized, rotated,
// to qOut); qh..qh+kvh-1: k heads (normalized, rotated, to the K cache row pos + row); then v heads (copied to the
// V cache row). Rows at or past the cache's end are not written.
struct QkrParams {
  const h16* qkv;
  const h16* qg;
  const h16* kg;
  const int64_t* pos;
  h16* kc;
  h16* vc;
  h16* q;
  int64_t t, cap;
  int qh, kvh;
  float eps;
  RopeTable tab;
};

__global__ __launch_bounds__(256) void qkRopeKvKernel(QkrParams p) {
  const int lane = threadIdx.x & 63;
  const int slots = p.qh + 2 * p.kvh;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= p.t * slots) return;
  const int64_t row = item / slots;
  const int slot = static_cast<int>(item - row * slots);
  const int64_t dq = static_cast<int64_t>(p.qh) * 128, dk = static_cast<int64_t>(p.kvh) * 128;
  const int64_t width = dq + 2 * dk;
  const int64_t prow = *p.pos + row;
  const bool inCache = prow >= 0 && prow < p.cap;
  const h16* xr;
  if (slot < p.qh) xr = p.qkv + row * width + slot * 128;
  else if (slot < p.qh + p.kvh) xr = p.qkv + row * width + dq + (slot - p.qh) * 128;
  else {
    if (!inCache) return;
    const int vh = slot - p.qh - p.kvh;
    const h16* vr = p.qkv + row * width + dq + dk + vh * 128;
    h16* o = p.vc + prow * dk + vh * 128;
    o[lane] = vr[lane];
    o[lane + 64] = vr[lane + 64];
    return;
  }
  const bool isQ = slot < p.qh;
  const h16* g = isQ ? p.qg : p.kg;
  const float r = rmsFactor(rowSumSq(xr, 128, lane), 128, p.eps);
  const h16 lo = rmsElem(xr[lane], g[lane], r), hi = rmsElem(xr[lane + 64], g[lane + 64], r);
  h16 a, b;
  ropePair(static_cast<float>(lo), static_cast<float>(hi), prow, p.tab.invf[lane], a, b);
  h16* o;
  if (isQ) {
    o = p.q + row * dq + slot * 128;
  } else {
    if (!inCache) return;
    o = p.kc + prow * dk + (slot - p.qh) * 128;
  }
  o[lane] = a;
  o[lane + 64] = b;
}

// ---- GEMV (M = 1) over a packed weight W^T [rows, K]: two weight rows per wave ---------------------------------
enum : int { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_F32 = 2 };

struct GemvF16Params {
  const h16* x;      // the activation row [K]
  const h16* gamma;  // RMSNorm gain [K] (prologue) or null
  const h16* wt;     // W^T [rows, K]
  const h16* bias;   // [N] or null
  const h16* res;    // [N] or null
  void* out;         // f16 [N] (f32 for EPI_F32)
  int64_t n, k;
  float eps;
};

__device__ __forceinline__ float siluMul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// CH > 0: K == 512 CH, and every lane's CH chunks of both rows are loaded before any math (the x chunks first: the
// in-order memory counter then lets the RMS statistics wait for x alone while the weights stream in). The statistics
// use rowSumSq's order (the lane's chunks ascending, then the butterfly), so the prologue matches the row kernel
// bit for bit. CH = 0: any K % 8 == 0, chunk by chunk.
template <int EPI, bool RMS, int CH>
__global__ __launch_bounds__(256) void gemvF16Kernel(GemvF16Params p) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  int64_t r0, r1;
  if constexpr (EPI == EPI_SWIGLU) {
    if (wv >= p.n) return;
    r0 = wv;
    r1 = p.n + wv;
  } else {
    r0 = 2 * wv;
    if (r0 >= p.n) return;
    r1 = min<int64_t>(r0 + 1, p.n - 1);
  }
  const h16* w0 = p.wt + r0 * p.k;
  const h16* w1 = p.wt + r1 * p.k;
  float a0 = 0.0f, a1 = 0.0f;
  auto dot = [&](half8 xv, const half8& u, const half8& v, int64_t c, float r) {
    if constexpr (RMS) {
      const half8 gv = ld8(p.gamma + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = rmsElem(xv[e], gv[e], r);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xf = static_cast<float>(xv[e]);
      a0 = fmaf(xf, static_cast<float>(u[e]), a0);
      a1 = fmaf(xf, static_cast<float>(v[e]), a1);
    }
  };
  if constexpr (CH > 0) {
    half8 xs[CH], u[CH], v[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) xs[j] = ld8(p.x + 8 * (lane + 64 * j));
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      u[j] = ldStream8(w0 + 8 * (lane + 64 * j));
      v[j] = ldStream8(w1 + 8 * (lane + 64 * j));
    }
    float r = 1.0f;
    if constexpr (RMS) {
      float sq = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) sq = fmaf(static_cast<float>(xs[j][e]), static_cast<float>(xs[j][e]), sq);
      r = rmsFactor(waveSum(sq), p.k, p.eps);
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) dot(xs[j], u[j], v[j], lane + 64 * j, r);
  } else {
    float r = 1.0f;
    if constexpr (RMS) r = rmsFactor(rowSumSq(p.x, p.k, lane), p.k, p.eps);
    const int64_t chunks = p.k / 8, full = chunks / 64;
#pragma unroll 4
    for (int64_t i = 0; i < full; ++i) {
      const int64_t c = lane + 64 * i;
      dot(ld8(p.x + 8 * c), ldStream8(w0 + 8 * c), ldStream8(w1 + 8 * c), c, r);
    }
    if (lane + 64 * full < chunks) {
      const int64_t c = lane + 64 * full;
      dot(ld8(p.x + 8 * c), ldStream8(w0 + 8 * c), ldStream8(w1 + 8 * c), c, r);
    }
  }
  a0 = waveSum(a0);
  a1 = waveSum(a1);
  if (lane != 0) return;
  if constexpr (EPI == EPI_F32) {
    float* o = static_cast<float*>(p.out);
    o[r0] = a0;
    if (r1 != r0) o[r1] = a1;
  } else if constexpr (EPI == EPI_SWIGLU) {
    static_cast<h16*>(p.out)[wv] = toH16(siluMul(a0, a1));
  } else {
    h16* o = static_cast<h16*>(p.out);
    float y0 = a0, y1 = a1;
    if (p.bias) {
      y0 += static_cast<float>(p.bias[r0]);
      y1 += static_cast<float>(p.bias[r1]);
    }
    if (p.res) {
      y0 = static_cast<float>(p.res[r0]) + y0;
      y1 = static_cast<float>(p.res[r1]) + y1;
    }
    o[r0] = toH16(y0);
    if (r1 != r0) o[r1] = toH16(y1);
  }
}

// launches the GEMV with the chunk count fixed at compile time for K = 2048 and 6144 (Qwen3's inner sizes)
template <int EPI, bool RMS>
void launchGemvF16(const GemvF16Params& p, unsigned blocks, hipStream_t s) {
  if (p.k == 2048)
    hipLaunchKernelGGL((gemvF16Kernel<EPI, RMS, 4>), dim3(blocks), dim3(256), 0, s, p);
  else if (p.k == 6144)
    hipLaunchKernelGGL((gemvF16Kernel<EPI, RMS, 12>), dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gemvF16Kernel<EPI, RMS, 0>), dim3(blocks), dim3(256), 0, s, p);
}

// ---- GEMM (M > 1) on f16 MFMA 32x32x16 ----------------------------------------------------------------------
// A f16 [M, lda] row-major, B given as W^T [rows, K] (both K-contiguous, so every MFMA operand of a lane is one
// 16-byte run of 8 k). Workgroup tile 64 (M) x 128 (B rows), 4 waves as 2 x 2, each 32 rows x two 32-column blocks
// (the A fragment feeds two MFMAs). K stages of 64 through padded LDS rows (72 halves: the 32 lanes of a fragment
// read hit distinct banks), double-buffered, fed from a ring of four register sets (loads run three stages ahead);
// loads and stores are unconditional (clamped), four stages per loop iteration, the remainder peeled.
// SwiGLU: the tile's B rows are 64 gate rows (W^T rows o0..o0+63) and the 64 matching up rows (N + o0 ..), so a
// wave's two blocks hold gate and up of the same outputs and the epilogue is elementwise in registers.
// Split-K: grid z = split, K range [z kSplit, ...); raw tile sums go to part [split][M][W] (W = N, or 2N with the
// up half at column N + n for SwiGLU) and gemmF16ReduceKernel applies the epilogue.
struct GemmF16Params {
  const h16* a;
  const h16* bt;
  const h16* bias;
  const h16* res;
  h16* c;
  float* part;
  int64_t m, n, k, lda;
  int64_t kSplit;
  int split;
};

constexpr int GBM = 64, GBN = 128, GBK = 64, GLD = GBK + 8;
constexpr int GA = GBM * GBK / 8 / 256, GB = GBN * GBK / 8 / 256;  // 16-byte chunks per thread per stage

template <bool SWIGLU, bool KTAIL>
__global__ __launch_bounds__(256, 2) void gemmF16Kernel(GemmF16Params p) {
  __shared__ __attribute__((aligned(16))) h16 As[2][GBM * GLD];
  __shared__ __attribute__((aligned(16))) h16 Bs[2][GBN * GLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5, wr = wave >> 1, wc = wave & 1;
  const GridItem gi = xcdOrder();
  const int64_t m0 = static_cast<int64_t>(gi.y) * GBM;
  const int64_t kb = p.split > 1 ? gi.z * p.kSplit : 0;
  const int64_t ke = p.split > 1 ? min<int64_t>(kb + p.kSplit, p.k) : p.k;
  // staging: chunk id = tid + 256 i -> tile row id / 8, k offset 8 (id % 8)
  constexpr int CPR = GBK / 8;
  const int sc = (tid % CPR) * 8;
  const h16* ap[GA];
  const h16* bp[GB];
#pragma unroll
  for (int i = 0; i < GA; ++i) ap[i] = p.a + min<int64_t>(m0 + (tid + 256 * i) / CPR, p.m - 1) * p.lda;
#pragma unroll
  for (int i = 0; i < GB; ++i) {
    const int r = (tid + 256 * i) / CPR;
    int64_t row;
    if constexpr (SWIGLU) {
      const int64_t o = min<int64_t>(static_cast<int64_t>(gi.x) * 64 + (r & 63), p.n - 1);
      row = r < 64 ? o : p.n + o;
    } else {
      row = min<int64_t>(static_cast<int64_t>(gi.x) * GBN + r, p.n - 1);
    }
    bp[i] = p.bt + row * p.k;
  }
  // a ring of GD register sets: stage s's tile is loaded into set s % GD while it is GD - 1 stages ahead of the
  // stage whose MFMAs run, so each load has GD - 2 stages of MFMA work to arrive in before its LDS store
  constexpr int GD = 4;
  half8 ra[GD][GA], rb[GD][GB];
  auto gload = [&](int64_t k0, int s) {
    const int64_t kk = min<int64_t>(k0 + sc, ke - 8);
#pragma unroll
    for (int i = 0; i < GA; ++i) ra[s][i] = ld8(ap[i] + kk);
#pragma unroll
    for (int i = 0; i < GB; ++i) rb[s][i] = ld8(bp[i] + kk);
  };
  auto sstore = [&](int buf, int64_t k0, int s) {
    const bool zero = KTAIL && k0 + sc >= ke;
    const half8 z = {};
#pragma unroll
    for (int i = 0; i < GA; ++i) st8(&As[buf][((tid + 256 * i) / CPR) * GLD + sc], zero ? z : ra[s][i]);
#pragma unroll
    for (int i = 0; i < GB; ++i) st8(&Bs[buf][((tid + 256 * i) / CPR) * GLD + sc], zero ? z : rb[s][i]);
  };
  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.0f;
  const int64_t stages = (ke - kb + GBK - 1) / GBK;
  auto kOf = [&](int64_t st) { return kb + min<int64_t>(st, stages - 1) * GBK; };
  // stage st: MFMAs on LDS buffer st & 1; loads stage st + GD - 1 into set (st + GD - 1) % GD; stores stage st + 1
  // from set (st + 1) % GD into the other buffer. Loads past the last stage reload it (unconditional).
  auto stage = [&](int64_t st, int buf, int sLoad, int sStore) {
    constexpr int Q = GBK / 16;
    half8 af[Q], bf0[Q], bf1[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      af[q] = ld8(&As[buf][(32 * wr + lr) * GLD + 16 * q + 8 * lh]);
      bf0[q] = ld8(&Bs[buf][(32 * wc + lr) * GLD + 16 * q + 8 * lh]);
      bf1[q] = ld8(&Bs[buf][(64 + 32 * wc + lr) * GLD + 16 * q + 8 * lh]);
    }
    gload(kOf(st + GD - 1), sLoad);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[q], bf0[q], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[q], bf1[q], acc1, 0, 0, 0);
    }
    sstore(buf ^ 1, kOf(st + 1), sStore);
    __syncthreads();
  };
#pragma unroll
  for (int j = 0; j < GD - 1; ++j) gload(kOf(j), j);
  sstore(0, kb, 0);
  __syncthreads();
  int64_t st = 0;
  for (; st + GD <= stages; st += GD) {
    stage(st, 0, 3, 1);
    stage(st + 1, 1, 0, 2);
    stage(st + 2, 0, 1, 3);
    stage(st + 3, 1, 2, 0);
  }
  if (st < stages) stage(st, 0, 3, 1);
  if (st + 1 < stages) stage(st + 1, 1, 0, 2);
  if (st + 2 < stages) stage(st + 2, 0, 1, 3);
  // accumulator r of a block: row 8 (r / 4) + 4 lh + r % 4 of the wave's 32, column lr of the block
  const int64_t lastRow = p.m - 1;
  if (p.split > 1) {
    const int64_t w = SWIGLU ? 2 * p.n : p.n;
    float* pp = p.part + static_cast<int64_t>(gi.z) * p.m * w;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t gm = m0 + 32 * wr + 8 * (r >> 2) + 4 * lh + (r & 3);
      if (gm > lastRow) continue;
      if constexpr (SWIGLU) {
        const int64_t gn = static_cast<int64_t>(gi.x) * 64 + 32 * wc + lr;
        if (gn < p.n) {
          pp[gm * w + gn] = acc0[r];
          pp[gm * w + p.n + gn] = acc1[r];
        }
      } else {
        const int64_t gn = static_cast<int64_t>(gi.x) * GBN + 32 * wc + lr;
        if (gn < p.n) pp[gm * w + gn] = acc0[r];
        if (gn + 64 < p.n) pp[gm * w + gn + 64] = acc1[r];
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t gm = m0 + 32 * wr + 8 * (r >> 2) + 4 * lh + (r & 3);
    if (gm > lastRow) continue;
    if constexpr (SWIGLU) {
      const int64_t gn = static_cast<int64_t>(gi.x) * 64 + 32 * wc + lr;
      if (gn < p.n) p.c[gm * p.n + gn] = toH16(siluMul(acc0[r], acc1[r]));
    } else {
      const int64_t gn = static_cast<int64_t>(gi.x) * GBN + 32 * wc + lr;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = gn + 64 * j;
        if (col >= p.n) continue;
        float y = j ? acc1[r] : acc0[r];
        if (p.bias) y += static_cast<float>(p.bias[col]);
        if (p.res) y = static_cast<float>(p.res[gm * p.n + col]) + y;
        p.c[gm * p.n + col] = toH16(y);
      }
    }
  }
}

// Wide form (SwiGLU at M >= 256, any GEMM at M >= 1024): workgroup tile 128 (M) x 128 (B rows), 4 waves as 2 x 2,
// each 64 rows x two 32-column blocks (2 x 2 MFMA blocks: every A and B fragment feeds two MFMAs), which halves the
// global and LDS bytes per MFMA against the 64 x 128 tile. Staged K-major through unpadded, XOR-swizzled LDS rows
// from two register sets; B row layout (SwiGLU: 64 gate rows, then the 64 matching up rows), split-K partials and
// epilogues as gemmF16Kernel.
constexpr int WBM = 128, WBN = 128;
constexpr int WA = WBM * GBK / 8 / 256, WB = WBN * GBK / 8 / 256;  // 16-byte chunks per thread per stage

template <bool SWIGLU, bool KTAIL>
__global__ __launch_bounds__(256, 2) void gemmF16WideKernel(GemmF16Params p) {
  // unpadded 64-half rows; 16-byte chunk c of row r at slot c ^ ((r >> 1) & 7): a 16-lane store phase covers two
  // whole rows (all 64 banks) and a fragment read (rows lr of a 32-row block, one chunk each) hits 16 distinct
  // 4-bank groups per phase
  __shared__ __attribute__((aligned(16))) h16 As[2][WBM * GBK];
  __shared__ __attribute__((aligned(16))) h16 Bs[2][WBN * GBK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5, wr = wave >> 1, wc = wave & 1;
  const GridItem gi = xcdOrder();
  const int64_t m0 = static_cast<int64_t>(gi.y) * WBM;
  const int64_t kb = p.split > 1 ? gi.z * p.kSplit : 0;
  const int64_t ke = p.split > 1 ? min<int64_t>(kb + p.kSplit, p.k) : p.k;
  constexpr int CPR = GBK / 8;
  const int sc = (tid % CPR) * 8;
  const h16* ap[WA];
  const h16* bp[WB];
#pragma unroll
  for (int i = 0; i < WA; ++i) ap[i] = p.a + min<int64_t>(m0 + (tid + 256 * i) / CPR, p.m - 1) * p.lda;
#pragma unroll
  for (int i = 0; i < WB; ++i) {
    const int r = (tid + 256 * i) / CPR;
    int64_t row;
    if constexpr (SWIGLU) {
      const int64_t o = min<int64_t>(static_cast<int64_t>(gi.x) * 64 + (r & 63), p.n - 1);
      row = r < 64 ? o : p.n + o;
    } else {
      row = min<int64_t>(static_cast<int64_t>(gi.x) * WBN + r, p.n - 1);
    }
    bp[i] = p.bt + row * p.k;
  }
  // LDS offset (halves) of this thread's i-th staged chunk
  auto swz = [&](int i) {
    const int r = (tid + 256 * i) / CPR, c = tid % CPR;
    return r * GBK + 8 * (c ^ ((r >> 1) & 7));
  };
  // fragment reads: row 32 b + lr of a tile, chunk 2 q + lh -> slot (2 q + lh) ^ ((lr >> 1) & 7)
  int fo[GBK / 16];
#pragma unroll
  for (int q = 0; q < GBK / 16; ++q) fo[q] = lr * GBK + 8 * ((2 * q + lh) ^ ((lr >> 1) & 7));
  // two register sets: stage st + 2's tile is loaded while stage st's MFMAs run; it is stored after stage st + 1's
  // (a deeper ring of four sets measured no faster: 254 VGPRs)
  half8 ra[2][WA], rb[2][WB];
  auto gload = [&](int64_t k0, int s) {
    const int64_t kk = min<int64_t>(k0 + sc, ke - 8);
#pragma unroll
    for (int i = 0; i < WA; ++i) ra[s][i] = ld8(ap[i] + kk);
#pragma unroll
    for (int i = 0; i < WB; ++i) rb[s][i] = ld8(bp[i] + kk);
  };
  auto sstore = [&](int buf, int64_t k0, int s) {
    const bool zero = KTAIL && k0 + sc >= ke;
    const half8 z = {};
#pragma unroll
    for (int i = 0; i < WA; ++i) st8(&As[buf][swz(i)], zero ? z : ra[s][i]);
#pragma unroll
    for (int i = 0; i < WB; ++i) st8(&Bs[buf][swz(i)], zero ? z : rb[s][i]);
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int64_t stages = (ke - kb + GBK - 1) / GBK;
  auto kOf = [&](int64_t st) { return kb + min<int64_t>(st, stages - 1) * GBK; };
  // stage st: MFMAs on LDS buffer st & 1, k step by k step (each step's four fragments read just before its four
  // MFMAs); loads stage st + 2 into set st & 1 (its stage st is in LDS already) and stores stage st + 1 from the
  // other set into the other buffer. Loads past the last stage reload it (unconditional).
  auto stage = [&](int64_t st, int buf, int sLoad, int sStore) {
    constexpr int Q = GBK / 16;
    gload(kOf(st + 2), sLoad);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      half8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = ld8(&As[buf][(64 * wr + 32 * i) * GBK + fo[q]]);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = ld8(&Bs[buf][(64 * j + 32 * wc) * GBK + fo[q]]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    sstore(buf ^ 1, kOf(st + 1), sStore);
    __syncthreads();
  };
  gload(kOf(0), 0);
  gload(kOf(1), 1);
  sstore(0, kb, 0);
  __syncthreads();
  // set roles alternate: stage st loads into set st & 1 and stores from set (st + 1) & 1
  int64_t st = 0;
  for (; st + 2 <= stages; st += 2) {
    stage(st, 0, 0, 1);
    stage(st + 1, 1, 1, 0);
  }
  if (st < stages) stage(st, 0, 0, 1);
  // accumulator r of block (i, j): row 64 wr + 32 i + 8 (r / 4) + 4 lh + r % 4, column lr of B block j
  const int64_t lastRow = p.m - 1;
  if (p.split > 1) {
    const int64_t w = SWIGLU ? 2 * p.n : p.n;
    float* pp = p.part + static_cast<int64_t>(gi.z) * p.m * w;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gm = m0 + 64 * wr + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (gm > lastRow) continue;
        if constexpr (SWIGLU) {
          const int64_t gn = static_cast<int64_t>(gi.x) * 64 + 32 * wc + lr;
          if (gn < p.n) {
            pp[gm * w + gn] = acc[i][0][r];
            pp[gm * w + p.n + gn] = acc[i][1][r];
          }
        } else {
          const int64_t gn = static_cast<int64_t>(gi.x) * WBN + 32 * wc + lr;
          if (gn < p.n) pp[gm * w + gn] = acc[i][0][r];
          if (gn + 64 < p.n) pp[gm * w + gn + 64] = acc[i][1][r];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t gm = m0 + 64 * wr + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
      if (gm > lastRow) continue;
      if constexpr (SWIGLU) {
        const int64_t gn = static_cast<int64_t>(gi.x) * 64 + 32 * wc + lr;
        if (gn < p.n) p.c[gm * p.n + gn] = toH16(siluMul(acc[i][0][r], acc[i][1][r]));
      } else {
        const int64_t gn = static_cast<int64_t>(gi.x) * WBN + 32 * wc + lr;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t col = gn + 64 * j;
          if (col >= p.n) continue;
          float y = acc[i][j][r];
          if (p.bias) y += static_cast<float>(p.bias[col]);
          if (p.res) y = static_cast<float>(p.res[gm * p.n + col]) + y;
          p.c[gm * p.n + col] = toH16(y);
        }
      }
    }
}

// split-K reduction: the partial planes summed in order, then the epilogue
template <bool SWIGLU>
__global__ __launch_bounds__(256) void gemmF16ReduceKernel(GemmF16Params p) {
  const int64_t total = p.m * p.n, w = SWIGLU ? 2 * p.n : p.n, plane = p.m * w;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / p.n, col = i - row * p.n;
    float y = 0.0f, u = 0.0f;
    for (int z = 0; z < p.split; ++z) {
      y += p.part[z * plane + row * w + col];
      if (SWIGLU) u += p.part[z * plane + row * w + p.n + col];
    }
    if constexpr (SWIGLU) {
      p.c[i] = toH16(siluMul(y, u));
    } else {
      if (p.bias) y += static_cast<float>(p.bias[col]);
      if (p.res) y = static_cast<float>(p.res[i]) + y;
      p.c[i] = toH16(y);
    }
  }
}

// ---- causal GQA over the caches, T > 1: flash tiles on MFMA --------------------------------------------------
// Workgroup = NW waves = 32 queries (positions pos + q0 ..) of one q head; wave w takes key tiles w, w + NW, ...
// (32 keys each) of the head's kv head, and the NW partial (max, sum, O) states merge through LDS at the end.
// S^T = K Q^T on f16 MFMA 32x32x16 (products of f16 values are exact in f32, sums in f32): lane (lr, lh) feeds
// K[key lr][dims 16 s + 8 lh ..] and Q[query lr][same dims], so its accumulator column is query lr with 16 of the
// tile's keys (8 (r / 4) + 4 lh + r % 4), the other 16 in lane ^ 32; the online softmax runs in f32 on those.
// O^T = V^T P^T: the B operand of step st is lane's own P values r = 8 st + e, i.e. keys
// 16 st + 8 (e / 4) + 4 lh + e % 4, fed as two f16 parts (hi = f16(p), lo = f16(p - hi)) so P keeps ~22 bits; the
// A operand (V^T at those keys) is read from the wave's V tile, transposed into LDS as [dim][key].
constexpr int QHD = 128;
constexpr int VT_LD = 40;  // keys per V^T row in LDS (32 + 8 pad)

struct GqaParams {
  const h16* q;
  const h16* kc;
  const h16* vc;
  const int64_t* pos;
  h16* out;
  float* part;
  int64_t t, cap;
  int qh, kvh;
  int chunks, sub;  // T = 1: partials (waves) per head, each over sub consecutive 64-key chunks
  float scale;  // 1 / sqrt(128)
  unsigned long long* err;  // the GPU's error record: positions outside the cache
};

template <int NW>
__global__ __launch_bounds__(64 * NW) void gqaFlashKernel(GqaParams p) {
  __shared__ __attribute__((aligned(16))) h16 Vt[NW][QHD * VT_LD];
  __shared__ float mS[NW][32], lS[NW][32];
  __shared__ float oS[NW][32][33];
  const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t dq = static_cast<int64_t>(p.qh) * QHD, dk = static_cast<int64_t>(p.kvh) * QHD;
  const int64_t kvOff = static_cast<int64_t>(h / (p.qh / p.kvh)) * QHD;
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t p0 = *p.pos;
  const int64_t nk = p0 < 0 ? 0 : min<int64_t>(p0 + p.t, p.cap);  // keys that exist
  const int64_t qpos = p0 + q0 + lr;                                  // this lane's query position
  const float sc = p.scale * kLog2e;
  half8 qf[8];
  {
    const h16* qr = p.q + min<int64_t>(q0 + lr, p.t - 1) * dq + h * QHD + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = ld8(qr + 16 * s);
  }
  const int64_t kEnd = min<int64_t>(nk, p0 + q0 + 32);
  const int tiles = kEnd > 0 ? static_cast<int>((kEnd + 31) / 32) : 0;
  h16* vt = Vt[wave];
  f32x16 o[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (int tile = wave; tile < tiles; tile += NW) {
    const int64_t k0 = static_cast<int64_t>(tile) * 32;
    half8 kf[8];
    const h16* kr = p.kc + min<int64_t>(k0 + lr, nk - 1) * dk + kvOff + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) kf[s] = ld8(kr + 16 * s);
    // V tile -> LDS as V^T [dim][key]: lane (key lr, dim octets lh + 2 i)
    half8 vv[8];
    const h16* vr = p.vc + min<int64_t>(k0 + lr, nk - 1) * dk + kvOff;
#pragma unroll
    for (int i = 0; i < 8; ++i) vv[i] = ld8(vr + 8 * (lh + 2 * i));
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
    for (int st = 0; st < 8; ++st) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[st], qf[st], s, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[(8 * (lh + 2 * i) + e) * VT_LD + lr] = vv[i][e];
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
      s[r] = (key >= nk || key > qpos) ? -INFINITY : s[r] * sc;
      mt = fmaxf(mt, s[r]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mx = fmaxf(m, mt);
    const float mn = mx == -INFINITY ? 0.0f : mx;  // a tile wholly past this query: nothing to add
    const float corr = __builtin_amdgcn_exp2f(m - mn);
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - mn);
      ls += s[r];
    }
    ls += __shfl_xor(ls, 32, 64);
    l = l * corr + ls;
    m = mx;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[b][r] *= corr;
    // the wave's V^T stores before its reads: LDS serves one wave's operations in order; the fence keeps the
    // compiler from moving the reads (other lanes' data) above the stores
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      half8 ph, pl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = s[8 * st + e];
        ph[e] = static_cast<h16>(v);
        pl[e] = static_cast<h16>(v - static_cast<float>(ph[e]));
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const h16* row = vt + (32 * b + lr) * VT_LD + 16 * st + 4 * lh;
        half8 va;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          va[e] = row[e];
          va[4 + e] = row[8 + e];
        }
        o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[b], 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // this tile's V^T reads before the next tile's stores
  }
  // merge the waves, one 32-dim block at a time
  if (lh == 0) {
    mS[wave][lr] = m;
    lS[wave][lr] = l;
  }
  __syncthreads();
  constexpr int TPQ = 2 * NW, DPT = 32 / TPQ;  // threads per query, dims per thread and 32-dim block
  const int q = tid / TPQ, d0 = (tid % TPQ) * DPT;
  float mxw = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) mxw = fmaxf(mxw, mS[w][q]);
  float scw[NW], wsum = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    scw[w] = lS[w][q] > 0.0f ? __builtin_amdgcn_exp2f(mS[w][q] - mxw) : 0.0f;
    wsum += scw[w] * lS[w][q];
  }
  const float inv = 1.0f / wsum;
  const int64_t qrow = q0 + q;
  const bool noRow = p0 + qrow >= p.cap || p0 < 0;
  // recorded once, by the thread of head 0 that owns the first query without a cache row
  if (noRow && qrow < p.t && d0 == 0 && blockIdx.y == 0 && qrow == (p0 < 0 ? 0 : p.cap - p0))
    raiseDeviceError(p.err, LK_DEVERR_POSITION, p0 + qrow);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) oS[wave][lr][8 * (r >> 2) + 4 * lh + (r & 3)] = o[b][r];
    __syncthreads();
    if (qrow < p.t) {
      h16* orow = p.out + qrow * dq + h * QHD + 32 * b + d0;
#pragma unroll
      for (int d = 0; d < DPT; ++d) {
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) acc += scw[w] * oS[w][q][d0 + d];
        orow[d] = noRow ? static_cast<h16>(__builtin_nanf("")) : toH16(acc * inv);
      }
    }
    __syncthreads();
  }
}

// merged decode attention value d of one head from its partials (m, l, o[128]), in partial order, one pass:
// out = sum_c w_c o_c[d] / sum_c w_c l_c with w_c = 2^(m_c - M), M the running max (the sums rescaled when it
// grows). The partials go in blocks of MB whose loads are issued together (predicated), so a merge costs one memory
// round trip per block: 16-wide blocks up to 16 partials (a short cache's one block), 64-wide beyond (a head has at
// most 128 partials: two round trips; 16-wide blocks took 8 and 22 us at 32768 rows, 64-wide ones cost the short
// case 0.6 us). The width depends only on the partial count, so every caller merges with the same bits.
template <int MB>
__device__ __forceinline__ h16 mergeDimBlocks(const float* part, int used, int d) {
  float m = -INFINITY, l = 0.0f, acc = 0.0f;
  for (int c0 = 0; c0 < used; c0 += MB) {
    float mc[MB], lc[MB], oc[MB];
#pragma unroll
    for (int c = 0; c < MB; ++c) {
      const bool in = c0 + c < used;
      const float* pc = part + (c0 + c) * (QHD + 2);
      mc[c] = in ? pc[0] : -INFINITY;
      lc[c] = in ? pc[1] : 0.0f;
      oc[c] = in ? pc[2 + d] : 0.0f;
    }
    float mb = m;
#pragma unroll
    for (int c = 0; c < MB; ++c) mb = fmaxf(mb, mc[c]);
    if (mb == -INFINITY) continue;  // nothing live yet
    const float r = __builtin_amdgcn_exp2f(m - mb);  // 0 while m is -inf
    l *= r;
    acc *= r;
#pragma unroll
    for (int c = 0; c < MB; ++c) {
      const float w = lc[c] > 0.0f ? __builtin_amdgcn_exp2f(mc[c] - mb) : 0.0f;
      l = fmaf(w, lc[c], l);
      acc = fmaf(w, oc[c], acc);
    }
    m = mb;
  }
  return toH16(acc / l);
}

__device__ __forceinline__ h16 mergeDim(const float* part, int used, int d) {
  return used <= 16 ? mergeDimBlocks<16>(part, used, d) : mergeDimBlocks<64>(part, used, d);
}

// ---- causal GQA, T = 1: one wave per (q head, 64-key chunk), partial (m, l, o[128]) to the workspace, then one
// workgroup per q head merges the chunks in order.
constexpr int DCH = 64;

// One wave's chunk (GqaChunk, shared by the split and the fused decode kernels, so both give the same bits):
// lane (g = lane / 16, d8 = lane % 16) owns dims 8 d8 .. 8 d8 + 7 of keys kb + g + 4 i, i < 16. A load instruction
// reads 4 whole 256-byte head rows (coalesced); a score is the lane's 8-term dot summed over the 16 lanes of its row
// by DPP (the same bits in every lane of the row); the chunk max / sum and P.V cross the 4 rows by permlane swaps.
// Rows are loaded from rows clamped to 0 .. pos; the row pos itself takes this step's key / value when the caller
// has them (its cache row may be written concurrently).
struct GqaChunk {
  half8 kr[16], vr[16];
  int64_t kb, nk;
  int g, d8;

  // NT: non-temporal loads (a cache streamed once, as by the split kernel)
  template <bool NT = false>
  __device__ __forceinline__ void load(const h16* kc, const h16* vc, int64_t nkeys, int ch, int64_t dk,
                                       int64_t kvOff) {
    const int lane = threadIdx.x & 63;
    g = lane >> 4;
    d8 = lane & 15;
    kb = static_cast<int64_t>(ch) * DCH;
    nk = nkeys;
    const int64_t last = nk > 0 ? nk - 1 : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t row = min<int64_t>(kb + g + 4 * i, last);
      if constexpr (NT) {
        kr[i] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(kc + row * dk + kvOff + 8 * d8));
        vr[i] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(vc + row * dk + kvOff + 8 * d8));
      } else {
        kr[i] = ld8(kc + row * dk + kvOff + 8 * d8);
        vr[i] = ld8(vc + row * dk + kvOff + 8 * d8);
      }
    }
    // all 32 row loads in flight before the first use (left alone, the scheduler spreads them through the dots
    // to save registers, and the chunk then waits on memory several times)
    __builtin_amdgcn_sched_barrier(0);
  }

  struct Result {
    float m, l;     // chunk max and sum of 2^(s - m) (-inf, 0 for a chunk past the live keys)
    float acc[8];   // sum of 2^(s - m) v over the chunk, this lane's 8 dims (the same in every row of the wave)
  };

  // q8: this lane's 8 query dims (f32). newKey: position whose key / value are knew / vnew (-1: none). Scores in
  // log2 units: dot * scale * log2 e.
  __device__ __forceinline__ Result compute(const float (&q8)[8], int64_t newKey, const half8& knew,
                                            const half8& vnew, float scale) const {
    float sc[16];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t key = kb + g + 4 * i;
      const half8 kk = key == newKey ? knew : kr[i];
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = fmaf(q8[e], static_cast<float>(kk[e]), dot);
      dot = rowSum16(dot);
      sc[i] = key < nk ? dot * scale * kLog2e : -INFINITY;
      m = fmaxf(m, sc[i]);
    }
    m = crossRowMax(m);
    float l = 0.0f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t key = kb + g + 4 * i;
      const float w = key < nk ? __builtin_amdgcn_exp2f(sc[i] - m) : 0.0f;
      l += w;
      const half8 vv = key == newKey ? vnew : vr[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(w, static_cast<float>(vv[e]), acc[e]);
    }
    Result r;
    r.m = m;
    r.l = crossRowSum(l);
#pragma unroll
    for (int e = 0; e < 8; ++e) r.acc[e] = crossRowSum(acc[e]);
    return r;
  }

  // writes the partial (m, l, o[128]): lane 0 m and l, row 0 the 128 dims
  __device__ __forceinline__ static void store(const Result& r, float* part) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) {
      part[0] = r.m;
      part[1] = r.l;
    }
    if ((lane >> 4) == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[2 + 8 * (lane & 15) + e] = r.acc[e];
    }
  }

  // online combination of two chunk results (the running one first), both rescaled to the larger max
  __device__ __forceinline__ static Result combine(const Result& a, const Result& b) {
    Result r;
    r.m = fmaxf(a.m, b.m);
    const float wa = a.l > 0.0f ? __builtin_amdgcn_exp2f(a.m - r.m) : 0.0f;
    const float wb = b.l > 0.0f ? __builtin_amdgcn_exp2f(b.m - r.m) : 0.0f;
    r.l = a.l * wa + b.l * wb;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.acc[e] = a.acc[e] * wa + b.acc[e] * wb;
    return r;
  }
};

// caches of more than 128 chunks: a wave takes ceil(chunks / 128) consecutive chunks, so a head has at most 128
// partials to merge
constexpr int kGqaMaxWaves = 128;
inline void gqaSplit(int64_t cap, int* waves, int* sub) {
  const int64_t c = (cap + DCH - 1) / DCH;
  const int64_t sb = c > kGqaMaxWaves ? (c + kGqaMaxWaves - 1) / kGqaMaxWaves : 1;
  *sub = static_cast<int>(sb);
  *waves = static_cast<int>((c + sb - 1) / sb);
}

// two q heads of a kv group per wave (their K / V rows read once) on caches of 128 or more chunks, where the
// kernels are bandwidth-bound (32768 rows: 65 -> 50 us); on short caches, which are latency-bound, the halved grid
// and doubled per-wave work cost more (config 5 at pos 416: 7.7 -> 9.1 us)
inline bool pairHeads(int qh, int kvh, int64_t cap) {
  return (qh / kvh) % 2 == 0 && (cap + DCH - 1) / DCH >= kGqaMaxWaves;
}

// H q heads of one kv group per wave (H = 2 when the group size is even): the K / V rows are loaded once and each
// head's partial is the single-head arithmetic on them, so H changes no bits.
template <int H>
__global__ __launch_bounds__(64) void gqaDecodeChunkKernel(GqaParams p) {
  const int h0 = blockIdx.x * H, w = blockIdx.y, lane = threadIdx.x;
  const int64_t dk = static_cast<int64_t>(p.kvh) * QHD;
  const int64_t kvOff = static_cast<int64_t>(h0 / (p.qh / p.kvh)) * QHD;
  const int64_t p0 = *p.pos;
  float* part[H];
#pragma unroll
  for (int k = 0; k < H; ++k) part[k] = p.part + (static_cast<int64_t>(h0 + k) * p.chunks + w) * (QHD + 2);
  const int64_t nk = (p0 < 0 || p0 >= p.cap) ? 0 : p0 + 1;
  if (nk == 0 && h0 == 0 && w == 0 && lane == 0) raiseDeviceError(p.err, LK_DEVERR_POSITION, p0);
  const int ch0 = w * p.sub;
  if (static_cast<int64_t>(ch0) * DCH >= nk) return;  // past the live keys: the merge reads no partial of it
  half8 qh8[H];
#pragma unroll
  for (int k = 0; k < H; ++k) qh8[k] = ld8(p.q + (h0 + k) * QHD + 8 * (lane & 15));
  GqaChunk c;
  c.load<true>(p.kc, p.vc, nk, ch0, dk, kvOff);
  float q8[H][8];
#pragma unroll
  for (int k = 0; k < H; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) q8[k][e] = static_cast<float>(qh8[k][e]);
  const half8 none = {};
  GqaChunk::Result r[H];
#pragma unroll
  for (int k = 0; k < H; ++k) r[k] = c.compute(q8[k], -1, none, none, p.scale);
  for (int j = 1; j < p.sub; ++j) {
    c.load<true>(p.kc, p.vc, nk, ch0 + j, dk, kvOff);
#pragma unroll
    for (int k = 0; k < H; ++k) r[k] = GqaChunk::combine(r[k], c.compute(q8[k], -1, none, none, p.scale));
  }
#pragma unroll
  for (int k = 0; k < H; ++k) c.store(r[k], part[k]);
}

__global__ __launch_bounds__(128) void gqaDecodeMergeKernel(GqaParams p) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int64_t p0 = *p.pos;
  const float* part = p.part + static_cast<int64_t>(h) * p.chunks * (QHD + 2);
  h16* o = p.out + static_cast<int64_t>(h) * QHD + d;
  if (p0 < 0 || p0 >= p.cap) {
    *o = static_cast<h16>(__builtin_nanf(""));
    if (h == 0 && d == 0) raiseDeviceError(p.err, LK_DEVERR_POSITION, p0);
    return;
  }
  const int64_t span = static_cast<int64_t>(DCH) * p.sub;  // keys per partial
  *o = mergeDim(part, static_cast<int>(min<int64_t>(p.chunks, (p0 + span) / span)), d);
}

// ---- T = 1 with the QK-norm / RoPE / KV write and the merge folded in: a chunk wave normalizes and rotates its q
// head from the raw projections itself; the chunk holding pos takes the new key and value from them too (never
// from the cache row being written), and the first q head of each kv group writes that row to both caches. Each
// wave holding live keys then writes its chunk partial, fences it and counts itself on its head's counter (waves past
// pos return at once: counting them only queued same-address atomics ahead of the merge); the last live wave of the
// head to arrive (no wave ever waits) reads the head's partials after an acquire fence, merges them as the merge
// kernel does (mergeDim) and resets the counter. Values and roundings are those of qkRopeKvKernel +
// gqaDecodeChunkKernel + gqaDecodeMergeKernel (the same helpers), so the output is identical.
struct GqaDecParams {
  const h16* qkv;  // [1, qh 128 + 2 kvh 128]
  const h16* qg;
  const h16* kg;
  const int64_t* pos;
  h16* kc;
  h16* vc;
  float* part;         // [qh, chunks, 130] (workspace)
  h16* out;            // [1, qh 128]
  unsigned* counters;  // [qh], zero between launches
  int64_t cap;
  int qh, kvh;
  int chunks, sub;  // partials (waves) per head, each over sub consecutive 64-key chunks
  float scale, eps;
  RopeTable tab;
  unsigned long long* err;  // the GPU's error record: positions outside the cache
};

// live: the head's waves holding keys (only they count themselves; the others return at once)
__device__ __forceinline__ void decodeMergeIfLast(const GqaDecParams& p, int h, int lane, int live) {
  __shared__ unsigned lastFlag;
  __threadfence();  // release: this wave's partial is in L2 before it is counted
  if (lane == 0) lastFlag = atomicAdd(&p.counters[h], 1u) == static_cast<unsigned>(live - 1);
  __syncthreads();
  if (!lastFlag) return;
  __threadfence();  // acquire: the other waves' partials (and no stale L1 lines) from here on
  const int used = live;
  const float* ph = p.part + static_cast<int64_t>(h) * p.chunks * (QHD + 2);
  h16* o = p.out + static_cast<int64_t>(h) * QHD;
  o[lane] = mergeDim(ph, used, lane);
  o[lane + 64] = mergeDim(ph, used, lane + 64);
  if (lane == 0) p.counters[h] = 0u;
}

// One wave's part of the fused T = 1 step: QK-norm + RoPE of its H q heads from the raw projections, the new key /
// value when its chunks hold pos (written to both caches by the first q head of the kv group), then its chunks'
// attention results r[H]. All loads are issued first, in the order the in-order memory counter needs: the raw q / k /
// v values (the norms wait for them alone), then the chunk's K and V rows. qs, kn, vn: this wave's own LDS slices.
// Requires kb = w sub 64 < nk.
template <int H>
__device__ __forceinline__ void qkrWave(const GqaDecParams& p, int h0, int w, int64_t p0, int64_t nk, float (*qs)[QHD],
                                        h16* kn, h16* vn, GqaChunk::Result (&r)[H]) {
  const int lane = threadIdx.x & 63;
  const int grp = p.qh / p.kvh;
  const int64_t dq = static_cast<int64_t>(p.qh) * QHD, dk = static_cast<int64_t>(p.kvh) * QHD;
  const int64_t kvOff = static_cast<int64_t>(h0 / grp) * QHD;
  const int ch0 = w * p.sub;
  const int64_t kb = static_cast<int64_t>(ch0) * DCH;
  const bool hasNew = p0 < kb + static_cast<int64_t>(DCH) * p.sub;  // this wave's chunks hold key pos (kb <= pos)
  const int cl = lane & 15;           // rowSumSq's chunk of a 128-wide head (lanes 16.. add nothing)
  const h16* xk = p.qkv + dq + kvOff;
  const h16* xv = p.qkv + dq + dk + kvOff;
  half8 qc[H];
  h16 q0[H], q1[H];
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const h16* xq = p.qkv + (h0 + k) * QHD;
    qc[k] = ld8(xq + 8 * cl);
    q0[k] = xq[lane];
    q1[k] = xq[lane + 64];
  }
  const h16 gq0 = p.qg[lane], gq1 = p.qg[lane + 64];
  half8 kc8 = {};
  h16 k0 = 0, k1 = 0, gk0 = 0, gk1 = 0, v0 = 0, v1 = 0;
  if (hasNew) {
    kc8 = ld8(xk + 8 * cl);
    k0 = xk[lane];
    k1 = xk[lane + 64];
    gk0 = p.kg[lane];
    gk1 = p.kg[lane + 64];
    v0 = xv[lane];
    v1 = xv[lane + 64];
  }
  GqaChunk c;
  c.load(p.kc, p.vc, nk, ch0, dk, kvOff);
  auto headSumSq = [&](const half8& c8) {
    float sq = 0.0f;
    if (lane < 16) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sq = fmaf(static_cast<float>(c8[e]), static_cast<float>(c8[e]), sq);
    }
    return waveSum(sq);
  };
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const float rf = rmsFactor(headSumSq(qc[k]), QHD, p.eps);
    h16 a, b;
    ropePair(static_cast<float>(rmsElem(q0[k], gq0, rf)), static_cast<float>(rmsElem(q1[k], gq1, rf)), p0,
             p.tab.invf[lane], a, b);
    qs[k][lane] = static_cast<float>(a);
    qs[k][lane + 64] = static_cast<float>(b);
  }
  if (hasNew) {
    const float rf = rmsFactor(headSumSq(kc8), QHD, p.eps);
    h16 a, b;
    ropePair(static_cast<float>(rmsElem(k0, gk0, rf)), static_cast<float>(rmsElem(k1, gk1, rf)), p0, p.tab.invf[lane],
             a, b);
    kn[lane] = a;
    kn[lane + 64] = b;
    vn[lane] = v0;
    vn[lane + 64] = v1;
    if (h0 % grp == 0) {  // one wave per kv head writes the new row to both caches
      p.kc[p0 * dk + kvOff + lane] = a;
      p.kc[p0 * dk + kvOff + lane + 64] = b;
      p.vc[p0 * dk + kvOff + lane] = v0;
      p.vc[p0 * dk + kvOff + lane + 64] = v1;
    }
  }
  // the slices are this wave's alone and a wave's LDS accesses complete in order: no workgroup barrier
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int d8 = lane & 15;
  float q8[H][8];
#pragma unroll
  for (int k = 0; k < H; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) q8[k][e] = qs[k][8 * d8 + e];
  const half8 none = {};
  const int64_t newKey = hasNew ? p0 : -1;
  const half8 knew = hasNew ? ld8(kn + 8 * d8) : none, vnew = hasNew ? ld8(vn + 8 * d8) : none;
#pragma unroll
  for (int k = 0; k < H; ++k) r[k] = c.compute(q8[k], newKey, knew, vnew, p.scale);
  for (int j = 1; j < p.sub; ++j) {
    c.load(p.kc, p.vc, nk, ch0 + j, dk, kvOff);
#pragma unroll
    for (int k = 0; k < H; ++k) r[k] = GqaChunk::combine(r[k], c.compute(q8[k], newKey, knew, vnew, p.scale));
  }
}

// A position outside the cache: NaN outputs for the H heads (written by their first wave), no cache write, the error
// recorded once.
template <int H>
__device__ __forceinline__ void qkrBadPosition(const GqaDecParams& p, int h0, int w, int64_t p0) {
  const int lane = threadIdx.x & 63;
  if (h0 == 0 && w == 0 && lane == 0) raiseDeviceError(p.err, LK_DEVERR_POSITION, p0);
  if (w == 0)
#pragma unroll
    for (int k = 0; k < H; ++k) {
      p.out[static_cast<int64_t>(h0 + k) * QHD + lane] = static_cast<h16>(__builtin_nanf(""));
      p.out[static_cast<int64_t>(h0 + k) * QHD + lane + 64] = static_cast<h16>(__builtin_nanf(""));
    }
}

// One wave per (H q heads of one kv group, sub-chunk range); each head's merge is run by the last wave counted on
// that head's counter (decodeMergeIfLast).
template <int H>
__global__ __launch_bounds__(64) void gqaDecodeQkrKernel(GqaDecParams p) {
  __shared__ float qs[H][QHD];
  __shared__ __attribute__((aligned(16))) h16 kn[QHD];
  __shared__ __attribute__((aligned(16))) h16 vn[QHD];
  const int h0 = blockIdx.x * H, w = blockIdx.y, lane = threadIdx.x;
  const int64_t p0 = *p.pos;
  const int64_t nk = (p0 < 0 || p0 >= p.cap) ? 0 : p0 + 1;
  if (nk == 0) {
    qkrBadPosition<H>(p, h0, w, p0);
    return;
  }
  const int64_t span = static_cast<int64_t>(DCH) * p.sub;  // keys per wave
  const int live = static_cast<int>((nk + span - 1) / span);
  if (static_cast<int64_t>(w) * span >= nk) return;  // past the live keys: no partial, not counted
  GqaChunk::Result r[H];
  qkrWave<H>(p, h0, w, p0, nk, qs, kn, vn, r);
#pragma unroll
  for (int k = 0; k < H; ++k) {
    GqaChunk::store(r[k], p.part + (static_cast<int64_t>(h0 + k) * p.chunks + w) * (QHD + 2));
    decodeMergeIfLast(p, h0 + k, lane, live);
  }
}

// Short caches (chunks <= kQkrWgWaves, sub = 1): one workgroup per q head, wave w on chunk w. The live waves leave
// their partials in LDS and, after one workgroup barrier, the first 128 threads merge them (mergeDim, one dim each):
// no workspace round trip, fence or counter. Same helpers, so the same bits as gqaDecodeQkrKernel<1>.
constexpr int kQkrWgWaves = 8;  // 512 threads: the 256 VGPRs a chunk wave needs (220) without spills
__global__ __launch_bounds__(64 * kQkrWgWaves) void gqaDecodeQkrWgKernel(GqaDecParams p) {
  __shared__ float qs[kQkrWgWaves][1][QHD];
  __shared__ __attribute__((aligned(16))) h16 kn[kQkrWgWaves][QHD];
  __shared__ __attribute__((aligned(16))) h16 vn[kQkrWgWaves][QHD];
  __shared__ float parts[kQkrWgWaves * (QHD + 2)];
  const int h0 = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t p0 = *p.pos;
  const int64_t nk = (p0 < 0 || p0 >= p.cap) ? 0 : p0 + 1;
  if (nk == 0) {  // uniform over the workgroup: every wave returns before the barrier
    qkrBadPosition<1>(p, h0, w, p0);
    return;
  }
  const int live = static_cast<int>((nk + DCH - 1) / DCH);
  if (static_cast<int64_t>(w) * DCH < nk) {
    GqaChunk::Result r[1];
    qkrWave<1>(p, h0, w, p0, nk, qs[w], kn[w], vn[w], r);
    GqaChunk::store(r[0], parts + w * (QHD + 2));
  }
  __syncthreads();
  for (int d = threadIdx.x; d < QHD; d += blockDim.x)  // one wave (a one-chunk cache) merges both halves
    p.out[static_cast<int64_t>(h0) * QHD + d] = mergeDim(parts, live, d);
}

// ---- row copies, gathers, elementwise -----------------------------------------------------------------------
// kv_write: rows pos..pos+T-1 of both caches = k, v (8 halves per thread); rows past the cache are dropped
__global__ void kvWriteF16Kernel(h16* __restrict__ kc, h16* __restrict__ vc, const h16* __restrict__ k,
                                 const h16* __restrict__ v, const int64_t* __restrict__ pos, int64_t t, int64_t d,
                                 int64_t cap) {
  const int64_t p0 = *pos, d8 = d / 8, total = t * d8;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d8, c = (i - r * d8) * 8, row = p0 + r;
    if (row < 0 || row >= cap) continue;
    st8(kc + row * d + c, ld8(k + r * d + c));
    st8(vc + row * d + c, ld8(v + r * d + c));
  }
}

// embedding: out[i] = table[ids[i]] (an id out of range gives a NaN row). scatter: the j-th row whose id is padId
// (counted over ids[0 .. i)) becomes audio[j] (NaN row when j >= A), other rows copy x. One workgroup per row.
__global__ __launch_bounds__(256) void embedScatterF16Kernel(const h16* __restrict__ table, const int64_t* __restrict__ ids,
                                                             const h16* __restrict__ x, const h16* __restrict__ audio,
                                                             h16* __restrict__ out, int64_t vocab, int64_t d,
                                                             int64_t na, int64_t padId, int mode,
                                                             unsigned long long* err) {
  __shared__ int cnt[4];
  const int64_t i = blockIdx.x;
  const int64_t id = ids[i];
  const h16* src = nullptr;
  if (mode == 0) {
    if (id >= 0 && id < vocab) src = table + id * d;
  } else {
    if (id == padId) {
      int c = 0;
      for (int64_t j = threadIdx.x; j < i; j += 256) c += ids[j] == padId;
      for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
      if ((threadIdx.x & 63) == 0) cnt[threadIdx.x >> 6] = c;
      __syncthreads();
      const int64_t j = cnt[0] + cnt[1] + cnt[2] + cnt[3];
      if (j < na) src = audio + j * d;
    } else {
      src = x + i * d;
    }
  }
  h16* o = out + i * d;
  if (!src && threadIdx.x == 0)
    raiseDeviceError(err, mode == 0 ? LK_DEVERR_INDEX : LK_DEVERR_AUDIO_ROWS, mode == 0 ? id : i);
  for (int64_t c = threadIdx.x; c < d; c += 256) o[c] = src ? src[c] : static_cast<h16>(__builtin_nanf(""));
}

// op 0: a + b; 1: silu(a) * b (g / (1 + exp(-g)) * u); f32 math, one rounding
__global__ void eltF16Kernel(const h16* __restrict__ a, const h16* __restrict__ b, h16* __restrict__ out, int64_t n,
                             int op) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float x = static_cast<float>(a[i]), y = static_cast<float>(b[i]);
    out[i] = toH16(op == 0 ? x + y : siluMul(x, y));
  }
}

// W f16[K, N] -> W^T f16[N, K] through 32 x 32 LDS tiles
__global__ __launch_bounds__(256) void transposeF16Kernel(const h16* __restrict__ w, h16* __restrict__ wt, int64_t k,
                                                          int64_t n) {
  __shared__ h16 tile[32][33];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 32, k0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8)
    if (k0 + r < k && n0 + tx < n) tile[r][tx] = w[(k0 + r) * n + n0 + tx];
  __syncthreads();
  for (int r = ty; r < 32; r += 8)
    if (n0 + r < n && k0 + tx < k) wt[(n0 + r) * k + k0 + tx] = tile[tx][r];
}

}  // namespace lkd

// ---- C-ABI ----------------------------------------------------------------------------------------------------
namespace {

bool aligned16(const void* a) { return (reinterpret_cast<uintptr_t>(a) & 15) == 0; }

lkd::RopeTable ropeTable(float theta) {
  lkd::RopeTable t;
  for (int j = 0; j < 64; ++j) t.invf[j] = 1.0f / std::pow(theta, static_cast<float>(2 * j) / 128.0f);
  return t;
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : 2; }

}  // namespace

extern "C" {

int lk_hip_f16_rms_lm_head(const void* x, const void* g, const void* table, float* out, int64_t t, int64_t d, int64_t v,
                           float eps, void* stream);

int64_t lk_hip_f16_gemm_workspace_bytes(int64_t m, int64_t n, int swiglu) {
  return 8 * m * n * (swiglu ? 2 : 1) * 4;
}

// out f16[M, N] = epi(x f16[M, K] @ W), W given packed as W^T f16[N', K] (N' = N, or 2N = [gate | up] with
// swiglu). epi: bias f16[N] (or null), then res f16[M, N] (or null) added; swiglu: silu(gate) * up. K % 8 == 0 and
// 16-byte aligned x, W^T. workspace (optional): split-K partials for a small grid (NULL: never splits).
int lk_hip_f16_gemm(const void* x, const void* wt, const void* bias, const void* res, void* out, int64_t m, int64_t n,
                    int64_t k, int swiglu, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lkd;
  if (m < 0 || n <= 0 || k <= 0 || k % 8 != 0 || !aligned16(x) || !aligned16(wt)) return 1;
  if (m == 0) return 0;
  if (swiglu && (bias || res)) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (m == 1) {
    GemvF16Params g{static_cast<const h16*>(x), nullptr, static_cast<const h16*>(wt), static_cast<const h16*>(bias),
                    static_cast<const h16*>(res), out, n, k, 0.0f};
    const int64_t waves = swiglu ? n : (n + 1) / 2;
    const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
    if (swiglu) launchGemvF16<EPI_SWIGLU, false>(g, blocks, s);
    else launchGemvF16<EPI_PLAIN, false>(g, blocks, s);
    return launched();
  }
  GemmF16Params p{static_cast<const h16*>(x), static_cast<const h16*>(wt), static_cast<const h16*>(bias),
                  static_cast<const h16*>(res), static_cast<h16*>(out), nullptr, m, n, k, k, k, 1};
  // the wide tile where it measured faster: SwiGLU at M >= 256 (Qwen3's 416-row gate/up: 57 -> 49 us) and any
  // M >= 1024 (4096^3: 471 -> 706 TFLOP/s); at M = 416 the plain shapes fill the chip better with 64-row tiles
  const bool wide = swiglu ? m >= 256 : m >= 1024;
  const unsigned gx = static_cast<unsigned>(swiglu ? (n + 63) / 64 : (n + GBN - 1) / GBN);
  const unsigned gy = static_cast<unsigned>(wide ? (m + WBM - 1) / WBM : (m + GBM - 1) / GBM);
  const int64_t tiles = static_cast<int64_t>(gx) * gy;
  int split = 1;
  if (workspace && tiles < 192 && k >= 1024) {
    split = static_cast<int>(std::min<int64_t>({8, 384 / tiles, k / 512}));
    while (split > 1 && static_cast<int64_t>(split) * m * n * (swiglu ? 2 : 1) * 4 > workspace_bytes) --split;
  }
  if (split > 1) {
    p.kSplit = ((k + split - 1) / split + GBK - 1) / GBK * GBK;
    split = static_cast<int>((k + p.kSplit - 1) / p.kSplit);
    p.split = split;
    p.part = static_cast<float*>(workspace);
  }
  const bool tail = (p.split > 1 ? p.kSplit : k) % GBK != 0 || k % GBK != 0;
  const dim3 grid(gx, gy, static_cast<unsigned>(split));
  if (wide && swiglu) {
    if (tail) hipLaunchKernelGGL((gemmF16WideKernel<true, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemmF16WideKernel<true, false>), grid, dim3(256), 0, s, p);
  } else if (wide) {
    if (tail) hipLaunchKernelGGL((gemmF16WideKernel<false, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemmF16WideKernel<false, false>), grid, dim3(256), 0, s, p);
  } else if (swiglu) {
    if (tail) hipLaunchKernelGGL((gemmF16Kernel<true, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemmF16Kernel<true, false>), grid, dim3(256), 0, s, p);
  } else {
    if (tail) hipLaunchKernelGGL((gemmF16Kernel<false, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemmF16Kernel<false, false>), grid, dim3(256), 0, s, p);
  }
  if (split > 1) {
    const unsigned rb = static_cast<unsigned>(std::min<int64_t>((m * n + 255) / 256, 4096));
    if (swiglu) hipLaunchKernelGGL((gemmF16ReduceKernel<true>), dim3(rb), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemmF16ReduceKernel<false>), dim3(rb), dim3(256), 0, s, p);
  }
  return launched();
}

// rmsnorm(x, g) @ W [swiglu]. M = 1: one GEMV whose waves normalize the row; M > 1: normalized rows into ws
// f16[M, K], then lk_hip_f16_gemm.
int lk_hip_f16_rms_gemm(const void* x, const void* g, const void* wt, void* out, void* ws, int64_t m, int64_t n,
                        int64_t k, float eps, int swiglu, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lkd;
  if (m < 0 || n <= 0 || k <= 0 || k % 8 != 0 || !aligned16(x) || !aligned16(g) || !aligned16(wt)) return 1;
  if (m == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (m == 1) {
    GemvF16Params p{static_cast<const h16*>(x), static_cast<const h16*>(g), static_cast<const h16*>(wt), nullptr,
                    nullptr, out, n, k, eps};
    const int64_t waves = swiglu ? n : (n + 1) / 2;
    const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
    if (swiglu) launchGemvF16<EPI_SWIGLU, true>(p, blocks, s);
    else launchGemvF16<EPI_PLAIN, true>(p, blocks, s);
    return launched();
  }
  if (!aligned16(ws)) return 1;
  hipLaunchKernelGGL(k == 2048 ? rmsGroupsKernel<2048> : rmsGroupsKernel<0>, dim3(static_cast<unsigned>((m + 3) / 4)),
                     dim3(256), 0, s,
                     static_cast<const h16*>(x), static_cast<const h16*>(g), static_cast<h16*>(ws), m, k, eps);
  if (launched()) return 2;
  return lk_hip_f16_gemm(ws, wt, nullptr, nullptr, out, m, n, k, swiglu, workspace, workspace_bytes, stream);
}

// out f32[1, V] = x[T-1] . table[V, D]^T
int lk_hip_f16_lm_head(const void* x, const void* table, float* out, int64_t t, int64_t d, int64_t v, void* stream) {
  return lk_hip_f16_rms_lm_head(x, nullptr, table, out, t, d, v, 0.0f, stream);
}

// out f32[1, V] = rmsnorm(x[T-1], g) . table^T (g null: no norm); the row is normalized by every wave itself
int lk_hip_f16_rms_lm_head(const void* x, const void* g, const void* table, float* out, int64_t t, int64_t d, int64_t v,
                           float eps, void* stream) {
  using namespace lkd;
  if (t <= 0 || v <= 0 || d <= 0 || d % 8 != 0 || !aligned16(x) || !aligned16(table) || (g && !aligned16(g))) return 1;
  GemvF16Params p{static_cast<const h16*>(x) + (t - 1) * d, static_cast<const h16*>(g), static_cast<const h16*>(table),
                  nullptr, nullptr, out, v, d, eps};
  const unsigned blocks = static_cast<unsigned>(((v + 1) / 2 + 3) / 4);
  if (g) launchGemvF16<EPI_F32, true>(p, blocks, static_cast<hipStream_t>(stream));
  else launchGemvF16<EPI_F32, false>(p, blocks, static_cast<hipStream_t>(stream));
  return launched();
}

// rows of x f16[R, C] normalized in groups of `width` (C for rmsnorm, the head width for rmsnorm_heads)
int lk_hip_f16_rmsnorm(const void* x, const void* g, void* out, int64_t rows, int64_t c, int64_t width, float eps,
                       void* stream) {
  using namespace lkd;
  if (rows < 0 || c <= 0 || width <= 0 || width % 8 != 0 || c % width != 0 || !aligned16(x) || !aligned16(g) ||
      !aligned16(out))
    return 1;
  const int64_t groups = rows * (c / width);
  if (groups == 0) return 0;
  hipLaunchKernelGGL(width == 2048 ? rmsGroupsKernel<2048> : rmsGroupsKernel<0>,
                     dim3(static_cast<unsigned>((groups + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const h16*>(x), static_cast<const h16*>(g),
                     static_cast<h16*>(out), groups, width, eps);
  return launched();
}

int lk_hip_f16_rope(const void* x, const int64_t* pos, void* out, int64_t t, int64_t c, float theta, void* stream) {
  using namespace lkd;
  if (t < 0 || c <= 0 || c % 128 != 0) return 1;
  const int64_t items = t * (c / 128);
  if (items == 0) return 0;
  hipLaunchKernelGGL(ropeKernel, dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const h16*>(x), pos, static_cast<h16*>(out), t, c,
                     ropeTable(theta));
  return launched();
}

int lk_hip_f16_qknorm_rope_kv(const void* qkv, const void* qg, const void* kg, const int64_t* pos, void* kc, void* vc,
                              void* q, int64_t t, int qh, int kvh, int64_t cap, float eps, float theta, void* stream) {
  using namespace lkd;
  if (t < 0 || qh <= 0 || kvh <= 0 || cap <= 0 || !aligned16(qkv)) return 1;
  if (t == 0) return 0;
  QkrParams p{static_cast<const h16*>(qkv), static_cast<const h16*>(qg), static_cast<const h16*>(kg), pos,
              static_cast<h16*>(kc), static_cast<h16*>(vc), static_cast<h16*>(q), t, cap, qh, kvh, eps,
              ropeTable(theta)};
  const int64_t items = t * (qh + 2 * kvh);
  hipLaunchKernelGGL(qkRopeKvKernel, dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p);
  return launched();
}

int64_t lk_hip_f16_attention_workspace_bytes(int qh, int64_t cap) {
  int waves = 0, sub = 0;
  lkd::gqaSplit(cap, &waves, &sub);
  return static_cast<int64_t>(qh) * waves * (lkd::QHD + 2) * 4;
}

// causal GQA: q f16[T, qh 128], caches f16[cap, kvh 128] holding rows 0..pos+T-1 -> out f16[T, qh 128].
// T = 1 needs the workspace (lk_hip_f16_attention_workspace_bytes); returns 3 when it is too small.
int lk_hip_f16_attention_gqa(const void* q, const void* kc, const void* vc, const int64_t* pos, void* out, int64_t t,
                             int qh, int kvh, int64_t cap, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lkd;
  if (t < 0 || qh <= 0 || kvh <= 0 || qh % kvh != 0 || cap <= 0 || !aligned16(q) || !aligned16(kc) || !aligned16(vc))
    return 1;
  if (t == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int chunks = 0, sub = 0;
  gqaSplit(cap, &chunks, &sub);
  GqaParams p{static_cast<const h16*>(q), static_cast<const h16*>(kc), static_cast<const h16*>(vc), pos,
              static_cast<h16*>(out), static_cast<float*>(workspace), t, cap, qh, kvh, chunks, sub,
              1.0f / std::sqrt(static_cast<float>(QHD)), lkh::deviceErrorRecord()};
  if (t == 1) {
    if (!workspace || workspace_bytes < lk_hip_f16_attention_workspace_bytes(qh, cap)) return 3;
    if (pairHeads(qh, kvh, cap))
      hipLaunchKernelGGL(gqaDecodeChunkKernel<2>, dim3(static_cast<unsigned>(qh / 2), static_cast<unsigned>(chunks)),
                         dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL(gqaDecodeChunkKernel<1>, dim3(static_cast<unsigned>(qh), static_cast<unsigned>(chunks)),
                         dim3(64), 0, s, p);
    hipLaunchKernelGGL(gqaDecodeMergeKernel, dim3(static_cast<unsigned>(qh)), dim3(128), 0, s, p);
    return launched();
  }
  // 8 waves per 32-query block: a causal block holds few key tiles, so more waves in flight per block
  // (Qwen3 416-id prefill 3.94 -> 3.89 ms against 4)
  hipLaunchKernelGGL(gqaFlashKernel<8>, dim3(static_cast<unsigned>((t + 31) / 32), static_cast<unsigned>(qh)),
                     dim3(512), 0, s, p);
  return launched();
}

// decode step (T = 1) attention with the QK-norm / RoPE / KV write and the chunk merge folded in:
// qkv f16[1, 128 (qh + 2 kvh)] -> out f16[1, 128 qh]; row pos of both caches written. counters: qh unsigned ints,
// zero before the first call (every call leaves them zero); workspace: lk_hip_f16_attention_workspace_bytes
// (returns 3 when short). Calls sharing counters or workspace must be stream-ordered.
int lk_hip_f16_attention_decode_qkr(const void* qkv, const void* qg, const void* kg, const int64_t* pos, void* kc,
                                    void* vc, void* out, unsigned* counters, int qh, int kvh, int64_t cap, float eps,
                                    float theta, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lkd;
  if (qh <= 0 || kvh <= 0 || qh % kvh != 0 || cap <= 0 || !counters || !aligned16(qkv) || !aligned16(kc) ||
      !aligned16(vc))
    return 1;
  if (!workspace || workspace_bytes < lk_hip_f16_attention_workspace_bytes(qh, cap)) return 3;
  int chunks = 0, sub = 0;
  gqaSplit(cap, &chunks, &sub);
  GqaDecParams p{static_cast<const h16*>(qkv), static_cast<const h16*>(qg), static_cast<const h16*>(kg), pos,
                 static_cast<h16*>(kc), static_cast<h16*>(vc), static_cast<float*>(workspace), static_cast<h16*>(out),
                 counters, cap, qh, kvh, chunks, sub, 1.0f / std::sqrt(static_cast<float>(QHD)), eps, ropeTable(theta),
                 lkh::deviceErrorRecord()};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (sub == 1 && chunks <= kQkrWgWaves)
    hipLaunchKernelGGL(gqaDecodeQkrWgKernel, dim3(static_cast<unsigned>(qh)), dim3(64 * static_cast<unsigned>(chunks)),
                       0, s, p);
  else if (pairHeads(qh, kvh, cap))
    hipLaunchKernelGGL(gqaDecodeQkrKernel<2>, dim3(static_cast<unsigned>(qh / 2), static_cast<unsigned>(chunks)),
                       dim3(64), 0, s, p);
  else
    hipLaunchKernelGGL(gqaDecodeQkrKernel<1>, dim3(static_cast<unsigned>(qh), static_cast<unsigned>(chunks)),
                       dim3(64), 0, s, p);
  return launched();
}


int lk_hip_f16_kv_write(void* kc, void* vc, const void* k, const void* v, const int64_t* pos, int64_t t, int64_t d,
                        int64_t cap, void* stream) {
  using namespace lkd;
  if (t < 0 || d <= 0 || d % 8 != 0 || !aligned16(kc) || !aligned16(vc) || !aligned16(k) || !aligned16(v)) return 1;
  if (t == 0) return 0;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((t * d / 8 + 255) / 256, 4096));
  hipLaunchKernelGGL(kvWriteF16Kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<h16*>(kc), static_cast<h16*>(vc), static_cast<const h16*>(k),
                     static_cast<const h16*>(v), pos, t, d, cap);
  return launched();
}

int lk_hip_f16_embedding(const int64_t* ids, const void* table, void* out, int64_t t, int64_t vocab, int64_t d,
                         void* stream) {
  using namespace lkd;
  if (t < 0 || d <= 0) return 1;
  if (t == 0) return 0;
  hipLaunchKernelGGL(embedScatterF16Kernel, dim3(static_cast<unsigned>(t)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const h16*>(table), ids, nullptr, nullptr,
                     static_cast<h16*>(out), vocab, d, int64_t{0}, int64_t{0}, 0, lkh::deviceErrorRecord());
  return launched();
}

int lk_hip_f16_scatter_audio(const void* x, const int64_t* ids, const void* audio, void* out, int64_t t, int64_t d,
                             int64_t na, int64_t pad_id, void* stream) {
  using namespace lkd;
  if (t < 0 || d <= 0 || na < 0) return 1;
  if (t == 0) return 0;
  hipLaunchKernelGGL(embedScatterF16Kernel, dim3(static_cast<unsigned>(t)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), nullptr, ids, static_cast<const h16*>(x),
                     static_cast<const h16*>(audio), static_cast<h16*>(out), int64_t{0}, d, na, pad_id, 1,
                     lkh::deviceErrorRecord());
  return launched();
}

// op 0: a + b; 1: silu(a) * b
int lk_hip_f16_elementwise(const void* a, const void* b, void* out, int64_t n, int op, void* stream) {
  using namespace lkd;
  if (n < 0 || op < 0 || op > 1) return 1;
  if (n == 0) return 0;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 8192));
  hipLaunchKernelGGL(eltF16Kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const h16*>(a), static_cast<const h16*>(b), static_cast<h16*>(out), n, op);
  return launched();
}

// W f16[K, N] -> W^T f16[N, K] (the packed operand of the GEMM / GEMV)
int lk_hip_f16_transpose(const void* w, void* wt, int64_t k, int64_t n, void* stream) {
  using namespace lkd;
  if (k < 0 || n < 0) return 1;
  if (k == 0 || n == 0) return 0;
  hipLaunchKernelGGL(transposeF16Kernel, dim3(static_cast<unsigned>((n + 31) / 32), static_cast<unsigned>((k + 31) / 32)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const h16*>(w),
                     static_cast<h16*>(wt), k, n);
  return launched();
}

}  // extern "C"

// ---- registry: the reference's f16 GPU op names (kernels/gpu/f16_gpu.cpp:1011-1050) ---------------------------
// GEMM-like ops take the weight packed as W^T f16[N', K] (the contract leaves the layout to the kernel: the
// reference packs at prepare time, this backend once at model build through transpose_f16_gpu).
namespace lkh {

namespace {

constexpr int64_t kWsReserve = 65536;  // the workspace's first 64 KiB are kept for counters of other kernels

void* wsPtr(ExecCtx& ctx) {
  return ctx.workspace && ctx.workspaceBytes > kWsReserve ? static_cast<char*>(ctx.workspace) + kWsReserve : nullptr;
}
int64_t wsBytes(ExecCtx& ctx) {
  return ctx.workspace && ctx.workspaceBytes > kWsReserve ? static_cast<int64_t>(ctx.workspaceBytes) - kWsReserve : 0;
}

// gemm[_opt] / gemm_bias[_opt] / gemm_add_opt / gemm_swiglu_opt: x[M, K], wt[N', K] [, b[N] | res[M, N]] -> [M, N]
template <int KIND>  // 0 plain, 1 bias, 2 residual, 3 swiglu
void runGemmF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t m = it.next(), k = it.next(), nr = it.next(), k2 = it.next();
  LK_REQUIRE(ctx, k2 == k, "gemm_f16: w must be packed W^T f16[N, K]");
  LK_REQUIRE(ctx, KIND != 3 || nr % 2 == 0, "gemm_swiglu_f16: w must be packed [gate | up]^T f16[2N, K]");
  const int64_t n = KIND == 3 ? nr / 2 : nr;
  const void* bias = KIND == 1 ? a.ptrs[2] : nullptr;
  const void* res = KIND == 2 ? a.ptrs[2] : nullptr;
  void* out = a.ptrs[KIND == 1 || KIND == 2 ? 3 : 2];
  status(ctx, lk_hip_f16_gemm(a.ptrs[0], a.ptrs[1], bias, res, out, m, n, k, KIND == 3, wsPtr(ctx), wsBytes(ctx),
                              ctx.stream),
         "gemm_f16: launch failed (K % 8 == 0 and 16-byte aligned operands needed)");
}

// rmsnorm_gemm[_swiglu]_opt: x[M, K], g[K], wt[N', K] -> (y[M, N], ws[M, K]); float eps
template <bool SWIGLU>
void runRmsGemmF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t m = it.next(), k = it.next();
  LK_REQUIRE(ctx, it.next() == k, "rmsnorm_gemm_f16: g must be f16[K]");
  const int64_t nr = it.next();
  LK_REQUIRE(ctx, it.next() == k, "rmsnorm_gemm_f16: w must be packed W^T f16[N, K]");
  const int64_t n = SWIGLU ? nr / 2 : nr;
  status(ctx, lk_hip_f16_rms_gemm(a.ptrs[0], a.ptrs[1], a.ptrs[2], a.ptrs[3], a.ptrs[4], m, n, k, F(a, 0, 1e-6f),
                                  SWIGLU ? 1 : 0, wsPtr(ctx), wsBytes(ctx), ctx.stream),
         "rmsnorm_gemm_f16: launch failed");
}

// lm_head_last[_opt]: x[T, D], table[V, D] -> f32[1, V]
void runLmHeadF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d = it.next(), v = it.next();
  LK_REQUIRE(ctx, it.next() == d, "lm_head_last_f16: table must be f16[V, D]");
  status(ctx, lk_hip_f16_lm_head(a.ptrs[0], a.ptrs[1], P<float>(a, 2), t, d, v, ctx.stream),
         "lm_head_last_f16: launch failed");
}

// rmsnorm: x[R, C], g[C]; rmsnorm_heads: x[R, C], g[hd]; float eps
template <bool HEADS>
void runRmsNormF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t r = it.next(), c = it.next(), w = it.next();
  LK_REQUIRE(ctx, HEADS ? c % w == 0 : w == c, "rmsnorm_f16: g width does not divide the row");
  status(ctx, lk_hip_f16_rmsnorm(a.ptrs[0], a.ptrs[1], a.ptrs[2], r, c, w, F(a, 0, 1e-6f), ctx.stream),
         "rmsnorm_f16: launch failed (width % 8 == 0 and 16-byte aligned rows needed)");
}

// rope: x[T, C], pos[1]; float theta
void runRopeF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), c = it.next();
  LK_REQUIRE(ctx, c % 128 == 0, "rope_f16: heads must be 128 wide");
  status(ctx, lk_hip_f16_rope(a.ptrs[0], P<int64_t>(a, 1), a.ptrs[2], t, c, F(a, 0, 1e6f), ctx.stream),
         "rope_f16: launch failed");
}

// qknorm_rope_kv_opt (inout kc, vc): qkv[T, Dq + 2 Dk], qg[128], kg[128], pos[1], kc[P, Dk], vc[P, Dk] -> q[T, Dq];
// floats eps, theta
void runQkrF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), w = it.next(), hq = it.next(), hk = it.next();
  it.skip(1);
  const int64_t cap = it.next(), dk = it.next();
  LK_REQUIRE(ctx, hq == 128 && hk == 128, "qknorm_rope_kv_f16: heads must be 128 wide");
  LK_REQUIRE(ctx, dk % 128 == 0 && w > 2 * dk && (w - 2 * dk) % 128 == 0, "qknorm_rope_kv_f16: bad qkv width");
  status(ctx, lk_hip_f16_qknorm_rope_kv(a.ptrs[0], a.ptrs[1], a.ptrs[2], P<int64_t>(a, 3), a.ptrs[4], a.ptrs[5],
                                        a.ptrs[6], t, static_cast<int>((w - 2 * dk) / 128),
                                        static_cast<int>(dk / 128), cap, F(a, 0, 1e-6f), F(a, 1, 1e6f), ctx.stream),
         "qknorm_rope_kv_f16: launch failed");
}

// attention_gqa[_opt]: q[T, Dq], kc[P, Dk], vc[P, Dk], pos[1] -> [T, Dq]; attrs kv_heads, q_heads
void runGqaF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), dq = it.next(), cap = it.next(), dk = it.next();
  it.skip(2 + 1 + 2);
  const int kvh = static_cast<int>(it.next()), qh = static_cast<int>(it.next());
  LK_REQUIRE(ctx, kvh > 0 && qh > 0 && qh % kvh == 0 && dq == 128 * qh && dk == 128 * kvh,
             "attention_gqa_f16: head_dim must be 128 and q_heads a multiple of kv_heads");
  const int rc = lk_hip_f16_attention_gqa(a.ptrs[0], a.ptrs[1], a.ptrs[2], P<int64_t>(a, 3), a.ptrs[4], t, qh, kvh,
                                          cap, wsPtr(ctx), wsBytes(ctx), ctx.stream);
  status(ctx, rc, rc == 3 ? "attention_gqa_f16: workspace too small" : "attention_gqa_f16: launch failed");
}

// kv_write (inout kc, vc): kc[P, D], vc[P, D], k[T, D], v[T, D], pos[1]; no outs
void runKvWriteF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t cap = it.next(), d = it.next();
  it.skip(2);
  const int64_t t = it.next();
  status(ctx, lk_hip_f16_kv_write(a.ptrs[0], a.ptrs[1], a.ptrs[2], a.ptrs[3], P<int64_t>(a, 4), t, d, cap, ctx.stream),
         "kv_write_f16: launch failed");
}

// embedding: ids[T], table[V, D] -> [T, D]
void runEmbeddingF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), v = it.next(), d = it.next();
  status(ctx, lk_hip_f16_embedding(P<int64_t>(a, 0), a.ptrs[1], a.ptrs[2], t, v, d, ctx.stream),
         "embedding_f16: launch failed");
}

// scatter_audio: x[T, D], ids[T], audio[A, D] -> [T, D]; attr pad_id
void runScatterAudioF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d = it.next();
  it.skip(1);
  const int64_t na = it.next();
  it.skip(1 + 2);
  const int64_t padId = it.next();
  status(ctx, lk_hip_f16_scatter_audio(a.ptrs[0], P<int64_t>(a, 1), a.ptrs[2], a.ptrs[3], t, d, na, padId, ctx.stream),
         "scatter_audio_f16: launch failed");
}

// attention_decode_qkr_opt (backend; inout kc, vc, counters): qkv[1, W], qg[128], kg[128], pos[1], kc[P, Dk],
// vc[P, Dk], counters i32[qh] -> out f16[1, Dq]; floats eps, theta
void runDecQkrF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  LK_REQUIRE(ctx, it.next() == 1, "attention_decode_qkr_f16: qkv must be f16[1, W]");
  const int64_t w = it.next();
  it.skip(3);
  const int64_t cap = it.next(), dk = it.next();
  it.skip(2);
  const int64_t qh = it.next();
  LK_REQUIRE(ctx, dk % 128 == 0 && w - 2 * dk == 128 * qh, "attention_decode_qkr_f16: bad shapes");
  const int rc = lk_hip_f16_attention_decode_qkr(a.ptrs[0], a.ptrs[1], a.ptrs[2], P<int64_t>(a, 3), a.ptrs[4],
                                                 a.ptrs[5], a.ptrs[7], P<unsigned>(a, 6), static_cast<int>(qh),
                                                 static_cast<int>(dk / 128), cap, F(a, 0, 1e-6f), F(a, 1, 1e6f),
                                                 wsPtr(ctx), wsBytes(ctx), ctx.stream);
  status(ctx, rc, rc == 3 ? "attention_decode_qkr_f16: workspace too small" : "attention_decode_qkr_f16: launch failed");
}

// rmsnorm_lm_head_last_opt (backend): x[T, D], g[D], table[V, D] -> f32[1, V]; float eps
void runRmsLmHeadF16(ExecCtx& ctx, const KernelArgs& a) {
  Ints it(a);
  const int64_t t = it.next(), d = it.next();
  it.skip(1);
  const int64_t v = it.next();
  status(ctx, lk_hip_f16_rms_lm_head(a.ptrs[0], a.ptrs[1], a.ptrs[2], P<float>(a, 3), t, d, v, F(a, 0, 1e-6f),
                                     ctx.stream),
         "rmsnorm_lm_head_last_f16: launch failed");
}

template <int OP>
void runEltF16(ExecCtx& ctx, const KernelArgs& a) {
  status(ctx, lk_hip_f16_elementwise(a.ptrs[0], a.ptrs[1], a.ptrs[2], a.ints[0] * a.ints[1], OP, ctx.stream),
         "elementwise_f16: launch failed");
}

// transpose_f16_gpu (MI355X backend, weight packing): w[K, N] -> [N, K]
void runTransposeF16(ExecCtx& ctx, const KernelArgs& a) {
  status(ctx, lk_hip_f16_transpose(a.ptrs[0], a.ptrs[1], a.ints[0], a.ints[1], ctx.stream), "transpose_f16: failed");
}

}  // namespace

void registerF16Kernels() {
  const Device G = Device::Gpu;
  registerKernel({"gemm_f16_gpu", G, runGemmF16<0>, 2, 1});
  registerKernel({"gemm_opt_f16_gpu", G, runGemmF16<0>, 2, 1});
  registerKernel({"gemm_bias_f16_gpu", G, runGemmF16<1>, 3, 1});
  registerKernel({"gemm_bias_opt_f16_gpu", G, runGemmF16<1>, 3, 1});
  registerKernel({"gemm_add_opt_f16_gpu", G, runGemmF16<2>, 3, 1});
  registerKernel({"gemm_swiglu_opt_f16_gpu", G, runGemmF16<3>, 2, 1});
  registerKernel({"rmsnorm_gemm_opt_f16_gpu", G, runRmsGemmF16<false>, 3, 2});
  registerKernel({"rmsnorm_gemm_swiglu_opt_f16_gpu", G, runRmsGemmF16<true>, 3, 2});
  registerKernel({"lm_head_last_f16_gpu", G, runLmHeadF16, 2, 1});
  registerKernel({"lm_head_last_opt_f16_gpu", G, runLmHeadF16, 2, 1});
  registerKernel({"rmsnorm_f16_gpu", G, runRmsNormF16<false>, 2, 1});
  registerKernel({"rmsnorm_heads_f16_gpu", G, runRmsNormF16<true>, 2, 1});
  registerKernel({"rope_f16_gpu", G, runRopeF16, 2, 1});
  registerKernel({"qknorm_rope_kv_opt_f16_gpu", G, runQkrF16, 6, 1});
  registerKernel({"attention_gqa_f16_gpu", G, runGqaF16, 4, 1});
  registerKernel({"attention_gqa_opt_f16_gpu", G, runGqaF16, 4, 1});
  registerKernel({"kv_write_f16_gpu", G, runKvWriteF16, 5, 0});
  registerKernel({"embedding_f16_gpu", G, runEmbeddingF16, 2, 1});
  registerKernel({"scatter_audio_f16_gpu", G, runScatterAudioF16, 3, 1});
  registerKernel({"add_f16_gpu", G, runEltF16<0>, 2, 1});
  registerKernel({"silu_mul_f16_gpu", G, runEltF16<1>, 2, 1});
  registerKernel({"transpose_f16_gpu", G, runTransposeF16, 1, 1});
  registerKernel({"attention_decode_qkr_opt_f16_gpu", G, runDecQkrF16, 7, 1});
  registerKernel({"rmsnorm_lm_head_last_opt_f16_gpu", G, runRmsLmHeadF16, 3, 1});
}

}  // namespace lkh
