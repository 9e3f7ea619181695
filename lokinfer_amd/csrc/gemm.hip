// f32 GEMM family on CDNA4 matrix cores (v_mfma_f32_32x32x2f32), LDS-staged and double-buffered, with the
// epilogues the reference fuses (bias, ReLU, gelu_tanh, residual, output scale) and two operand loaders:
//   A: row-major [M, lda]              or channel-last implicit im2col of a conv1d input x [L, Ci]
//      (optionally with a per-channel affine + Snake / leaky prologue applied while staging)
//   B: row-major [K, ldb] ("NN")       or row-major B^T [N, ldb] ("NT": conv weights [Co, K*Ci], tied LM heads)
//
// Reference kernels this family replaces (lariaus/lokinfer):
//   gemm_f32_gpu_mps / gemm_nt_f32_gpu_mps      kernels/gpu/mps.mm:41-84
//   gemm_bias[_relu]_f32_gpu                    kernels/gpu/kokoro_lc.cpp:460-581, gemm.metal:82-341
//   gemm_steel*_f32_gpu, gemm_nt_steel_f32_gpu  kernels/gpu/kokoro_lc.cpp:391-409, gemm_steel.metal:81-133
//   conv1d_lc_f32_gpu / conv1d_lc_res_f32_gpu   kernels/gpu/kokoro_lc.cpp:81-109, kokoro_lc.metal:62-128
//   gemv4*_f32_gpu                              kernels/gpu/transformer_gpu.cpp:233-251, kokoro_tok.metal:878-924
//   gemv_rows_f32_gpu, gemv1_bias_f32_gpu       kernels/gpu/kokoro_lc.cpp:227-267, vision.metal:266-284
//
// Design (gfx950): 256-thread workgroups = 4 wave64s in a 2x2 layout; each wave owns a (BM/2)x(BN/2) block of
// 32x32 MFMA tiles and accumulates over K in steps of 2. Per 16-deep K tile both operands are staged in LDS
// k-major ([16][BM], [16][BN]) so that a wave's MFMA operand fetch is 32 consecutive floats per k row.
#include "common.h"
#include "lokinfer_hip.h"

#include <cstdlib>

namespace lkd {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum : int { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };
enum : int { PRE_NONE = 0, PRE_SNAKE = 1, PRE_LEAKY = 2 };
enum : int { A_ROWMAJOR = 0, A_CONV = 1 };
enum : int { B_NN = 0, B_NT = 1 };

struct GemmParams {
  const float* a;
  const float* b;
  const float* bias;  // [N] or null
  const float* res;   // [M, ldr] or null
  float* c;
  int64_t m, n, k;
  int64_t lda, ldb, ldc, ldr;
  int act;
  float scale;
  // conv loader (A_CONV): x = a [L, Ci]; row t reads x[t * stride - pad + kk * dil]
  int64_t convL, convCi;
  int convStride, convPad, convDil;
  // optional prologue on the conv input: v = (x - af[c]) * af[C + c] + af[2C + c]; snake(alpha) / leaky(slope)
  const float* affine;
  const float* alpha;
  int pre;
  float slope;
  // optional per-(128-row chunk, channel) (mean, M2) of the output, [ceil(M / 128), N, 2] (conv tap kernel)
  float* stats;
  // split-K across workgroups (gemmSplitKKernel): grid z = split, K range [z kSplit, (z + 1) kSplit); with
  // splitk > 1 the raw tile sums go to part [splitk][M][N] and gemmSplitReduceKernel applies the epilogue
  float* part;
  int64_t kSplit;
  int splitk;
  // work order: row blocks fastest within an XCD's range (B larger than A: an XCD then reads a slice of B and all
  // of A through its L2), else column blocks fastest
  int yFast;
};

constexpr int BK = 16;
constexpr int NT = 256;

__device__ __forceinline__ float preAct(const GemmParams& p, float v, int c) {
  if (p.affine) {
    const int64_t C = p.convCi;
    v = (v - p.affine[c]) * p.affine[C + c] + p.affine[2 * C + c];
  }
  if (p.pre == PRE_SNAKE) {
    const float a = p.alpha[c];
    v = v + (1.0f / a) * snakeSinSq(a * v);
  } else if (p.pre == PRE_LEAKY) {
    v = v >= 0.0f ? v : v * p.slope;
  }
  return v;
}

// 4 consecutive elements of A along k for row `row`, k0..k0+3 (zero outside the matrix).
template <int AM>
__device__ __forceinline__ float4 loadA4(const GemmParams& p, int64_t row, int64_t k0) {
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
  if (row >= p.m) return r;
  if constexpr (AM == A_ROWMAJOR) {
    const float* src = p.a + row * p.lda + k0;
    if (k0 + 3 < p.k && ((p.lda & 3) == 0)) {
      r = *reinterpret_cast<const float4*>(src);
    } else {
      if (k0 < p.k) r.x = src[0];
      if (k0 + 1 < p.k) r.y = src[1];
      if (k0 + 2 < p.k) r.z = src[2];
      if (k0 + 3 < p.k) r.w = src[3];
    }
  } else {
    // k = kk * Ci + ci, Ci % 16 == 0: a 16-deep K tile never straddles two taps.
    if (k0 >= p.k) return r;
    const int64_t kk = k0 / p.convCi, ci = k0 - kk * p.convCi;
    const int64_t t = row * p.convStride - p.convPad + kk * p.convDil;
    if (t < 0 || t >= p.convL) return r;
    r = *reinterpret_cast<const float4*>(p.a + t * p.convCi + ci);
    if (p.pre != PRE_NONE || p.affine) {
      r.x = preAct(p, r.x, static_cast<int>(ci));
      r.y = preAct(p, r.y, static_cast<int>(ci + 1));
      r.z = preAct(p, r.z, static_cast<int>(ci + 2));
      r.w = preAct(p, r.w, static_cast<int>(ci + 3));
    }
  }
  return r;
}

// NN: 4 consecutive elements of B along n for row k (zero outside).
__device__ __forceinline__ float4 loadBnn4(const GemmParams& p, int64_t k, int64_t n0) {
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
  if (k >= p.k) return r;
  const float* src = p.b + k * p.ldb + n0;
  if (n0 + 3 < p.n && ((p.ldb & 3) == 0)) {
    r = *reinterpret_cast<const float4*>(src);
  } else {
    if (n0 < p.n) r.x = src[0];
    if (n0 + 1 < p.n) r.y = src[1];
    if (n0 + 2 < p.n) r.z = src[2];
    if (n0 + 3 < p.n) r.w = src[3];
  }
  return r;
}

// NT: 4 consecutive elements of B^T along k for column n (zero outside).
__device__ __forceinline__ float4 loadBnt4(const GemmParams& p, int64_t n, int64_t k0) {
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n >= p.n) return r;
  const float* src = p.b + n * p.ldb + k0;
  if (k0 + 3 < p.k && ((p.ldb & 3) == 0)) {
    r = *reinterpret_cast<const float4*>(src);
  } else {
    if (k0 < p.k) r.x = src[0];
    if (k0 + 1 < p.k) r.y = src[1];
    if (k0 + 2 < p.k) r.z = src[2];
    if (k0 + 3 < p.k) r.w = src[3];
  }
  return r;
}

// Writes a wave's TM x TN block of 32x32 accumulators: c = (act(acc + bias) + res) * scale for the elements
// inside the matrix, leaving the stored values in acc. Done in phases (per-column bias, then every residual load,
// then every store) so that no global load sits between two stores: the compiler cannot prove that the output
// does not alias bias or res, and would otherwise wait out a load latency per element. Loads use clamped
// indices; elements outside the matrix are computed but not stored.
// D[i][j] of a 32x32x2 MFMA: j = lane % 32, i = 8 * (r / 4) + 4 * (lane / 32) + r % 4 for accumulator r.
template <int TM, int TN>
__device__ __forceinline__ void storeTile(const GemmParams& p, v16f (&acc)[TM][TN], int64_t rowBase,
                                          int64_t colBase, int lrow, int lk) {
  const int64_t lastRow = p.m - 1, lastCol = p.n - 1;
  float bcol[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) bcol[j] = p.bias ? p.bias[min<int64_t>(colBase + j * 32 + lrow, lastCol)] : 0.0f;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = acc[i][j][r] + bcol[j];
        if (p.act == ACT_RELU) v = fmaxf(v, 0.0f);
        else if (p.act == ACT_GELU) v = geluTanh(v);
        acc[i][j][r] = v;
      }
  if (p.res) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col = min<int64_t>(colBase + j * 32 + lrow, lastCol);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = min<int64_t>(rowBase + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3), lastRow);
          acc[i][j][r] += p.res[row * p.ldr + col];
        }
      }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = colBase + j * 32 + lrow;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = rowBase + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        acc[i][j][r] *= p.scale;
        if (row <= lastRow && col <= lastCol) p.c[row * p.ldc + col] = acc[i][j][r];
      }
    }
}

// The general form (FAST = false) is held to 168 VGPRs, three waves per SIMD (10 spills, outside the K loop's
// MFMA body): 162 -> 123 us on the Kokoro decoder's im2col conv GEMM. The FAST form fits 168 by itself.
template <int BM, int BN, int AM, int BMODE, bool FAST = false>
__global__ __launch_bounds__(NT, FAST ? 2 : 3) void gemmMfmaKernel(GemmParams p) {
  constexpr int WTM = BM / 2, WTN = BN / 2;    // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA tiles per wave
  constexpr int PADA = 4, PADB = 4;
  constexpr int LDA_S = BM + PADA, LDB_S = BN + PADB;
  constexpr int A4 = BM * BK / 4 / NT;  // float4 loads per thread (A tile)
  constexpr int B4 = BN * BK / 4 / NT;
  static_assert(A4 >= 1 && B4 >= 1, "tile too small for 256 threads");

  __shared__ float As[2][BK][LDA_S];
  __shared__ float Bs[2][BK][LDB_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const GridItem gi = xcdOrder();  // column blocks of one row block share an XCD's L2
  const int64_t m0 = static_cast<int64_t>(gi.y) * BM;
  const int64_t n0 = static_cast<int64_t>(gi.x) * BN;

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // FAST (row-major A, 16-byte aligned operands, K % BK == 0, N % 4 == 0 for NN; checked by the launcher):
  // float4 loads from clamped indices (rows / columns past the matrix feed outputs that are never stored) into
  // two register sets, issued unconditionally one stage ahead of their LDS store, pairs of stages with no branch
  // inside (a load or store behind a branch makes the compiler's wait counting assume the path without it).
  // Otherwise one register set with element-guarded loads.
  using RA = float4[A4];
  using RB = float4[B4];
  float4 ra0[A4], rb0[B4], ra1[A4], rb1[B4];
  const int64_t lastRow = p.m - 1, lastCol = p.n - 1;
  auto gload = [&](int64_t kt, RA& ra, RB& rb) {
    const int64_t k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx >> 2, kq = (idx & 3) * 4;
      if constexpr (FAST)
        ra[i] = *reinterpret_cast<const float4*>(p.a + min<int64_t>(m0 + row, lastRow) * p.lda + k0 + kq);
      else
        ra[i] = loadA4<AM>(p, m0 + row, k0 + kq);
    }
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int idx = tid + i * NT;
      if constexpr (BMODE == B_NN) {
        const int kr = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
        if constexpr (FAST)
          rb[i] = *reinterpret_cast<const float4*>(p.b + (k0 + kr) * p.ldb + min<int64_t>(n0 + nq, p.n - 4));
        else
          rb[i] = loadBnn4(p, k0 + kr, n0 + nq);
      } else {
        const int col = idx >> 2, kq = (idx & 3) * 4;
        if constexpr (FAST)
          rb[i] = *reinterpret_cast<const float4*>(p.b + min<int64_t>(n0 + col, lastCol) * p.ldb + k0 + kq);
        else
          rb[i] = loadBnt4(p, n0 + col, k0 + kq);
      }
    }
  };
  auto sstore = [&](int buf, const RA& ra, const RB& rb) {
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx >> 2, kq = (idx & 3) * 4;
      As[buf][kq + 0][row] = ra[i].x;
      As[buf][kq + 1][row] = ra[i].y;
      As[buf][kq + 2][row] = ra[i].z;
      As[buf][kq + 3][row] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int idx = tid + i * NT;
      if constexpr (BMODE == B_NN) {
        const int kr = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[buf][kr][nq]) = rb[i];
      } else {
        const int col = idx >> 2, kq = (idx & 3) * 4;
        Bs[buf][kq + 0][col] = rb[i].x;
        Bs[buf][kq + 1][col] = rb[i].y;
        Bs[buf][kq + 2][col] = rb[i].z;
        Bs[buf][kq + 3][col] = rb[i].w;
      }
    }
  };

  const int64_t nk = (p.k + BK - 1) / BK;
  const int lrow = lane & 31, lk = lane >> 5;
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK; ks += 2) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = As[buf][ks + lk][wm * WTM + i * 32 + lrow];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bs[buf][ks + lk][wn * WTN + j * 32 + lrow];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  };
  gload(0, ra0, rb0);
  sstore(0, ra0, rb0);
  if constexpr (FAST) {
    // stage kt computes from buffer kt & 1 while stage kt + 1 (register set (kt + 1) & 1) is in flight; it
    // stores that set into the other buffer at its end (the last stage stores an unread copy)
    gload(min<int64_t>(1, nk - 1), ra1, rb1);
    __syncthreads();
    auto stage = [&](int64_t kt, RA& nra, RB& nrb, RA& fra, RB& frb) {
      mfmas(static_cast<int>(kt & 1));
      sstore(static_cast<int>((kt + 1) & 1), nra, nrb);
      gload(min<int64_t>(kt + 2, nk - 1), fra, frb);
      __syncthreads();
    };
    int64_t kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      stage(kt, ra1, rb1, ra0, rb0);
      stage(kt + 1, ra0, rb0, ra1, rb1);
    }
    if (kt < nk) stage(kt, ra1, rb1, ra0, rb0);
  } else {
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
      const int buf = static_cast<int>(kt & 1);
      if (kt + 1 < nk) gload(kt + 1, ra0, rb0);
      mfmas(buf);
      if (kt + 1 < nk) sstore(buf ^ 1, ra0, rb0);
      __syncthreads();
    }
  }

  storeTile<TM, TN>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lrow, lk);
}

// GEMM for few output tiles (M of a few hundred, e.g. ALBERT at T = 487 or an LSTM input projection): 64 x BN
// workgroup tiles with K staged 64 deep, and wave w of the 4 computing the WHOLE tile over k-slice w (16 deep) of
// every stage. One barrier then covers 8 * 2 * BN / 32 MFMAs per wave (32 at BN = 64) instead of the 8 of a
// 64x64 tile split 2x2 over the waves; the four partial tiles are summed through LDS in a fixed order at the end
// (deterministic), followed by the phased epilogue. A: row-major [M, lda]. B: NN [K, ldb] staged k-major
// ([k][BN + 8]: the two lane halves of a read sit 4 rows = 32 banks apart), or NT [N, ldb] staged like A.
// A (and NT B) tiles are [row][4 slots of 4 k], slot swizzled by (row >> 2) & 3; a slice's 16 k are fed to the
// MFMAs in the order 8 g + 4 half + q, as in the conv kernel. Needs K, lda, ldb (and N for NN) % 4 == 0 and
// 16-byte aligned operands (checked by the launcher).
// KTAIL: K is not a multiple of the 64-deep stage, so the last stage's tail is zeroed when staged (without it,
// no select on the loaded registers exists to pull the wait for a load ahead of the MFMAs that cover it).
template <int BN, int BMODE, bool KTAIL>
__global__ __launch_bounds__(NT, 2) void gemmSplitKKernel(GemmParams p) {
  constexpr int BM = 64, KS = 64;
  constexpr int TM = 2, TN = BN / 32;
  constexpr int LDBK = BN + 8;
  constexpr int A4 = BM * KS / 4 / NT, B4 = BN * KS / 4 / NT;
  constexpr int A_FL = 2 * 4 * BM * 16;                                // floats of the A buffers
  constexpr int B_FL = BMODE == B_NN ? 2 * KS * LDBK : 2 * 4 * BN * 16;
  constexpr int RED_FL = 4 * BM * BN;
  constexpr int SMEM = A_FL + B_FL > RED_FL ? A_FL + B_FL : RED_FL;
  static_assert(A4 >= 1 && B4 >= 1, "staging slots");
  __shared__ __attribute__((aligned(16))) float smem[SMEM];
  v4f* As = reinterpret_cast<v4f*>(smem);             // [buf][slice][BM * 4]
  float* Bsf = smem + A_FL;                            // NN: [buf][KS * LDBK]
  v4f* Bsv = reinterpret_cast<v4f*>(smem + A_FL);     // NT: [buf][slice][BN * 4]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, lk = lane >> 5;
  const GridItem gi = p.yFast ? xcdOrderYFast() : xcdOrder();
  const int64_t m0 = static_cast<int64_t>(gi.y) * BM, n0 = static_cast<int64_t>(gi.x) * BN;
  const int64_t lastRow = p.m - 1, lastCol = p.n - 1;
  // this workgroup's K range (the whole K without a split)
  const int64_t kb = p.splitk > 1 ? gi.z * p.kSplit : 0;
  const int64_t ke = p.splitk > 1 ? min<int64_t>(kb + p.kSplit, p.k) : p.k;

  // two register sets: the next stage's tile is stored to LDS while the one after it is still in flight
  v4f ra[2][A4], rb[2][B4];
  auto gload = [&](int64_t k0, v4f (&ra)[A4], v4f (&rb)[B4]) {
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int idx = tid + i * NT, row = idx >> 4, kq = (idx & 15) * 4;
      ra[i] = *reinterpret_cast<const v4f*>(p.a + min<int64_t>(m0 + row, lastRow) * p.lda +
                                            min<int64_t>(k0 + kq, ke - 4));
    }
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int idx = tid + i * NT;
      if constexpr (BMODE == B_NN) {
        const int kr = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
        rb[i] = *reinterpret_cast<const v4f*>(p.b + min<int64_t>(k0 + kr, ke - 1) * p.ldb +
                                              min<int64_t>(n0 + nq, p.n - 4));
      } else {
        const int col = idx >> 4, kq = (idx & 15) * 4;
        rb[i] = *reinterpret_cast<const v4f*>(p.b + min<int64_t>(n0 + col, lastCol) * p.ldb +
                                              min<int64_t>(k0 + kq, ke - 4));
      }
    }
  };
  // The k tail (k >= K, loaded from clamped addresses) is zeroed here, when the data is first touched, so that
  // no wait for the loads sits between their issue and the MFMAs.
  auto sstore = [&](int buf, int64_t k0, const v4f (&ra)[A4], const v4f (&rb)[B4]) {
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int idx = tid + i * NT, row = idx >> 4, kq = (idx & 15) * 4;
      const int slice = kq >> 4, slot = (kq >> 2) & 3;
      As[(buf * 4 + slice) * BM * 4 + row * 4 + (slot ^ ((row >> 2) & 3))] = !KTAIL || k0 + kq < ke ? ra[i] : zero;
    }
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int idx = tid + i * NT;
      if constexpr (BMODE == B_NN) {
        const int kr = idx / (BN / 4), nq = (idx % (BN / 4)) * 4;
        *reinterpret_cast<v4f*>(Bsf + buf * KS * LDBK + kr * LDBK + nq) = !KTAIL || k0 + kr < ke ? rb[i] : zero;
      } else {
        const int col = idx >> 4, kq = (idx & 15) * 4;
        const int slice = kq >> 4, slot = (kq >> 2) & 3;
        Bsv[(buf * 4 + slice) * BN * 4 + col * 4 + (slot ^ ((col >> 2) & 3))] = !KTAIL || k0 + kq < ke ? rb[i] : zero;
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t stages = (ke - kb + KS - 1) / KS;
  auto stage = [&](int64_t st, int buf, v4f (&ra_next)[A4], v4f (&rb_next)[B4], v4f (&ra_far)[A4],
                   v4f (&rb_far)[B4]) {
    v4f af[2][TM];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = i * 32 + lr;
        af[g][i] = As[(buf * 4 + wave) * BM * 4 + row * 4 + ((2 * g + lk) ^ ((row >> 2) & 3))];
      }
    float bq[2][4][TN];
    if constexpr (BMODE == B_NN) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            bq[g][q][j] = Bsf[buf * KS * LDBK + (16 * wave + 8 * g + 4 * lk + q) * LDBK + j * 32 + lr];
    } else {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = j * 32 + lr;
          const v4f bv = Bsv[(buf * 4 + wave) * BN * 4 + col * 4 + ((2 * g + lk) ^ ((col >> 2) & 3))];
#pragma unroll
          for (int q = 0; q < 4; ++q) bq[g][q][j] = bv[q];
        }
    }
    // unconditional, clamped to the last stage (a load or store behind a branch makes the compiler's wait
    // counting assume the path without it, i.e. wait for the loads just issued before every LDS store)
    gload(kb + min<int64_t>(st + 2, stages - 1) * KS, ra_far, rb_far);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[g][i][q], bq[g][q][j], acc[i][j], 0, 0, 0);
    sstore(buf ^ 1, kb + min<int64_t>(st + 1, stages - 1) * KS, ra_next, rb_next);  // last stage: unread copy
    __syncthreads();
  };
  // stage st computes from LDS buffer st & 1, stores stage st + 1 (register set (st + 1) & 1) and has stage st + 2
  // in flight into register set st & 1; pairs of stages with no branch inside, an odd last stage peeled
  gload(kb, ra[0], rb[0]);
  sstore(0, kb, ra[0], rb[0]);
  gload(kb + min<int64_t>(1, stages - 1) * KS, ra[1], rb[1]);
  __syncthreads();
  int64_t st = 0;
  for (; st + 1 < stages; st += 2) {
    stage(st, 0, ra[1], rb[1], ra[0], rb[0]);
    stage(st + 1, 1, ra[0], rb[0], ra[1], rb[1]);
  }
  if (st < stages) stage(st, 0, ra[1], rb[1], ra[0], rb[0]);

  // partial tiles -> LDS (the staging buffers are free after the last barrier), fixed-order sum, epilogue
  float* red = smem;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        red[(wave * BM + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3)) * BN + j * 32 + lr] = acc[i][j][r];
  __syncthreads();
  constexpr int PER = BM * BN / NT;  // outputs per thread: 4 threads per row, PER contiguous columns each
  const int row = tid >> 2, c0 = (tid & 3) * PER;
  const int64_t grow = m0 + row;
  float v[PER];
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const int o = row * BN + c0 + c;
    v[c] = ((red[o] + red[BM * BN + o]) + red[2 * BM * BN + o]) + red[3 * BM * BN + o];
  }
  if (p.splitk > 1) {  // raw sums of this K range; the reduction applies the epilogue
    float* pp = p.part + static_cast<int64_t>(gi.z) * p.m * p.n;
    if (grow <= lastRow) {
#pragma unroll
      for (int c = 0; c < PER; ++c) {
        const int64_t gcol = n0 + c0 + c;
        if (gcol <= lastCol) pp[grow * p.n + gcol] = v[c];
      }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const int64_t gcol = min<int64_t>(n0 + c0 + c, lastCol);
    float x = v[c] + (p.bias ? p.bias[gcol] : 0.0f);
    if (p.act == ACT_RELU) x = fmaxf(x, 0.0f);
    else if (p.act == ACT_GELU) x = geluTanh(x);
    v[c] = x;
  }
  if (p.res) {
#pragma unroll
    for (int c = 0; c < PER; ++c)
      v[c] += p.res[min<int64_t>(grow, lastRow) * p.ldr + min<int64_t>(n0 + c0 + c, lastCol)];
  }
  if (grow <= lastRow) {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int64_t gcol = n0 + c0 + c;
      if (gcol <= lastCol) p.c[grow * p.ldc + gcol] = v[c] * p.scale;
    }
  }
}

// Split-K reduction of gemmSplitKKernel: c = (act(sum_z part[z] + bias) + res) * scale, the z sum in order.
__global__ __launch_bounds__(256) void gemmSplitReduceKernel(GemmParams p) {
  const int64_t total = p.m * p.n;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / p.n, col = i - row * p.n;
    float x = 0.0f;
#pragma unroll
    for (int z = 0; z < 8; ++z)  // splitk <= 8, predicated so the loads are issued together
      if (z < p.splitk) x += p.part[z * total + i];
    x += p.bias ? p.bias[col] : 0.0f;
    if (p.act == ACT_RELU) x = fmaxf(x, 0.0f);
    else if (p.act == ACT_GELU) x = geluTanh(x);
    if (p.res) x += p.res[row * p.ldr + col];
    p.c[row * p.ldc + col] = x * p.scale;
  }
}

// Stride-1 channel-last conv with the taps innermost. For each 16-channel input chunk a workgroup stages the
// halo rows its BM output rows need (BM + (K-1) dil rows x 16 channels) once, with the affine + Snake / leaky
// prologue applied once per element; then every tap kk is a 16-deep MFMA step whose A operand is the same halo
// shifted by kk * dil rows and whose B operand is w[n0 .., kk, chunk] (16 contiguous floats per output channel
// in the [Co, K, Ci] weight). Compared with the flat im2col loop this reads each input element from L2 once per
// chunk instead of K times and evaluates the prologue once instead of K times. Steps = chunks x taps,
// double-buffered: B per step, the halo per chunk (prefetched into registers during the chunk's last tap).
//
// LDS layout: both operands row-major with their 16 channels contiguous ([row][16], row stride 20 floats), so a
// global float4 lands in LDS as one float4 (no transposition) and 16 consecutive rows of 16-byte reads cover all
// 64 banks once. The 16 channels of a chunk are fed to the MFMAs in the order ch(g, q, half) = 8 g + 4 half + q
// (MFMA step 4 g + q, lane half = lane / 32): a lane's 8 operand values of one tap are then two 16-byte reads
// per 32-row block, for A and B alike; the k order inside a chunk does not change the sum's terms.
constexpr int kLdRow = 20;  // floats per staged row (16 channels + 4 pad)

template <int BM>
struct TapCfg {
  static constexpr int maxHalo = BM == 128 ? 192 : 128;  // rows of halo the LDS holds (BM + (K-1) dil <= this)
};

template <int BM, int BN>
// 64 x 64: at most 168 VGPRs, three waves per SIMD (12 per CU) keep the MFMA pipe fed through the barriers.
// 128 x 128 needs 254 VGPRs: bounded to three waves it spilled 77 of them and ran 222 vs 159 us on the Kokoro
// decoder's conv, so it runs two.
__global__ __launch_bounds__(NT, BM == 128 ? 2 : 3) void convTapKernel(GemmParams p, int taps, int halo) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int MAXH = TapCfg<BM>::maxHalo;
  constexpr int B4 = BN * BK / 4 / NT;
  constexpr int H4 = MAXH * BK / 4 / NT;  // halo 4-float slots per thread
  static_assert(B4 >= 1 && H4 >= 1 && (MAXH * BK / 4) % NT == 0, "staging slots");

  __shared__ v4f Hs[2][MAXH * kLdRow / 4];
  __shared__ v4f Bs[2][BN * kLdRow / 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const GridItem gi = xcdOrder();  // column blocks of one row block share an XCD's L2
  const int64_t m0 = static_cast<int64_t>(gi.y) * BM;
  const int64_t n0 = static_cast<int64_t>(gi.x) * BN;
  const int64_t ci = p.convCi;
  // split-K (grid z): this workgroup's 16-channel chunks [cb, ce); the whole range without a split
  const int allChunks = static_cast<int>(ci / BK);
  const int cb = p.splitk > 1 ? static_cast<int>(gi.z * p.kSplit) : 0;
  const int ce = p.splitk > 1 ? min(allChunks, static_cast<int>(cb + p.kSplit)) : allChunks;
  const int steps = (ce - cb) * taps;
  const int64_t rowBase = m0 - p.convPad;  // input row of halo row 0
  const int cq = (tid & 3) * 4;            // the 4 channels of a chunk this thread stages (same for every slot)
  const int lastRow = static_cast<int>(p.convL - 1);

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  v4f rh[H4], rb[B4];
  const bool hasPre = p.pre != PRE_NONE || p.affine;
  // Raw halo loads from clamped rows (always in bounds, no branches); rows outside [0, L) become zero padding
  // at store time, after the prologue.
  auto loadHalo = [&](int chunk) {
    const float* src = p.a + static_cast<int64_t>(chunk) * BK + cq;
#pragma unroll
    for (int i = 0; i < H4; ++i) {
      const int hr = (tid + i * NT) >> 2;
      const int64_t t = min<int64_t>(max<int64_t>(rowBase + hr, 0), lastRow);
      if (hr < halo) rh[i] = *reinterpret_cast<const v4f*>(src + t * ci);
    }
  };
  // The prologue's per-channel parameters of a chunk (this thread's 4 channels): four 16-byte loads issued
  // together when the chunk's halo is stored (registers are not held across the MFMAs for them).
  v4f pmu = {0.f, 0.f, 0.f, 0.f}, psc = {1.f, 1.f, 1.f, 1.f}, pbe = {0.f, 0.f, 0.f, 0.f};
  v4f pal = {1.f, 1.f, 1.f, 1.f};
  auto loadParams = [&](int chunk) {
    const int64_t c0 = static_cast<int64_t>(chunk) * BK + cq;
    if (p.affine) {
      pmu = *reinterpret_cast<const v4f*>(p.affine + c0);
      psc = *reinterpret_cast<const v4f*>(p.affine + ci + c0);
      pbe = *reinterpret_cast<const v4f*>(p.affine + 2 * ci + c0);
    }
    if (p.pre == PRE_SNAKE) pal = *reinterpret_cast<const v4f*>(p.alpha + c0);
  };
  auto storeHalo = [&](int buf, int chunk) {
    if (hasPre) loadParams(chunk);
    float mu[4] = {pmu.x, pmu.y, pmu.z, pmu.w}, sc[4] = {psc.x, psc.y, psc.z, psc.w};
    float be[4] = {pbe.x, pbe.y, pbe.z, pbe.w}, al[4] = {pal.x, pal.y, pal.z, pal.w}, ial[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) ial[q] = 1.0f / al[q];
#pragma unroll
    for (int i = 0; i < H4; ++i) {
      const int hr = (tid + i * NT) >> 2;
      if (hr >= halo) continue;  // slots past this conv's halo are never read
      const int64_t t = rowBase + hr;
      float e[4] = {rh[i].x, rh[i].y, rh[i].z, rh[i].w};
      if (hasPre) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float u = p.affine ? (e[q] - mu[q]) * sc[q] + be[q] : e[q];
          if (p.pre == PRE_SNAKE) {
            u = u + ial[q] * snakeSinSq(al[q] * u);
          } else if (p.pre == PRE_LEAKY) {
            u = u >= 0.0f ? u : u * p.slope;
          }
          e[q] = u;
        }
      }
      const bool inside = t >= 0 && t <= lastRow;  // zero padding is applied after the prologue
      Hs[buf][hr * (kLdRow / 4) + (cq >> 2)] =
          inside ? v4f{e[0], e[1], e[2], e[3]} : v4f{0.f, 0.f, 0.f, 0.f};
    }
  };
  // B for step s = chunk * taps + kk: w[co][kk][chunk * 16 .. +15] (w is [Co, K, Ci] row-major = ldb K * Ci);
  // columns past N read the last valid row (never stored).
  auto loadB = [&](int s) {
    const int chunk = cb + s / taps, kk = s % taps;
    const float* src = p.b + static_cast<int64_t>(kk) * ci + static_cast<int64_t>(chunk) * BK + cq;
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int col = (tid + i * NT) >> 2;
      const int64_t n = min<int64_t>(n0 + col, p.n - 1);
      rb[i] = *reinterpret_cast<const v4f*>(src + n * p.ldb);
    }
  };
  auto storeB = [&](int buf) {
#pragma unroll
    for (int i = 0; i < B4; ++i) {
      const int col = (tid + i * NT) >> 2;
      Bs[buf][col * (kLdRow / 4) + (cq >> 2)] = rb[i];
    }
  };

  loadHalo(cb);
  storeHalo(0, cb);
  loadB(0);
  storeB(0);
  __syncthreads();
  const int lrow = lane & 31, lk = lane >> 5;
  const int aRow = wm * WTM + lrow, bRow = wn * WTN + lrow;
  for (int s = 0; s < steps; ++s) {
    const int lc = s / taps, kk = s - lc * taps, chunk = cb + lc;
    const int hbuf = lc & 1, bbuf = s & 1;
    const bool more = s + 1 < steps;
    const bool newChunk = more && kk == taps - 1;
    const int shift = kk * p.convDil;
    // this step's operand fragments first, then the next step's global prefetch (consumed after the MFMAs)
    v4f af[2][TM], bf[2][TN];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int i = 0; i < TM; ++i) af[g][i] = Hs[hbuf][(aRow + i * 32 + shift) * (kLdRow / 4) + 2 * g + lk];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[g][j] = Bs[bbuf][(bRow + j * 32) * (kLdRow / 4) + 2 * g + lk];
    }
    if (more) loadB(s + 1);
    if (newChunk) loadHalo(chunk + 1);
    // raised issue priority while this wave has MFMAs to issue (other waves' staging work yields to it)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[g][i][q], bf[g][j][q], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    if (more) storeB(bbuf ^ 1);
    if (newChunk) storeHalo(hbuf ^ 1, chunk + 1);
    __syncthreads();
  }

  if (p.splitk > 1) {  // raw partial tile of this chunk range; gemmSplitReduceKernel applies the epilogue
    float* pp = p.part + static_cast<int64_t>(gi.z) * p.m * p.n;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col = n0 + wn * WTN + j * 32 + lrow;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (row < p.m && col < p.n) pp[row * p.n + col] = acc[i][j][r];
        }
      }
    return;
  }
  storeTile<TM, TN>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lrow, lk);
  if (BM == 128 && p.stats) {
    // Per-(128-row chunk, channel) (mean, M2) of the stored output, two passes over the registers: this tile is
    // exactly chunk gi.y. A column's 128 rows sit in (wm, i, lane half, r); reduce r and i in registers,
    // the two lane halves with a shuffle, and the two wm waves through LDS.
    float* red = reinterpret_cast<float*>(&Hs[0][0]);  // reuse the staging LDS (free after the last barrier)
    const int n = static_cast<int>(min<int64_t>(BM, p.m - m0));
    float colSum[TN], colM2[TN], mean[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rloc = wm * WTM + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (rloc < n) s += acc[i][j][r];
        }
      colSum[j] = s + __shfl_xor(s, 32, 64);
    }
    if (lk == 0)
#pragma unroll
      for (int j = 0; j < TN; ++j) red[wm * BN + wn * WTN + j * 32 + lrow] = colSum[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = wn * WTN + j * 32 + lrow;
      mean[j] = (red[c] + red[BN + c]) / static_cast<float>(n);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rloc = wm * WTM + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          const float d = acc[i][j][r] - mean[j];
          if (rloc < n) s += d * d;
        }
      colM2[j] = s + __shfl_xor(s, 32, 64);
    }
    if (lk == 0)
#pragma unroll
      for (int j = 0; j < TN; ++j) red[wm * BN + wn * WTN + j * 32 + lrow] = colM2[j];
    __syncthreads();
    if (wm == 0 && lk == 0)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int c = wn * WTN + j * 32 + lrow;
        const int64_t col = n0 + c;
        if (col < p.n) {
          float* st = p.stats + (static_cast<int64_t>(gi.y) * p.n + col) * 2;
          st[0] = mean[j];
          st[1] = red[c] + red[BN + c];
        }
      }
  }
}

}  // namespace lkd

namespace lkh {

using lkd::GemmParams;

// Tile choice: 128x128 when it still yields a few hundred workgroups, else 64x64 (small M, e.g. ALBERT at
// T = 59 or the MNIST layers).
template <int AM, int BMODE>
static void launchGemm(GemmParams p, hipStream_t s, void* ws = nullptr, int64_t wsBytes = 0) {
  const int64_t big = static_cast<int64_t>(ceilDiv(p.m, 128)) * ceilDiv(p.n, 128);
  const bool aligned = ((reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.b)) & 15) == 0 &&
                       p.k % 4 == 0 && p.lda % 4 == 0 && p.ldb % 4 == 0 && p.k >= 4 &&
                       (BMODE == lkd::B_NT || (p.n % 4 == 0 && p.n >= 4));
  if (big >= 512) {
    dim3 grid(ceilDiv(p.n, 128), ceilDiv(p.m, 128));
    if (AM == lkd::A_ROWMAJOR && aligned && p.k % lkd::BK == 0)
      hipLaunchKernelGGL((lkd::gemmMfmaKernel<128, 128, AM, BMODE, AM == lkd::A_ROWMAJOR>), grid, dim3(lkd::NT), 0, s,
                         p);
    else
      hipLaunchKernelGGL((lkd::gemmMfmaKernel<128, 128, AM, BMODE>), grid, dim3(lkd::NT), 0, s, p);
  } else if (AM == lkd::A_ROWMAJOR && aligned) {
    p.yFast = p.n > p.m ? 1 : 0;  // consecutive workgroups on one XCD walk the longer output dimension
    // few output tiles: K split over the waves of a workgroup; 32-column tiles unless the 64-column grid alone
    // already gives every CU two workgroups (at M ~ 500, N = 2304 / 3072, 288-384 wide tiles left the last round
    // of workgroups a fraction of the chip: 40.9 -> 32.7 us and 42.8 -> 34.2 us with 32 columns)
    const bool wide = static_cast<int64_t>(ceilDiv(p.m, 64)) * ceilDiv(p.n, 64) >= 512;
    const int64_t tiles = static_cast<int64_t>(ceilDiv(p.n, wide ? 64 : 32)) * ceilDiv(p.m, 64);
    // and across workgroups when the grid still leaves CUs idle and K is long: 64-aligned K ranges of at least
    // 256, partial tiles in the workspace past its 64 KiB counter area, summed by gemmSplitReduceKernel
    // Long K over under 256 tiles (GPT-2's 512 x 3072 -> 768 MLP projection, ALBERT's 2048-deep FFN output) splits
    // in 4 too: 40.3 -> 33.5 us and 29.1 -> 27.8 us, where shorter K or more tiles only pay the reduction.
    int split = 1;
    if (ws && tiles < 256 && tiles >= 128 && p.k >= 2048) {
      split = static_cast<int>(std::min<int64_t>(4, p.k / 512));
      while (split > 1 && 65536 + static_cast<int64_t>(split) * p.m * p.n * 4 > wsBytes) --split;
    } else if (ws && tiles < 128 && p.k >= 512) {
      split = static_cast<int>(std::min<int64_t>({8, 512 / tiles, p.k / 256}));
      while (split > 1 && 65536 + static_cast<int64_t>(split) * p.m * p.n * 4 > wsBytes) --split;
      split = std::max(split, 1);
    }
    if (split > 1) {
      p.kSplit = ((p.k + split - 1) / split + 63) / 64 * 64;
      split = static_cast<int>((p.k + p.kSplit - 1) / p.kSplit);
      p.splitk = split;
      p.part = reinterpret_cast<float*>(static_cast<char*>(ws) + 65536);
    }
    const dim3 grid(ceilDiv(p.n, wide ? 64 : 32), ceilDiv(p.m, 64), static_cast<unsigned>(split));
    if (wide) {
      if (p.k % 64)
        hipLaunchKernelGGL((lkd::gemmSplitKKernel<64, BMODE, true>), grid, dim3(lkd::NT), 0, s, p);
      else
        hipLaunchKernelGGL((lkd::gemmSplitKKernel<64, BMODE, false>), grid, dim3(lkd::NT), 0, s, p);
    } else {
      if (p.k % 64)
        hipLaunchKernelGGL((lkd::gemmSplitKKernel<32, BMODE, true>), grid, dim3(lkd::NT), 0, s, p);
      else
        hipLaunchKernelGGL((lkd::gemmSplitKKernel<32, BMODE, false>), grid, dim3(lkd::NT), 0, s, p);
    }
    if (split > 1)
      hipLaunchKernelGGL(lkd::gemmSplitReduceKernel,
                         dim3(static_cast<unsigned>(std::min<int64_t>((p.m * p.n + 255) / 256, 8192))), dim3(256), 0,
                         s, p);
  } else {
    dim3 grid(ceilDiv(p.n, 64), ceilDiv(p.m, 64));
    hipLaunchKernelGGL((lkd::gemmMfmaKernel<64, 64, AM, BMODE>), grid, dim3(lkd::NT), 0, s, p);
  }
}

static GemmParams baseParams() {
  GemmParams p{};
  p.scale = 1.0f;
  p.convStride = 1;
  p.convDil = 1;
  return p;
}

}  // namespace lkh


// ---- typed C-ABI launchers ---------------------------------------------------------------------------------
extern "C" {

// out[M, N] = act(A[M, K] . B + bias) + res, then * scale. nt: B is given as B^T [N, K].
int lk_hip_gemm_f32(const float* a, const float* b, const float* bias, const float* res, float* out, int64_t m,
                    int64_t n, int64_t k, int nt, int act, float scale, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  if (m <= 0 || n <= 0 || k <= 0) return m >= 0 && n >= 0 && k >= 0 ? 0 : 1;
  lkd::GemmParams p = lkh::baseParams();
  p.a = a;
  p.b = b;
  p.bias = bias;
  p.res = res;
  p.c = out;
  p.m = m;
  p.n = n;
  p.k = k;
  p.lda = k;
  p.ldb = nt ? k : n;
  p.ldc = n;
  p.ldr = n;
  p.act = act;
  p.scale = scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nt) lkh::launchGemm<lkd::A_ROWMAJOR, lkd::B_NT>(p, s, workspace, workspace_bytes);
  else lkh::launchGemm<lkd::A_ROWMAJOR, lkd::B_NN>(p, s, workspace, workspace_bytes);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Split-K partials part[s] = A[:, s K/S : (s+1) K/S] . B[s K/S : (s+1) K/S, :] for s < splits, part [S, M, N]; the
// consumer sums the planes (lk_hip_add_bias_ln_sk_f32). K % (16 splits) == 0, K, N % 4 == 0, 16-byte aligned.
int lk_hip_gemm_splitk_f32(const float* a, const float* b, float* part, int64_t m, int64_t n, int64_t k, int splits,
                           void* stream) {
  if (splits < 1 || splits > 64 || k <= 0 || k % (16 * splits) != 0 || n % 4 != 0 || n <= 0) return 1;
  if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) != 0) return 1;
  if (m <= 0) return m == 0 ? 0 : 1;
  lkd::GemmParams p = lkh::baseParams();
  p.a = a;
  p.b = b;
  p.c = part;
  p.m = m;
  p.n = n;
  p.k = k;
  p.lda = k;
  p.ldb = n;
  p.ldc = n;
  p.ldr = n;
  if (splits > 1) {
    p.splitk = splits;
    p.kSplit = k / splits;
    p.part = part;
  }
  const int64_t kRange = k / splits;
  const bool wide = static_cast<int64_t>(lkh::ceilDiv(m, 64)) * lkh::ceilDiv(n, 64) * splits >= 192;
  const dim3 grid(lkh::ceilDiv(n, wide ? 64 : 32), lkh::ceilDiv(m, 64), static_cast<unsigned>(splits));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (wide) {
    if (kRange % 64)
      hipLaunchKernelGGL((lkd::gemmSplitKKernel<64, lkd::B_NN, true>), grid, dim3(lkd::NT), 0, s, p);
    else
      hipLaunchKernelGGL((lkd::gemmSplitKKernel<64, lkd::B_NN, false>), grid, dim3(lkd::NT), 0, s, p);
  } else {
    if (kRange % 64)
      hipLaunchKernelGGL((lkd::gemmSplitKKernel<32, lkd::B_NN, true>), grid, dim3(lkd::NT), 0, s, p);
    else
      hipLaunchKernelGGL((lkd::gemmSplitKKernel<32, lkd::B_NN, false>), grid, dim3(lkd::NT), 0, s, p);
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Channel-last conv1d as an implicit GEMM: x [L, Ci] (Ci % 16 == 0), w [Co, K, Ci], bias [Co] (or null),
// res [Lo, Co] (or null) -> out [Lo, Co] = (conv(pre(x)) + bias + res) * scale; pre = optional affine [3, Ci]
// then snake(alpha [Ci]) (pre = 1) or leaky(slope) (pre = 2); zero padding applies after pre.
int lk_hip_conv1d_lc_f32(const float* x, const float* w, const float* bias, const float* res, float* out, int64_t l,
                         int64_t ci, int64_t co, int64_t kw, int stride, int padding, int dilation, float scale,
                         const float* affine, const float* alpha, int pre, float slope, float* stats, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (ci % 16 != 0 || stride < 1 || dilation < 1 || padding < 0) return 1;
  const int64_t lo = (l + 2 * padding - static_cast<int64_t>(dilation) * (kw - 1) - 1) / stride + 1;
  if (lo <= 0 || co <= 0) return lo == 0 ? 0 : 1;
  if (kw == 1 && stride == 1 && padding == 0 && pre == 0 && !affine) {
    // one tap, no prologue: out = x W^T (+ bias, + res, * scale), the GEMM entry's NT form (W [Co, 1, Ci] = [Co, Ci])
    const int rc = lk_hip_gemm_f32(x, w, bias, res, out, lo, co, ci, 1, 0, scale, workspace, workspace_bytes, stream);
    if (rc || !stats) return rc;
    return lk_hip_channel_stats_lc_f32(out, stats, lo, co, stream);
  }
  lkd::GemmParams p = lkh::baseParams();
  p.a = x;
  p.b = w;
  p.bias = bias;
  p.res = res;
  p.c = out;
  p.m = lo;
  p.n = co;
  p.k = kw * ci;
  p.lda = ci;
  p.ldb = kw * ci;
  p.ldc = co;
  p.ldr = co;
  p.scale = scale;
  p.convL = l;
  p.convCi = ci;
  p.convStride = stride;
  p.convPad = padding;
  p.convDil = dilation;
  p.affine = affine;
  p.alpha = alpha;
  p.pre = pre;
  p.slope = slope;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t reach = static_cast<int64_t>(dilation) * (kw - 1);  // halo rows beyond the output tile
  const int64_t tiles = static_cast<int64_t>(lkh::ceilDiv(lo, 128)) * lkh::ceilDiv(co, 128);
  const bool big = tiles >= 256 && 128 + reach <= lkd::TapCfg<128>::maxHalo;
  bool statsDone = false;
  if (stride == 1 && (big || 64 + reach <= lkd::TapCfg<64>::maxHalo)) {
    if (big) {
      p.stats = stats;  // the 128-row tiles are exactly the statistics chunks
      statsDone = stats != nullptr;
      dim3 grid(lkh::ceilDiv(co, 128), lkh::ceilDiv(lo, 128));
      hipLaunchKernelGGL((lkd::convTapKernel<128, 128>), grid, dim3(lkd::NT), 0, s, p, static_cast<int>(kw),
                         static_cast<int>(128 + reach));
    } else {  // few output tiles (decoder / F0-N at frame rate): 64 x 64 tiles fill more of the 256 CUs
      // and split the 16-channel chunks over workgroups when even those leave CUs idle (at least 2 chunks per
      // split, partial tiles in the workspace past its 64 KiB counter area, epilogue in gemmSplitReduceKernel)
      const int64_t base = static_cast<int64_t>(lkh::ceilDiv(co, 64)) * lkh::ceilDiv(lo, 64);
      const int64_t chunks = ci / lkd::BK;
      int split = 1;
      if (workspace && base < 256 && chunks >= 4) {
        split = static_cast<int>(std::min<int64_t>({8, 512 / base, chunks / 2}));
        while (split > 1 && 65536 + static_cast<int64_t>(split) * lo * co * 4 > workspace_bytes) --split;
        split = std::max(split, 1);
      }
      if (split > 1) {
        p.kSplit = (chunks + split - 1) / split;
        split = static_cast<int>((chunks + p.kSplit - 1) / p.kSplit);
        p.splitk = split;
        p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 65536);
      }
      dim3 grid(lkh::ceilDiv(co, 64), lkh::ceilDiv(lo, 64), static_cast<unsigned>(split));
      hipLaunchKernelGGL((lkd::convTapKernel<64, 64>), grid, dim3(lkd::NT), 0, s, p, static_cast<int>(kw),
                         static_cast<int>(64 + reach));
      if (split > 1)
        hipLaunchKernelGGL(lkd::gemmSplitReduceKernel,
                           dim3(static_cast<unsigned>(std::min<int64_t>((lo * co + 255) / 256, 8192))), dim3(256), 0,
                           s, p);
    }
  } else {
    lkh::launchGemm<lkd::A_CONV, lkd::B_NT>(p, s);
  }
  if (hipGetLastError() != hipSuccess) return 2;
  if (stats && !statsDone) return lk_hip_channel_stats_lc_f32(out, stats, lo, co, stream);
  return 0;
}

}  // extern "C"
