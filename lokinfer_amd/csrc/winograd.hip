// The reference's Winograd / Toom-Cook 1-D conv op family (wino_tf[_snake|_leaky]_lc_f32_gpu,
// wino_mm[_res][_stats]_lc_f32_gpu, wino_adain_affine_lc_f32_gpu: python/lokinfer/ops/winograd.py:120-218,
// kernels/gpu/winograd.cpp:73-160 in lariaus/lokinfer), with the reference's operand layouts so that a graph built
// on those ops runs unchanged:
//   V  [d, A, rmax, C]: V[rho, xi, r, c] = sum_j BT[xi, j] h[rho + d (r M + j - pad / d), c], h = act(x), zero
//                       outside the residue class's rows
//   U  [A, N Ci, Co]   = G w per tap group (host wino_weights), tr = [BT (A x A) | AT (M x A)]
//   out[o, co] = (b + sum_xi AT[j, xi] sum_{g, ci} V[rho, xi, t + g, ci] U[xi, g Ci + ci, co] [+ res]) * scale,
//                o = rho + d (t M + j)
//   stats [d chunks, Co, 2]: (mean, M2) of each 128 output rows of a residue class
// The same kernels run this backend's Kokoro graph wherever their grid fills the chip (the generator's resblock
// and noise convs, the decoder's wide convs, conv_post).
//
// wino_mm: one workgroup per (64 output channels, 64 tiles, residue); 4 waves in 2 x 2, each 32 tiles x 32
// channels. Steps = points x 16-channel chunks; per step the V rows of the workgroup's tiles (+ N - 1 for the
// group shift) are staged [row][4 slots] (swizzled by (row >> 2) & 3) and U's N x 16 rows k-major; the point's
// GEMM accumulates over the groups with the A rows shifted by g, and after a point's last chunk AT[j, xi] folds
// it into the M output accumulators. Small grids split the steps over workgroups (split-K) and sum the partial
// rows in winoSplitReduceKernel (statistics then from the channel-stats kernel).
#include "common.h"
#include "lokinfer_hip.h"

#include <algorithm>
#include <cstdint>

namespace lkh {
int residueStats(const float* x, float* st, int64_t l, int64_t c, int d, int64_t chunks, hipStream_t s);  // kokoro.hip
}  // namespace lkh

namespace lkd {

typedef float v16w __attribute__((ext_vector_type(16)));
typedef float v4w __attribute__((ext_vector_type(4)));

constexpr int kWinoRows = 128;  // output rows per statistics chunk

// V[rho, xi, r, c4 .. c4 + 3] for R = 4 consecutive tile rows r per thread, i.e. per (rho, r / R, c4), channel
// quad fastest: the R tiles share their overlapping input rows, so a thread loads and activates M R + A - M rows
// once (1.19x the input instead of A / M = 1.75x at M = 4, A = 7) and writes R A rows of V. act: 0 none,
// 1 snake(affine), 2 leaky(affine); rows outside the residue class are zero (the conv pads after the activation).
template <int M, int A>
__global__ __launch_bounds__(256) void winoTfKernel(const float* __restrict__ x, const float* __restrict__ tr,
                                                   const float* __restrict__ af, const float* __restrict__ alpha,
                                                   float* __restrict__ v, int64_t l, int64_t c, int d, int padq,
                                                   int64_t rmax, int act, float slope) {
  constexpr int R = 4;
  constexpr int XR = M * R + A - M;  // input rows behind R tiles
  const int64_t c4n = c / 4;
  const int64_t groups = (rmax + R - 1) / R;
  const int64_t total = static_cast<int64_t>(d) * groups * c4n;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c4 = i % c4n, rg = (i / c4n) % groups;
    const int rho = static_cast<int>(i / (c4n * groups));
    const int64_t lr = rho < l ? (l - rho + d - 1) / d : 0;
    const int64_t r0 = rg * R;
    const int64_t q0 = r0 * M - padq;
    v4w mean = {0.f, 0.f, 0.f, 0.f}, scale = {1.f, 1.f, 1.f, 1.f}, beta = {0.f, 0.f, 0.f, 0.f};
    v4w al = {1.f, 1.f, 1.f, 1.f}, inv = {1.f, 1.f, 1.f, 1.f};
    if (act != 0) {
      mean = *reinterpret_cast<const v4w*>(af + 4 * c4);
      scale = *reinterpret_cast<const v4w*>(af + c + 4 * c4);
      beta = *reinterpret_cast<const v4w*>(af + 2 * c + 4 * c4);
    }
    if (act == 1) {
      al = *reinterpret_cast<const v4w*>(alpha + 4 * c4);
#pragma unroll
      for (int e = 0; e < 4; ++e) inv[e] = 1.0f / al[e];
    }
    v4w raw[XR];
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int64_t q = q0 + j;
      const int64_t qc = min<int64_t>(max<int64_t>(q, 0), max<int64_t>(lr - 1, 0));
      raw[j] = *reinterpret_cast<const v4w*>(x + min<int64_t>(rho + qc * d, l - 1) * c + 4 * c4);
    }
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int64_t q = q0 + j;
      v4w h = raw[j];
      if (act == 1) {
        h = (h - mean) * scale + beta;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = h[e] + inv[e] * snakeSinSq(al[e] * h[e]);
      } else if (act == 2) {
        h = (h - mean) * scale + beta;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = h[e] >= 0.0f ? h[e] : h[e] * slope;
      }
      const bool in = q >= 0 && q < lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) raw[j][e] = in ? h[e] : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const int64_t rr = r0 + t;
      if (rr >= rmax) break;
#pragma unroll
      for (int xi = 0; xi < A; ++xi) {
        v4w o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < A; ++j) o += tr[xi * A + j] * raw[M * t + j];
        *reinterpret_cast<v4w*>(v + ((static_cast<int64_t>(rho) * A + xi) * rmax + rr) * c + 4 * c4) = o;
      }
    }
  }
}

struct WinoMmArgs {
  const float* v;
  const float* u;
  const float* bias;
  const float* res;
  float* out;
  const float* tr;
  float* stats;
  float* part;  // split > 1: per-split raw output rows [split][Lo][Co], summed by winoSplitReduceKernel
  int64_t lo, ci, co, rmax, chunks;
  int d, split;
  float scale;
};

// OCC workgroups per CU. M = 4 at OCC = 3 fits 168 VGPRs (the few spills the bound costs sit before the step loop
// and in the epilogue): on grids of more than two workgroups per CU a third wave per SIMD keeps the matrix pipe fed
// through the other waves' barriers and LDS stores (K = 11 roofline launch 0.574 -> 0.599 of peak); smaller grids
// leave the third slot empty and run the unconstrained OCC = 2 form (176 VGPRs), which is 0.5% faster there.
//
// S: 16-channel sub-chunks per step (one tap group only). A step of one tap group and 16 channels is 8 MFMAs per
// wave, too few to cover the step's fixed costs (barrier, staging, the first operand reads); S sub-chunks make it
// 8 S MFMAs. Sub-chunk s of the step's 16 S channels has its own A plane, laid out as a 16-channel step's.
//
// UT: U given tiled (ops u_layout = 1), Ut [A, Co / 64, (Ci / 16) N 4 64 4]: per point and 64-column block, for
// each 16-channel chunk and tap group the 16 x 64 slab stored k-quad-major, [k4][col][4] (U row g Ci + 16 c + 4 k4 + q,
// column 64 cb + col). A step's U is then one contiguous run, staged with coalesced 16-byte loads straight into
// the LDS order Bs[e * 4 + k4][col] (e = g S + s), and a wave fetches an operand set's B fragments for eight MFMAs
// with two 16-byte reads: 4 N S reads per step in all, few enough for the LDS counter to wait on each read
// separately (with U k-major, the 16 N S + 2 N S reads of a step exceed it). The same MFMAs in the same order, so
// the same bits.
template <int M, int A, int N, int OCC = 2, int S = 1, bool UT = false>
__global__ __launch_bounds__(256, OCC) void winoMmKernel(WinoMmArgs p) {
  static_assert(S == 1 || N == 1, "sub-chunks only for one tap group");
  constexpr int TT = 64;              // tiles per workgroup
  constexpr int ROWS = TT + N - 1;    // staged V rows (group shift)
  constexpr int LDB = 64 + 8;         // k-major U rows: the two lane halves read 4 rows = 32 banks apart
  constexpr int AQ = ROWS * 4;
  constexpr int AS1 = (AQ + 255) / 256;  // staging float4s per thread and sub-chunk
  constexpr int AS = S * AS1;
  __shared__ v4w As[2][AS * 256];  // rows past ROWS: every thread stores, so no store sits behind a branch
  __shared__ float Bs[2][UT ? N * S * 16 * 64 : N * S * 16 * LDB];
  __shared__ float red[2][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lk = lane >> 5;
  // XCD-aware order: the channel blocks of a tile block read its V rows through one L2
  const GridItem wk = xcdOrder();
  const int d = p.d, rho = wk.z % d, sp = wk.z / d;
  const int64_t lor = rho < p.lo ? (p.lo - rho + d - 1) / d : 0;  // output rows of this residue class
  const int64_t t0 = static_cast<int64_t>(wk.y) * TT;
  if (t0 * M >= lor) return;
  const int64_t c0 = static_cast<int64_t>(wk.x) * 64;
  const int chunks = static_cast<int>(p.ci / (16 * S));
  const int steps = A * chunks;
  // split-K: this workgroup runs steps [sb, se) of the point-major step sequence; a point cut by the range is
  // folded with AT at the range's end, and AT is linear, so the splits' outputs sum to the full one
  const int sb = static_cast<int>(static_cast<int64_t>(steps) * sp / p.split);
  const int se = static_cast<int>(static_cast<int64_t>(steps) * (sp + 1) / p.split);
  const int nsteps = se - sb;
  const int64_t nci = static_cast<int64_t>(N) * p.ci;

  // staging: A rows (S planes of ROWS x 4 slots) over 256 threads, U (N S 16 rows x 16 float4) over 256 threads
  constexpr int BQ = N * S * 16 * 16;
  constexpr int BSL = BQ / 256;
  // two register sets: step t's operands live in set t & 1, loaded two steps ahead of their LDS store
  v4w ra0[AS], rb0[BSL], ra1[AS], rb1[BSL];
  auto gload = [&](int s, v4w(&ra)[AS], v4w(&rb)[BSL]) {
    const int xi = s / chunks, ch = s - xi * chunks;
    const float* vx =
        p.v + (static_cast<int64_t>(rho) * A + xi) * p.rmax * p.ci + static_cast<int64_t>(ch) * 16 * S;
#pragma unroll
    for (int i = 0; i < AS; ++i) {
      const int idx = tid + 256 * (i % AS1);
      const int row = min(idx >> 2, ROWS - 1), slot = idx & 3;
      const int64_t t = min<int64_t>(t0 + row, p.rmax - 1);  // rows past rmax only feed tiles never stored
      ra[i] = *reinterpret_cast<const v4w*>(vx + t * p.ci + 16 * (i / AS1) + 4 * slot);
    }
    const float* ux = UT ? p.u + (static_cast<int64_t>(xi) * (p.co / 64) + c0 / 64) * nci * 64 +
                               static_cast<int64_t>(ch) * (N * S * 1024)
                         : p.u + static_cast<int64_t>(xi) * nci * p.co + c0;
#pragma unroll
    for (int i = 0; i < BSL; ++i) {
      const int idx = tid + 256 * i;
      if constexpr (UT) {  // the step's slab, in the LDS order
        rb[i] = *reinterpret_cast<const v4w*>(ux + 4 * idx);
      } else {
        const int c4 = idx & 15, gk = idx >> 4, g = gk / (16 * S), k = gk % (16 * S);
        rb[i] =
            *reinterpret_cast<const v4w*>(ux + (static_cast<int64_t>(g) * p.ci + ch * 16 * S + k) * p.co + 4 * c4);
      }
    }
  };
  auto sstore = [&](int buf, const v4w(&ra)[AS], const v4w(&rb)[BSL]) {
#pragma unroll
    for (int i = 0; i < AS; ++i) {
      const int idx = tid + 256 * (i % AS1);
      const int row = idx >> 2, slot = idx & 3;
      As[buf][(i / AS1) * AS1 * 256 + row * 4 + (slot ^ ((row >> 2) & 3))] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BSL; ++i) {
      const int idx = tid + 256 * i;
      if constexpr (UT) {
        *reinterpret_cast<v4w*>(&Bs[buf][4 * idx]) = rb[i];
      } else {
        const int c4 = idx & 15, gk = idx >> 4;
        *reinterpret_cast<v4w*>(&Bs[buf][gk * LDB + 4 * c4]) = rb[i];
      }
    }
  };

  v16w acc, y[M];
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < M; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[j][r] = 0.0f;

  const int arow = 32 * wm + lr, bcol = 32 * wn + lr;
  // one step: MFMAs on LDS buffer s & 1; loads step s + 2 into (lra, lrb) = set s & 1 (its step s is already in
  // LDS), stores step s + 1 from (sra, srb) = set (s + 1) & 1 into the other buffer
  auto step = [&](int sl, v4w(&lra)[AS], v4w(&lrb)[BSL], const v4w(&sra)[AS], const v4w(&srb)[BSL]) {
    const int buf = sl & 1, s = sb + sl;
    const int xi = s / chunks, ch = s - xi * chunks;
    // operand sets (tap group g, sub-chunk s) = e = g S + s
    v4w af[N * S][2];
    float bq[N * S][2][4];
#pragma unroll
    for (int e = 0; e < N * S; ++e) {
      const int row = arow + e / S;
      const int plane = (e % S) * AS1 * 256;
#pragma unroll
      for (int h = 0; h < 2; ++h) af[e][h] = As[buf][plane + row * 4 + ((2 * h + lk) ^ ((row >> 2) & 3))];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (UT) {
          const v4w b4 = *reinterpret_cast<const v4w*>(&Bs[buf][((e * 4 + 2 * h + lk) * 64 + bcol) * 4]);
#pragma unroll
          for (int q = 0; q < 4; ++q) bq[e][h][q] = b4[q];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) bq[e][h][q] = Bs[buf][(e * 16 + 8 * h + 4 * lk + q) * LDB + bcol];
        }
      }
    }
    // unconditional (the last two steps reload the final step), so the wait before each LDS store counts only
    // the loads of the set it stores and never the ones just issued
    gload(min(s + 2, se - 1), lra, lrb);
#pragma unroll
    for (int e = 0; e < N * S; ++e)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[e][h][q], bq[e][h][q], acc, 0, 0, 0);
    if (ch == chunks - 1 || s == se - 1) {  // the point (or this split's part of it) is complete: fold it
#pragma unroll
      for (int j = 0; j < M; ++j) {
        const float at = p.tr[A * A + j * A + xi];
        y[j] += at * acc;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    }
    sstore(buf ^ 1, sra, srb);  // after the last step, into a buffer nothing reads
    __syncthreads();
  };

  gload(sb, ra0, rb0);
  sstore(0, ra0, rb0);
  gload(min(sb + 1, se - 1), ra1, rb1);
  __syncthreads();
  // pairs of steps with no branch inside, so every loop edge carries the same outstanding loads; an odd last
  // step is peeled
  int sl = 0;
  for (; sl + 1 < nsteps; sl += 2) {
    step(sl, ra0, rb0, ra1, rb1);
    step(sl + 1, ra1, rb1, ra0, rb0);
  }
  if (sl < nsteps) step(sl, ra0, rb0, ra1, rb1);

  if (p.split > 1) {  // raw partial rows; bias, residual, scale and statistics come in the reduction
    float* pp = p.part + static_cast<int64_t>(sp) * p.lo * p.co;
#pragma unroll
    for (int j = 0; j < M; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t uo = (t0 + 32 * wm + 8 * (r >> 2) + 4 * lk + (r & 3)) * M + j;
        if (uo < lor) pp[(rho + uo * d) * p.co + c0 + 32 * wn + lr] = y[j][r];
      }
    return;
  }

  // epilogue: register r = tile t0 + 32 wm + 8 (r / 4) + 4 lk + r % 4, channel c0 + bcol
  const int64_t col = c0 + bcol;
  const float bias = p.bias[col];
#pragma unroll
  for (int j = 0; j < M; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t t = t0 + 32 * wm + 8 * (r >> 2) + 4 * lk + (r & 3);
      const int64_t uo = t * M + j;
      float o = y[j][r] + bias;
      if (p.res && uo < lor) o += p.res[(rho + uo * d) * p.co + col];
      o *= p.scale;
      y[j][r] = o;
      if (uo < lor) p.out[(rho + uo * d) * p.co + col] = o;
    }
  if (p.stats) {
    // chunks of 128 rows of this residue class: M = 4: 32 tiles = one wave row (chunk 2 by + wm), reduced in the
    // wave; M = 2: 64 tiles = the workgroup (chunk by), the two wave rows combined through LDS.
    constexpr int TPC = kWinoRows / M;  // tiles per chunk
    const int64_t chunk = (t0 + 32 * wm) / TPC;
    const int64_t cbase = chunk * kWinoRows;
    const float nrows = static_cast<float>(min<int64_t>(kWinoRows, lor - cbase));
    float s1 = 0.0f;
#pragma unroll
    for (int j = 0; j < M; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t uo = (t0 + 32 * wm + 8 * (r >> 2) + 4 * lk + (r & 3)) * M + j;
        if (uo < lor) s1 += y[j][r];
      }
    s1 += __shfl_xor(s1, 32, 64);
    if constexpr (TPC == 64) {
      if (lk == 0) red[wm][bcol] = s1;
      __syncthreads();
      s1 = red[0][bcol] + red[1][bcol];
      __syncthreads();
    }
    const float mean = s1 / nrows;
    float s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < M; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t uo = (t0 + 32 * wm + 8 * (r >> 2) + 4 * lk + (r & 3)) * M + j;
        const float dv = y[j][r] - mean;
        if (uo < lor) s2 += dv * dv;
      }
    s2 += __shfl_xor(s2, 32, 64);
    if constexpr (TPC == 64) {
      if (lk == 0) red[wm][bcol] = s2;
      __syncthreads();
      s2 = red[0][bcol] + red[1][bcol];
    }
    const bool writer = lk == 0 && (TPC == 32 || wm == 0) && nrows > 0.0f;
    if (writer) {
      float* st = p.stats + ((static_cast<int64_t>(rho) * p.chunks + chunk) * p.co + col) * 2;
      st[0] = mean;
      st[1] = s2;
    }
  }
}

// Split-K reduction: out = (sum_s part[s] + bias [+ res]) * scale, the s sum in split order; one
// float4 of one row per thread, grid-stride (Co % 64 == 0, so a float4 never straddles two rows).
__global__ __launch_bounds__(256) void winoSplitReduceKernel(const float* __restrict__ part, int split,
                                                            const float* __restrict__ bias,
                                                            const float* __restrict__ res, float* __restrict__ out,
                                                            int64_t lo, int64_t co, float scale) {
  const int64_t n4 = lo * co / 4, plane = lo * co;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t e = 4 * i, col = e % co;
    v4w sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < 8; ++sp)  // split <= 8
      if (sp < split) sum += *reinterpret_cast<const v4w*>(part + sp * plane + e);
    v4w o = sum + *reinterpret_cast<const v4w*>(bias + col);
    if (res) o += *reinterpret_cast<const v4w*>(res + e);
    *reinterpret_cast<v4w*>(out + e) = o * scale;
  }
}

// AdaIN affine from wino_mm statistics (chunks per residue class of the dilation), 4 channels x 64 chunk slices
// per workgroup.
__global__ __launch_bounds__(kAffineThreads) void winoAffineKernel(const float* __restrict__ st,
                                                                  const float* __restrict__ gb,
                                                                  float* __restrict__ af, int64_t l, int64_t c, int d,
                                                                  int64_t chunks, int64_t creal, float eps) {
  adainAffineSlices(st, gb, af, l, c, d, chunks, creal, eps);
}

}  // namespace lkd

extern "C" {

int lk_hip_wino_tf_lc_f32(const float* x, const float* tr, const float* affine, const float* alpha, float* v,
                          int64_t l, int64_t c, int dilation, int padding, int kernel, int tile, int64_t v_rows,
                          int act, float slope, void* stream) {
  if (c % 4 != 0 || dilation < 1 || padding % dilation != 0 || (tile != 2 && tile != 4)) return 1;
  const int a = tile == 2 ? 4 : kernel == 3 ? 6 : 7;
  if (v_rows % (static_cast<int64_t>(dilation) * a) != 0) return 1;
  const int64_t rmax = v_rows / (static_cast<int64_t>(dilation) * a);
  const int64_t total = static_cast<int64_t>(dilation) * ((rmax + 3) / 4) * (c / 4);  // 4 tile rows per thread
  if (total == 0) return 0;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int padq = padding / dilation;
  if (a == 4)
    hipLaunchKernelGGL((lkd::winoTfKernel<2, 4>), dim3(blocks), dim3(256), 0, s, x, tr, affine, alpha, v, l, c,
                       dilation, padq, rmax, act, slope);
  else if (a == 6)
    hipLaunchKernelGGL((lkd::winoTfKernel<4, 6>), dim3(blocks), dim3(256), 0, s, x, tr, affine, alpha, v, l, c,
                       dilation, padq, rmax, act, slope);
  else
    hipLaunchKernelGGL((lkd::winoTfKernel<4, 7>), dim3(blocks), dim3(256), 0, s, x, tr, affine, alpha, v, l, c,
                       dilation, padq, rmax, act, slope);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace {

template <bool UT>
int winoMm(const float* v, const float* u, const float* bias, const float* res, float* out, const float* tr,
           float* stats, int64_t v_rows, int64_t ci, int64_t co, int64_t lo, int dilation, int groups, int kernel,
           int tile, float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  const int a = tile == 2 ? 4 : kernel == 3 ? 6 : 7;
  if (ci % 16 != 0 || co % 64 != 0 || dilation < 1 || groups < 1 || groups > 3 || lo < 1) return 1;
  if (v_rows % (static_cast<int64_t>(dilation) * a) != 0) return 1;  // V holds whole (residue, point) row blocks
  if ((tile == 2 && groups != 1) || (a == 6 && groups != 1) || (a == 7 && groups < 2)) return 1;
  const int64_t rmax = v_rows / (static_cast<int64_t>(dilation) * a);
  const int m = tile;
  const int64_t tiles = ((lo + dilation - 1) / dilation + m - 1) / m;  // residue class 0 is the longest
  if (rmax < tiles + groups - 1) return 1;  // V must hold every tile and its group shifts
  // split-K when the grid is too small to fill the chip (two workgroups per CU): at least 32 steps per split (fewer
  // measured slower than no split on MI355X: the partial rows' round trip and the second launch outweigh the extra
  // workgroups; so did splits up to three workgroups per CU at 16 steps), partials in the workspace past its 64 KiB
  // counter area
  const int64_t base = (co / 64) * ((tiles + 63) / 64) * dilation;
  const int steps = a * static_cast<int>(ci / 16);  // in 16-channel units
  // one tap group: 48 or 32 channels per pipeline step where they divide Ci
  const int sub = groups == 1 && tile == 4 ? ((ci / 16) % 3 == 0 ? 3 : (ci / 16) % 2 == 0 ? 2 : 1) : 1;
  int split = 1;
  if (workspace && base < 512) {
    split = static_cast<int>(std::min<int64_t>({8, 512 / base, steps / 32}));
    while (split > 1 && 65536 + static_cast<int64_t>(split) * lo * co * 4 > workspace_bytes) --split;
    split = std::max(split, 1);
  }
  float* part = split > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + 65536) : nullptr;
  lkd::WinoMmArgs p{v, u, bias, res, out, tr, stats, part, lo, ci, co, rmax,
                    ((lo + dilation - 1) / dilation + lkd::kWinoRows - 1) / lkd::kWinoRows, dilation, split, scale};
  const dim3 grid(static_cast<unsigned>(co / 64), static_cast<unsigned>((tiles + 63) / 64),
                  static_cast<unsigned>(dilation * split));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool occ3 = static_cast<int64_t>(grid.x) * grid.y * grid.z > 2 * 256;  // more than two per CU
  if (a == 4)
    hipLaunchKernelGGL((lkd::winoMmKernel<2, 4, 1, 2, 1, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6 && occ3 && sub == 3)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 3, 3, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6 && occ3 && sub == 2)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 3, 2, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6 && occ3)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 3, 1, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6 && sub == 3)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 2, 3, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6 && sub == 2)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 2, 2, UT>), grid, dim3(256), 0, s, p);
  else if (a == 6)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 6, 1, 2, 1, UT>), grid, dim3(256), 0, s, p);
  else if (groups == 2 && occ3)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 7, 2, 3, 1, UT>), grid, dim3(256), 0, s, p);
  else if (groups == 2)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 7, 2, 2, 1, UT>), grid, dim3(256), 0, s, p);
  else if (occ3)
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 7, 3, 3, 1, UT>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((lkd::winoMmKernel<4, 7, 3, 2, 1, UT>), grid, dim3(256), 0, s, p);
  if (split > 1) {
    hipLaunchKernelGGL(lkd::winoSplitReduceKernel,
                       dim3(static_cast<unsigned>(std::min<int64_t>((lo * co / 4 + 255) / 256, 8192))), dim3(256), 0,
                       s, part, split, bias, res, out, lo, co, scale);
    // the statistics of the summed output, per residue class as the fused epilogue writes them
    if (stats && lkh::residueStats(out, stats, lo, co, dilation, p.chunks, s)) return 2;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace

extern "C" {

int lk_hip_wino_mm_lc_f32(const float* v, const float* u, const float* bias, const float* res, float* out,
                          const float* tr, float* stats, int64_t v_rows, int64_t ci, int64_t co, int64_t lo,
                          int dilation, int groups, int kernel, int tile, float scale, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  return winoMm<false>(v, u, bias, res, out, tr, stats, v_rows, ci, co, lo, dilation, groups, kernel, tile, scale,
                       workspace, workspace_bytes, stream);
}

int lk_hip_wino_mm_ut_lc_f32(const float* v, const float* ut, const float* bias, const float* res, float* out,
                             const float* tr, float* stats, int64_t v_rows, int64_t ci, int64_t co, int64_t lo,
                             int dilation, int groups, int kernel, int tile, float scale, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  return winoMm<true>(v, ut, bias, res, out, tr, stats, v_rows, ci, co, lo, dilation, groups, kernel, tile, scale,
                      workspace, workspace_bytes, stream);
}

int lk_hip_wino_adain_affine_lc_f32(const float* stats, const float* gb, float* af, int64_t s, int64_t c,
                                    int64_t creal, int dilation, int64_t length, float eps, void* stream) {
  if (dilation < 1 || s % dilation != 0 || length < 1 || creal > c) return 1;
  hipLaunchKernelGGL(lkd::winoAffineKernel, dim3(lkh::ceilDiv(c, lkd::kAffineCh)), dim3(lkd::kAffineThreads), 0,
                     static_cast<hipStream_t>(stream),
                     stats, gb, af, length, c, dilation, s / dilation, creal, eps);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// wino_tf[_snake|_leaky]_lc_f32_gpu. ptrs: x, tr, [affine], [alpha], v. ints: x(L, C), tr(T), [affine(3, C)],
// [alpha(C)], v(R, C), dilation, groups, kernel, padding, tile; floats (leaky): slope.
template <int ACT>
void runWinoTf(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t l = a.ints[0], c = a.ints[1];
  const int o = ACT == 1 ? 6 : ACT == 2 ? 5 : 3;  // v dims
  const int64_t vr = a.ints[o];
  const int d = static_cast<int>(a.ints[o + 2]), k = static_cast<int>(a.ints[o + 4]);
  const int pad = static_cast<int>(a.ints[o + 5]), tile = static_cast<int>(a.ints[o + 6]);
  LK_REQUIRE(ctx, a.ints[o + 1] == c, "wino_tf: v must be f32[R, C]");
  const int vp = ACT == 1 ? 4 : ACT == 2 ? 3 : 2;
  const float slope = ACT == 2 && a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 0.0f;
  if (lk_hip_wino_tf_lc_f32(P<float>(a, 0), P<float>(a, 1), ACT ? P<float>(a, 2) : nullptr,
                            ACT == 1 ? P<float>(a, 3) : nullptr, P<float>(a, vp), l, c, d, pad, k, tile, vr, ACT, slope,
                            ctx.stream))
    ctx.error = "wino_tf: invalid configuration";
}

// wino_mm[_res][_stats]_lc_f32_gpu. ptrs: v, u, b, tr, x, [res], out, [stats]. ints: v(R, Ci), u(A, N Ci, Co),
// b(Co), tr(T), x(L, Ci), [res(Lo, Co)], out(Lo, Co), [stats(d chunks, Co, 2)], dilation, groups, kernel,
// padding, tile, [u_layout]; floats: [oscale]. u_layout 1 (this backend's addition; absent = 0, the reference's
// layout): u is U tiled, Ut(A, Co / 64, N Ci 64) (winoMmKernel's UT layout).
template <bool RES, bool STATS>
void runWinoMm(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t vr = a.ints[0], ci = a.ints[1];
  const int o = RES ? 11 : 9;
  const int at = o + 2 + (STATS ? 3 : 0);
  const int64_t co = a.ints[o + 1], lo = a.ints[o];
  const int d = static_cast<int>(a.ints[at]), groups = static_cast<int>(a.ints[at + 1]);
  const int k = static_cast<int>(a.ints[at + 2]), tile = static_cast<int>(a.ints[at + 4]);
  const bool ut = a.numInts > static_cast<uint32_t>(at + 5) && a.ints[at + 5] == 1;
  LK_REQUIRE(ctx,
             ut ? (a.ints[3] * 64 == co && a.ints[4] == groups * ci * 64)
                : (a.ints[4] == co && a.ints[3] == groups * ci),
             "wino_mm: u must be f32[A, N Ci, Co] (u_layout 1: f32[A, Co / 64, N Ci 64])");
  const int64_t alpha = tile == 2 ? 4 : k == 3 ? 6 : 7;  // transform points of this kernel size and tile
  LK_REQUIRE(ctx, a.ints[2] == alpha, "wino_mm: u's leading dim must be the transform's point count");
  LK_REQUIRE(ctx, d >= 1 && vr % (static_cast<int64_t>(d) * alpha) == 0,
             "wino_mm: v rows must be a multiple of dilation * points");
  const int outp = RES ? 6 : 5;
  const float scale = RES && a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1.0f;
  const auto mm = ut ? lk_hip_wino_mm_ut_lc_f32 : lk_hip_wino_mm_lc_f32;
  if (mm(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), RES ? P<float>(a, 5) : nullptr, P<float>(a, outp),
         P<float>(a, 3), STATS ? P<float>(a, outp + 1) : nullptr, vr, ci, co, lo, d, groups, k, tile, scale,
         ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream))
    ctx.error = "wino_mm: invalid configuration";
}

// wino_adain_affine_lc_f32_gpu. ptrs: stats, gb, af. ints: stats(S, C, 2), gb(2 Creal), af(3, C), dilation,
// length; floats: eps.
void runWinoAffine(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], c = a.ints[1], g2 = a.ints[3];
  const int d = static_cast<int>(a.ints[6]);
  const int64_t length = a.ints[7];
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  LK_REQUIRE(ctx, a.ints[2] == 2 && g2 % 2 == 0 && g2 / 2 <= c, "wino_adain_affine: bad stats / gb");
  if (lk_hip_wino_adain_affine_lc_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), s, c, g2 / 2, d, length, eps,
                                      ctx.stream))
    ctx.error = "wino_adain_affine: invalid configuration";
}

}  // namespace

void registerWinogradKernels() {
  const Device G = Device::Gpu;
  registerKernel({"wino_tf_lc_f32_gpu", G, runWinoTf<0>, 2, 1});
  registerKernel({"wino_tf_snake_lc_f32_gpu", G, runWinoTf<1>, 4, 1});
  registerKernel({"wino_tf_leaky_lc_f32_gpu", G, runWinoTf<2>, 3, 1});
  registerKernel({"wino_mm_lc_f32_gpu", G, runWinoMm<false, false>, 5, 1});
  registerKernel({"wino_mm_res_lc_f32_gpu", G, runWinoMm<true, false>, 6, 1});
  registerKernel({"wino_mm_stats_lc_f32_gpu", G, runWinoMm<false, true>, 5, 2});
  registerKernel({"wino_mm_res_stats_lc_f32_gpu", G, runWinoMm<true, true>, 6, 2});
  registerKernel({"wino_adain_affine_lc_f32_gpu", G, runWinoAffine, 2, 1});
}

}  // namespace lkh
