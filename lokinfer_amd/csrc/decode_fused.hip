// Fused decode-step kernels (batch-1 transformer decode, e.g. GPT-2 124M): the GEMV split in two launches
// (partial sums, then a reduction) is kept, but each reduction is folded into the kernel that consumes it, so a
// layer is 5 launches instead of 13. At decode sizes every launch costs a few microseconds whatever it does, so
// the step time follows the launch count.
//
//   lk_hip_gemv_partial_f32    part[S, N] of x[1, K] . W[K, N], S = ceil(K / (4 rpw)) row slices; the input x is
//                              (mode 0) a vector, (mode 1) gelu(sum of a previous partial + bias), (mode 2)
//                              the merge of decode-attention chunk partials (one head per 64 rows), or (mode 3)
//                              LayerNorm(sum of a previous partial + bias + residual), the sum also written out
//   lk_hip_attention_decode_part_f32
//                              decode attention whose q, k, v come as GEMV partials (+ bias): writes row pos of
//                              both caches and the per-(head, 64-key chunk) partials (m, l, acc[64])
//   lk_hip_reduce_ln_f32       sum = sum_s part[s] + bias + res; ln = LayerNorm(sum) (one workgroup)
//
// They replace the reference's gemv4*_f32_gpu / attention_decode_split_f32_gpu / add_bias_layernorm2_f32_gpu
// sequence (transformer_gpu.cpp:122-251, kokoro_tok.metal:36-117, 637-924 in lariaus/lokinfer) for one layer,
// with the same arithmetic per element: the sums over K are split into row slices and added in a fixed order
// (deterministic), softmax is of q / 8 (taken in log2 units), LayerNorm is two-pass with the biased variance.
#include "common.h"
#include "decode_chunk.h"
#include "lokinfer_hip.h"

#include <algorithm>
#include <cstdint>

namespace lkd {

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kDecHd = 64;     // head dim
constexpr int kDecChunk = 64;  // keys per decode chunk
constexpr int kPartStride = kDecHd + 2;
constexpr int kFastSlices = 12;  // partial-row slices whose loads are issued together

// rows per wave of the partial GEMV: 16 for K <= 1024, else 64 (12 slices at K = 768 and at K = 3072)
inline int64_t gemvRowsPerWave(int64_t k) { return k <= 1024 ? 16 : 64; }

#ifndef LK_GEMV_MIN_WGS
#define LK_GEMV_MIN_WGS 256
#endif
// A LayerNorm prologue (modes 3, 4) makes every workgroup load all slices of the whole input row (48 KB at
// K = 768), more than its share of the weights: those GEMVs take wider column blocks, hence fewer workgroups.
// GPT-2 decode, ms per step by this floor: 256 -> 0.3145, 200 -> 0.306, 128 -> 0.298, 64 -> 0.3085.
#ifndef LK_GEMV_MIN_WGS_LN
#define LK_GEMV_MIN_WGS_LN 128
#endif
// Column block of the partial GEMV: the widest of 256 / 128 / 64 columns whose grid still has minWgs
// workgroups, else 64.
inline int gemvColBlock(int64_t n, int64_t slices, int minWgs) {
  for (int cb = 256; cb > 64; cb /= 2)
    if (lkh::ceilDiv(n, cb) * slices >= minWgs) return cb;
  return 64;
}

// Workgroup = 4 waves over CB columns and 4 * RPW rows; wave w owns rows r0 + w RPW .. + RPW - 1. A wave row of
// CB / 4 lanes (float4 each) spans the CB columns, so a wave holds RS = 256 / CB such rows: lane subgroup q sums
// rows q, q + RS, q + 2 RS, ... of the wave's RPW. The subgroups combine by permlane swaps ((q0 + q1) + (q2 + q3)),
// the four wave sums in LDS as (w0 + w1) + (w2 + w3), and the workgroup writes slice blockIdx.y. Narrow column
// blocks multiply the workgroups of a small-N GEMV (N = 768: 36 at CB = 256, 144 at CB = 64) without adding row
// slices for the consumer to sum. The workgroup's slice of x is first formed in LDS according to XMODE.
struct LnIn {  // mode 3: x = LayerNorm(sum of xpart slices + xbias + res), workgroup (0, 0) writes the sum
  const float* res;
  const float* gamma;
  const float* beta;
  float* sumOut;
  float eps;
  // mode 4 (embedding): the sum is res[id] + xbias[id2] (rows of two tables with `rows` / `rows2` rows)
  const int64_t* id;
  const int64_t* id2;
  int64_t rows, rows2;
  unsigned long long* err;
};

// LayerNorm prologue over one row of K <= 1024 columns, K % 4 == 0; thread t < K / 4 owns columns 4t .. 4t + 3.
// The sum is ((slices of xpart, in order) + xbias) + res; load() issues every load, finish() (after the caller has
// issued its own loads) forms the sum, writes it to sumOut if asked, and returns this thread's 4 LayerNorm outputs
// (two-pass, biased variance; the workgroup is 4 waves). Threads past K / 4 return zeros.
struct LnRow {
  f4v pv[kFastSlices];
  f4v xb, rs, ga, be;
  int64_t c0;
  bool live;
  __device__ __forceinline__ void load(const float* xpart, int64_t xslices, const float* xbias, const float* res,
                                       const float* gamma, const float* beta, int64_t k) {
    c0 = 4 * static_cast<int64_t>(threadIdx.x);
    live = c0 < k;
    const int64_t cc = live ? c0 : 0;  // idle threads load column 0, never used
    const f4v zero = {0.f, 0.f, 0.f, 0.f};
    xb = zero;
    if (xslices > 0) {
#pragma unroll
      for (int i = 0; i < kFastSlices; ++i)
        pv[i] = *reinterpret_cast<const f4v*>(xpart + min<int64_t>(i, xslices - 1) * k + cc);
    }
    rs = *reinterpret_cast<const f4v*>(res + cc);
    if (xbias) xb = *reinterpret_cast<const f4v*>(xbias + cc);
    ga = *reinterpret_cast<const f4v*>(gamma + cc);
    be = *reinterpret_cast<const f4v*>(beta + cc);
  }
  __device__ __forceinline__ f4v finish(const float* xpart, int64_t xslices, int64_t k, float eps, float* sumOut,
                                        float (*scr)[4]) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const f4v zero = {0.f, 0.f, 0.f, 0.f};
    f4v sp = zero;
    if (xslices > 0) {
#pragma unroll
      for (int i = 0; i < kFastSlices; ++i)
        if (i < xslices) sp += pv[i];
      for (int64_t sl = kFastSlices; sl < xslices; ++sl)
        sp += *reinterpret_cast<const f4v*>(xpart + sl * k + (live ? c0 : 0));
    }
    const f4v v = live ? (sp + xb) + rs : zero;
    if (live && sumOut) *reinterpret_cast<f4v*>(sumOut + c0) = v;
    const float s1 = waveSumDpp((v.x + v.y) + (v.z + v.w));
    if (lane == 0) scr[0][wv] = s1;
    __syncthreads();
    const float mean = ((scr[0][0] + scr[0][1]) + (scr[0][2] + scr[0][3])) / static_cast<float>(k);
    const f4v d = v - mean;
    float s2 = live ? (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w) : 0.0f;
    s2 = waveSumDpp(s2);
    if (lane == 0) scr[1][wv] = s2;
    __syncthreads();
    const float var = ((scr[1][0] + scr[1][1]) + (scr[1][2] + scr[1][3])) / static_cast<float>(k);
    const float rstd = 1.0f / sqrtf(var + eps);
    return live ? d * rstd * ga + be : zero;
  }
};

// Sum of v over the RS lane subgroups of a wave (subgroup = 64 / RS consecutive lanes), in every subgroup.
template <int RS>
__device__ __forceinline__ float subgroupSum(float v) {
  if constexpr (RS == 1) {
    return v;
  } else {
    float r = v;
    if constexpr (RS == 4) {
      const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
      r = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
  }
}

template <int XMODE, int RPW, int CB>
__global__ __launch_bounds__(256) void gemvPartXKernel(const float* __restrict__ x, const float* __restrict__ xpart,
                                                      const float* __restrict__ xbias, int64_t xslices, int chunks,
                                                      LnIn ln, const float* __restrict__ w, float* __restrict__ part,
                                                      int64_t n, int64_t k) {
  constexpr int ROWS = 4 * RPW;
  __shared__ float xs[ROWS];
  constexpr int RS = 256 / CB, CL = CB / 4, LPW = RPW / RS;  // row subgroups, lanes per row, loads per lane
  static_assert(RPW % RS == 0, "rows per wave must split over the lane subgroups");
  __shared__ f4v wsum[4][CL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t rBase = static_cast<int64_t>(blockIdx.y) * ROWS;
  constexpr int B0 = LPW < 32 ? LPW : 32;
  const int cl = lane % CL, q = lane / CL;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * CB + 4 * cl;
  const int64_t r0 = rBase + static_cast<int64_t>(wv) * RPW + q;  // this lane's rows r0 + RS i
  const int64_t colc = min<int64_t>(col, n - 4);  // columns past N compute on a valid column, never stored
  f4v wr[B0];
  // Every load of the prologue is independent of the others and of the weights: all of them are issued at entry,
  // the prologue's own operands first (they are waited for first), then the first batch of weights, so the whole
  // prologue costs one memory round trip that overlaps the weight stream.
  auto loadWeights = [&]() {
#pragma unroll
    for (int i = 0; i < B0; ++i)
      wr[i] = __builtin_nontemporal_load(
          reinterpret_cast<const f4v*>(w + min<int64_t>(r0 + RS * i, k - 1) * n + colc));
  };
  if constexpr (XMODE == 0) {
    const float xv = tid < ROWS && rBase + tid < k ? x[rBase + tid] : 0.0f;
    loadWeights();
    if (tid < ROWS) xs[tid] = xv;
  } else if constexpr (XMODE == 1) {
    // x[r] = gelu(sum_s xpart[s, r] + xbias[r]), slices in order; ROWS <= 256: thread t owns row rBase + t
    static_assert(ROWS <= 256, "one row per thread");
    const int64_t r = rBase + tid;
    const bool live = tid < ROWS && r < k;
    const int64_t rc = min<int64_t>(r, k - 1);  // rows past K load a valid row, never used
    float pv[kFastSlices];
#pragma unroll
    for (int i = 0; i < kFastSlices; ++i) pv[i] = xpart[min<int64_t>(i, xslices - 1) * k + rc];
    const float bv = xbias[rc];
    loadWeights();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kFastSlices; ++i)
      if (i < xslices) s += pv[i];
    for (int64_t sl = kFastSlices; sl < xslices; ++sl) s += xpart[sl * k + rc];
    if (tid < ROWS) xs[tid] = live ? geluTanh(s + bv) : 0.0f;
  } else if constexpr (XMODE == 3 || XMODE == 4) {
    // the whole row: sum = slices in order + xbias + res (mode 4: two table rows), then its LayerNorm, of which
    // the workgroup keeps its own ROWS rows; workgroup (0, 0) writes the sum
    __shared__ float scr[2][4];
    const float* res = ln.res;
    const float* xb = xbias;
    bool bad = false;
    if constexpr (XMODE == 4) {
      const int64_t id = *ln.id, id2 = *ln.id2;
      const bool ok = id >= 0 && id < ln.rows, ok2 = id2 >= 0 && id2 < ln.rows2;
      bad = !ok || !ok2;
      if (bad && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0)
        raiseDeviceError(ln.err, LK_DEVERR_INDEX, ok ? id2 : id);
      res = ln.res + (ok ? id : 0) * k;
      xb = xbias + (ok2 ? id2 : 0) * k;
    }
    LnRow row;
    row.load(xpart, xslices, xb, res, ln.gamma, ln.beta, k);
    loadWeights();
    if constexpr (XMODE == 4) {
      if (bad) row.rs = f4v{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
    }
    const f4v y = row.finish(xpart, xslices, k, ln.eps, blockIdx.x == 0 && blockIdx.y == 0 ? ln.sumOut : nullptr,
                             scr);
    // this thread's columns that fall in the workgroup's rows rBase .. rBase + ROWS - 1
    if (row.live && row.c0 >= rBase && row.c0 < rBase + ROWS) *reinterpret_cast<f4v*>(&xs[row.c0 - rBase]) = y;
    if (rBase + ROWS > k && tid < ROWS && rBase + tid >= k) xs[tid] = 0.0f;
  } else {
    // rows rBase .. rBase + 63 are head blockIdx.y: merge its chunk partials (m, l, acc) in chunk order,
    // M = max m_c, out[d] = sum_c 2^{m_c - M} acc_c[d] / sum_c 2^{m_c - M} l_c (log2 units)
    static_assert(XMODE != 2 || ROWS == kDecHd, "attention merge needs 64 rows per workgroup");
    __shared__ float mrg[4][kDecHd];
    __shared__ float cw[64];
    const float* base = xpart + static_cast<int64_t>(blockIdx.y) * chunks * kPartStride;
    // thread (d = lane, chunk group wv) owns chunks wv, wv + 4, ... (chunks <= 64); wave 0 lane c also holds
    // chunk c's (m, l)
    float av[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = wv + 4 * i;
      av[i] = c < chunks ? base[c * kPartStride + 2 + lane] : 0.0f;
    }
    float mc = -INFINITY, lc = 0.0f;
    if (wv == 0 && lane < chunks) {
      mc = base[lane * kPartStride];
      lc = base[lane * kPartStride + 1];
    }
    loadWeights();
    if (wv == 0) {
      const float M = waveMaxDpp(mc);
      const float wc = lc > 0.0f ? __builtin_amdgcn_exp2f(mc - M) : 0.0f;
      cw[lane] = wc;
      const float L = waveSumDpp(lc * wc);
      if (lane == 0) xs[0] = L;  // xs doubles as a scratch slot until the merge below
    }
    __syncthreads();
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (wv + 4 * i < chunks) a += cw[wv + 4 * i] * av[i];
    mrg[wv][lane] = a;
    const float L = xs[0];
    __syncthreads();
    if (wv == 0) xs[lane] = ((mrg[0][lane] + mrg[1][lane]) + (mrg[2][lane] + mrg[3][lane])) / L;
    // NaN when the chunk kernel flagged an invalid position
  }
  __syncthreads();
  f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < B0; ++i) acc += xs[wv * RPW + q + RS * i] * wr[i];  // xs is 0 past K
#pragma unroll
  for (int b = B0; b < LPW; b += 32) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      wr[i] = __builtin_nontemporal_load(
          reinterpret_cast<const f4v*>(w + min<int64_t>(r0 + RS * (b + i), k - 1) * n + colc));
#pragma unroll
    for (int i = 0; i < 32; ++i) acc += xs[wv * RPW + q + RS * (b + i)] * wr[i];
  }
  acc.x = subgroupSum<RS>(acc.x);
  acc.y = subgroupSum<RS>(acc.y);
  acc.z = subgroupSum<RS>(acc.z);
  acc.w = subgroupSum<RS>(acc.w);
  if (q == 0) wsum[wv][cl] = acc;
  __syncthreads();
  if (wv == 0 && q == 0 && col < n)
    *reinterpret_cast<f4v*>(part + static_cast<int64_t>(blockIdx.y) * n + col) =
        (wsum[0][cl] + wsum[1][cl]) + (wsum[2][cl] + wsum[3][cl]);
}

// One wave per (head, 64-key chunk) (DecodeChunk), as the split decode kernel, but q / k / v of this step are
// the fixed-order sums of `slices` GEMV partial rows (+ bias). Every load is issued before the first wait: the
// partial rows first, then (once pos is known) the chunk's key and value rows. An invalid position writes NaN
// partials (no cache write) and is recorded in the GPU's error record.
__global__ __launch_bounds__(64) void decodeChunkPartKernel(const float* __restrict__ qpart, int64_t slices,
                                                           float* kc, float* vc, const int64_t* pos,
                                                           const float* __restrict__ bias, float* __restrict__ cpart,
                                                           int64_t cap, int heads, int chunks,
                                                           unsigned long long* err) {
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int g = lane >> 4, d4 = lane & 15;
  const int64_t D = static_cast<int64_t>(heads) * kDecHd, ld = 3 * D;
  float* part = cpart + (static_cast<int64_t>(h) * chunks + s) * kPartStride;
  const int64_t c4 = h * kDecHd + 4 * d4;  // this lane's 4 dims in a row of q, k or v
  // q / k / v partial rows: row g of the wave loads slices g, g + 4, g + 8 (issued at once; more in a tail
  // loop), the 4 row sums then combine as (r0 + r1) + (r2 + r3)
  constexpr int kRowSlices = kFastSlices / 4;
  f4v pq[kRowSlices], pk[kRowSlices], pv[kRowSlices];
#pragma unroll
  for (int i = 0; i < kRowSlices; ++i) {
    const float* row = qpart + min<int64_t>(g + 4 * i, slices - 1) * ld + c4;
    pq[i] = *reinterpret_cast<const f4v*>(row);
    pk[i] = *reinterpret_cast<const f4v*>(row + D);
    pv[i] = *reinterpret_cast<const f4v*>(row + 2 * D);
  }
  const f4v bq = *reinterpret_cast<const f4v*>(bias + c4), bk = *reinterpret_cast<const f4v*>(bias + D + c4),
            bv = *reinterpret_cast<const f4v*>(bias + 2 * D + c4);
  const int64_t ps = *pos;
  DecodeChunk ch;
  ch.load(kc, vc, ps, cap, s, D, c4);
  if (ch.badPos && h == 0 && s == 0 && lane == 0) raiseDeviceError(err, LK_DEVERR_POSITION, ps);
  f4v sq = {0.f, 0.f, 0.f, 0.f}, sk = sq, sv = sq;
#pragma unroll
  for (int i = 0; i < kRowSlices; ++i)
    if (g + 4 * i < slices) {
      sq += pq[i];
      sk += pk[i];
      sv += pv[i];
    }
  for (int64_t sl = kFastSlices + g; sl < slices; sl += 4) {
    const float* row = qpart + sl * ld + c4;
    sq += *reinterpret_cast<const f4v*>(row);
    sk += *reinterpret_cast<const f4v*>(row + D);
    sv += *reinterpret_cast<const f4v*>(row + 2 * D);
  }
  sq = f4v{crossRowSum(sq.x), crossRowSum(sq.y), crossRowSum(sq.z), crossRowSum(sq.w)};
  sk = f4v{crossRowSum(sk.x), crossRowSum(sk.y), crossRowSum(sk.z), crossRowSum(sk.w)};
  sv = f4v{crossRowSum(sv.x), crossRowSum(sv.y), crossRowSum(sv.z), crossRowSum(sv.w)};
  const f4v knew = sk + bk, vnew = sv + bv;
  if (ch.writesRow()) {
    *reinterpret_cast<f4v*>(kc + ps * D + c4) = knew;
    *reinterpret_cast<f4v*>(vc + ps * D + c4) = vnew;
  }
  ch.finish((sq + bq) * (0.125f * kLog2e), knew, vnew, part);
}

// Tied LM head of a decode step with the final LayerNorm and the greedy argmax folded in: x = LayerNorm(slices of
// part in order + bias + res) (every workgroup forms it in LDS from the partial rows), logits[r] = x . table[r, :]
// for r < rows, and per workgroup the (max logit, first row) pair over its rows, which argmaxKernel reduces.
// Wave w of workgroup b takes rows b * 4 + w + W i (W = 4 * grid waves) in two alternating halves of 4 rows (one
// reduced while the other loads); lane l holds columns 4 (l + 64 j), j < QPL (K <= 256 QPL).
constexpr int kLmRowBatch = 8;
constexpr int kLmGrid = 512;
template <int QPL>
__global__ __launch_bounds__(256) void lmHeadLnKernel(const float* __restrict__ part, int64_t slices,
                                                     const float* __restrict__ bias, const float* __restrict__ res,
                                                     const float* __restrict__ gamma, const float* __restrict__ beta,
                                                     float eps, const float* __restrict__ table,
                                                     float* __restrict__ logits, float* __restrict__ bestV,
                                                     int64_t* __restrict__ bestI, int64_t rows, int64_t k) {
  __shared__ f4v xrow[256];
  __shared__ float scr[2][4];
  __shared__ float wbV[4];
  __shared__ int64_t wbI[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t kq = k / 4;
  const int64_t W = static_cast<int64_t>(gridDim.x) * 4;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + wv;
  LnRow row;
  row.load(part, slices, bias, res, gamma, beta, k);
  // two halves of kLmRowBatch / 2 rows in ping-pong: while one half is reduced the other is in flight
  constexpr int H = kLmRowBatch / 2;
  f4v wa[H][QPL], wb[H][QPL];
  auto loadHalf = [&](f4v (&wr)[H][QPL], int64_t r0) {
#pragma unroll
    for (int b = 0; b < H; ++b) {
      const float* tr = table + min<int64_t>(r0 + W * b, rows - 1) * k;
#pragma unroll
      for (int j = 0; j < QPL; ++j)
        wr[b][j] = __builtin_nontemporal_load(
            reinterpret_cast<const f4v*>(tr + 4 * min<int64_t>(lane + 64 * j, kq - 1)));
    }
  };
  loadHalf(wa, wave);
  loadHalf(wb, wave + W * H);
  const f4v y = row.finish(part, slices, k, eps, nullptr, scr);
  if (row.live) xrow[tid] = y;
  __syncthreads();
  f4v xv[QPL];
#pragma unroll
  for (int j = 0; j < QPL; ++j) xv[j] = lane + 64 * j < kq ? xrow[lane + 64 * j] : f4v{0.f, 0.f, 0.f, 0.f};
  float best = -INFINITY;
  int64_t bi = INT64_MAX;
  // rows r0 + W b of one half: dot products, then (once the next loads of this half are issued) the row sums
  auto consume = [&](f4v (&wr)[H][QPL], int64_t r0) {
    float d[H];
#pragma unroll
    for (int b = 0; b < H; ++b) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < QPL; ++j) {
        const f4v t = xv[j] * wr[b][j];
        acc += (t.x + t.y) + (t.z + t.w);
      }
      d[b] = acc;
    }
    if (r0 + W * kLmRowBatch < rows) loadHalf(wr, r0 + W * kLmRowBatch);
#pragma unroll
    for (int b = 0; b < H; ++b) {
      const int64_t r = r0 + W * b;
      const float v = waveSumDpp(d[b]);
      if (r < rows) {
        if (lane == 0) logits[r] = v;
        if (v > best || (!(v < best) && r < bi)) {
          best = v;
          bi = r;
        }
      }
    }
  };
  for (int64_t r0 = wave; r0 < rows; r0 += W * kLmRowBatch) {
    consume(wa, r0);
    if (r0 + W * H < rows) consume(wb, r0 + W * H);
  }
  if (lane == 0) {
    wbV[wv] = best;
    wbI[wv] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      if (wbV[w] > best || (!(wbV[w] < best) && wbI[w] < bi)) {
        best = wbV[w];
        bi = wbI[w];
      }
    bestV[blockIdx.x] = best;
    bestI[blockIdx.x] = bi;
  }
}

constexpr int kRedMaxPerThread = 4;  // N <= 1024

__device__ __forceinline__ float blockSum1024(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  v = waveSum(v);
  __syncthreads();
  if (lane == 0) scratch[wv] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += scratch[i];
  return t;
}

// One 1024-thread workgroup: thread (c, q) sums slices q, q + 4, ... of columns c + 256 j; the quarter sums
// combine as (q0 + q1) + (q2 + q3); then sum = . + bias + res is written and LayerNorm'ed (two-pass, biased).
__global__ __launch_bounds__(1024) void reduceLnKernel(const float* __restrict__ part, int64_t slices,
                                                      const float* __restrict__ bias, const float* __restrict__ res,
                                                      const float* __restrict__ gamma, const float* __restrict__ beta,
                                                      float* __restrict__ sumOut, float* __restrict__ lnOut, int64_t n,
                                                      float eps) {
  __shared__ float red[4][256 * kRedMaxPerThread];
  __shared__ float scratch[16];
  const int tid = threadIdx.x, c = tid & 255, q = tid >> 8;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const int64_t col = c + 256 * j;
    float s = 0.0f;
    if (col < n) {
#pragma unroll 4
      for (int64_t sl = q; sl < slices; sl += 4) s += part[sl * n + col];
    }
    red[q][c + 256 * j] = s;
  }
  __syncthreads();
  // threads q == 0 own the columns; the others contribute zeros to the block sums
  float v[kRedMaxPerThread];
  float s1 = 0.0f;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const int64_t col = c + 256 * j;
    float x = 0.0f;
    if (q == 0 && col < n) {
      const int o = c + 256 * j;
      x = ((red[0][o] + red[1][o]) + (red[2][o] + red[3][o])) + bias[col] + res[col];
      sumOut[col] = x;
    }
    v[j] = x;
    s1 += x;
  }
  const float mean = blockSum1024(s1, scratch) / static_cast<float>(n);
  float s2 = 0.0f;
#pragma unroll
  for (int j = 0; j < kRedMaxPerThread; ++j) {
    const float d = v[j] - mean;
    if (q == 0 && c + 256 * j < n) s2 += d * d;
  }
  const float var = blockSum1024(s2, scratch) / static_cast<float>(n);
  const float rstd = 1.0f / sqrtf(var + eps);
  if (q == 0) {
#pragma unroll
    for (int j = 0; j < kRedMaxPerThread; ++j) {
      const int64_t col = c + 256 * j;
      if (col < n) lnOut[col] = (v[j] - mean) * rstd * gamma[col] + beta[col];
    }
  }
}

}  // namespace lkd

extern "C" {

int64_t lk_hip_gemv_partial_slices(int64_t k) {
  const int64_t rpw = lkd::gemvRowsPerWave(k);
  return (k + 4 * rpw - 1) / (4 * rpw);
}

}  // extern "C"

namespace {

int launchGemvPartial(int xmode, const float* x, const float* xpart, const float* xbias, int64_t xslices, int chunks,
                      const lkd::LnIn& ln, const float* w, float* part, int64_t n, int64_t k, void* stream) {
  if (n <= 0 || k <= 0 || n % 4 != 0) return 1;
  if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(part)) & 15) != 0) return 1;
  const int64_t rpw = lkd::gemvRowsPerWave(k);
  const int64_t slices = (k + 4 * rpw - 1) / (4 * rpw);
  const int cb = lkd::gemvColBlock(n, slices, xmode >= 3 ? LK_GEMV_MIN_WGS_LN : LK_GEMV_MIN_WGS);
  const dim3 grid(lkh::ceilDiv(n, cb), static_cast<unsigned>(slices));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define LK_GP_CB(MODE, R, CB) \
  hipLaunchKernelGGL((lkd::gemvPartXKernel<MODE, R, CB>), grid, dim3(256), 0, s, x, xpart, xbias, xslices, chunks, ln, \
                     w, part, n, k)
#define LK_GP(MODE, R)                    \
  do {                                    \
    if (cb == 256) LK_GP_CB(MODE, R, 256); \
    else if (cb == 128) LK_GP_CB(MODE, R, 128); \
    else LK_GP_CB(MODE, R, 64);           \
  } while (0)
  if (xmode == 0) {
    if (rpw == 16) LK_GP(0, 16);
    else LK_GP(0, 64);
  } else if (xmode == 1) {
    if (rpw == 16) LK_GP(1, 16);
    else LK_GP(1, 64);
  } else if (xmode == 2) {
    if (rpw != 16 || k % lkd::kDecHd != 0 || chunks <= 0 || chunks > 64) return 1;
    LK_GP(2, 16);
  } else if (xmode == 3 || xmode == 4) {
    if (k > 1024 || k % 4 != 0 || !ln.res || !ln.gamma || !ln.beta || !ln.sumOut || (xslices > 0 && !xpart)) return 1;
    if (xmode == 4 && (xslices != 0 || !xbias || !ln.id || !ln.id2 || ln.rows <= 0 || ln.rows2 <= 0)) return 1;
    // the LayerNorm prologue reads and writes whole float4 columns
    if (((reinterpret_cast<uintptr_t>(xpart) | reinterpret_cast<uintptr_t>(xbias) |
          reinterpret_cast<uintptr_t>(ln.res) | reinterpret_cast<uintptr_t>(ln.gamma) |
          reinterpret_cast<uintptr_t>(ln.beta) | reinterpret_cast<uintptr_t>(ln.sumOut)) & 15) != 0)
      return 1;
    if (xmode == 3) LK_GP(3, 16);
    else LK_GP(4, 16);
  } else {
    return 1;
  }
#undef LK_GP
#undef LK_GP_CB
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace

extern "C" {

int lk_hip_gemv_partial_f32(int xmode, const float* x, const float* xpart, const float* xbias, int64_t xslices,
                            int chunks, const float* res, const float* gamma, const float* beta, float* sum_out,
                            float eps, const float* w, float* part, int64_t n, int64_t k, void* stream) {
  if (xmode < 0 || xmode > 3) return 1;
  const lkd::LnIn ln{res, gamma, beta, sum_out, eps, nullptr, nullptr, 0, 0, nullptr};
  return launchGemvPartial(xmode, x, xpart, xbias, xslices, chunks, ln, w, part, n, k, stream);
}

int lk_hip_gemv_partial_embed_ln_f32(const float* table, const int64_t* id, const float* table2, const int64_t* id2,
                                     int64_t rows, int64_t rows2, const float* gamma, const float* beta, float eps,
                                     const float* w, float* part, float* sum_out, int64_t n, int64_t k,
                                     void* stream) {
  const lkd::LnIn ln{table, gamma, beta, sum_out, eps, id, id2, rows, rows2, lkh::deviceErrorRecord()};
  return launchGemvPartial(4, nullptr, nullptr, table2, 0, 0, ln, w, part, n, k, stream);
}

int lk_hip_attention_decode_part_f32(const float* qkv_part, int64_t slices, float* kc, float* vc, const int64_t* pos,
                                     const float* bias, float* chunk_part, int64_t cap, int heads, void* stream) {
  if (heads <= 0 || cap <= 0 || slices <= 0) return 1;
  const int chunks = static_cast<int>((cap + lkd::kDecChunk - 1) / lkd::kDecChunk);
  hipLaunchKernelGGL(lkd::decodeChunkPartKernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(chunks)),
                     dim3(64), 0, static_cast<hipStream_t>(stream), qkv_part, slices, kc, vc, pos, bias, chunk_part,
                     cap, heads, chunks, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_lm_head_ln_argmax_f32(const float* part, int64_t slices, const float* bias, const float* res,
                                 const float* gamma, const float* beta, float eps, const float* table, float* logits,
                                 int64_t* argmax, int64_t rows, int64_t k, void* workspace, int64_t workspaceBytes,
                                 void* stream) {
  if (rows <= 0 || k <= 0 || k > 1024 || k % 4 != 0 || slices < 0 || (slices > 0 && !part)) return 1;
  if (((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(res) |
        reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta) | reinterpret_cast<uintptr_t>(table)) &
       15) != 0)
    return 1;
  const int64_t grid = std::min<int64_t>(lkd::kLmGrid, (rows + 3) / 4);
  if (!workspace || workspaceBytes < grid * 16) return 3;
  auto* bestI = static_cast<int64_t*>(workspace);
  auto* bestV = reinterpret_cast<float*>(bestI + grid);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int qpl = static_cast<int>((k / 4 + 63) / 64);
#define LK_LM(Q)                                                                                                   \
  hipLaunchKernelGGL(lkd::lmHeadLnKernel<Q>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, part, slices, bias, \
                     res, gamma, beta, eps, table, logits, bestV, bestI, rows, k)
  switch (qpl) {
    case 1: LK_LM(1); break;
    case 2: LK_LM(2); break;
    case 3: LK_LM(3); break;
    default: LK_LM(4); break;
  }
#undef LK_LM
  if (hipGetLastError() != hipSuccess) return 2;
  return lk_hip_argmax_pairs_f32(bestV, bestI, argmax, grid, stream);
}

int lk_hip_reduce_ln_f32(const float* part, int64_t slices, const float* bias, const float* res, const float* gamma,
                         const float* beta, float* sum_out, float* ln_out, int64_t n, float eps, void* stream) {
  if (n <= 0 || n > 256 * lkd::kRedMaxPerThread || slices <= 0) return 1;
  hipLaunchKernelGGL(lkd::reduceLnKernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), part, slices,
                     bias, res, gamma, beta, sum_out, ln_out, n, eps);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// gemv_partial_f32_gpu(x[1, K], w[K, N]) -> part[S, N]
void runGemvPartial(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t k = a.ints[1], n = a.ints[3];
  LK_REQUIRE(ctx, a.ints[0] == 1 && a.ints[2] == k && a.ints[4] == lk_hip_gemv_partial_slices(k) && a.ints[5] == n,
             "gemv_partial: expected x [1, K], w [K, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(0, P<float>(a, 0), nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, nullptr, 0.0f,
                              P<float>(a, 1), P<float>(a, 2), n, k, ctx.stream))
    ctx.error = "gemv_partial: N % 4 != 0 or unaligned operands";
}

// gemv_partial_gelu_f32_gpu(xpart[Sx, K], xbias[K], w[K, N]) -> part[S, N], x = gelu(sum xpart + xbias)
void runGemvPartialGelu(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t sx = a.ints[0], k = a.ints[1], n = a.ints[4];
  LK_REQUIRE(ctx, a.ints[2] == k && a.ints[3] == k && a.ints[5] == lk_hip_gemv_partial_slices(k) && a.ints[6] == n,
             "gemv_partial_gelu: expected xpart [Sx, K], xbias [K], w [K, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(1, nullptr, P<float>(a, 0), P<float>(a, 1), sx, 0, nullptr, nullptr, nullptr, nullptr,
                              0.0f, P<float>(a, 2), P<float>(a, 3), n, k, ctx.stream))
    ctx.error = "gemv_partial_gelu: N % 4 != 0 or unaligned operands";
}

// gemv_partial_attn_f32_gpu(chunks[H, C, 66], w[64 H, N]) -> part[S, N], x = merged decode attention
void runGemvPartialAttn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t h = a.ints[0], c = a.ints[1], k = a.ints[3], n = a.ints[4];
  LK_REQUIRE(ctx, a.ints[2] == lkd::kPartStride && k == 64 * h && a.ints[5] == lk_hip_gemv_partial_slices(k) &&
                      a.ints[6] == n,
             "gemv_partial_attn: expected chunks [H, C, 66], w [64 H, N] -> [slices(K), N]");
  if (lk_hip_gemv_partial_f32(2, nullptr, P<float>(a, 0), nullptr, 0, static_cast<int>(c), nullptr, nullptr, nullptr,
                              nullptr, 0.0f, P<float>(a, 1), P<float>(a, 2), n, k, ctx.stream))
    ctx.error = "gemv_partial_attn: invalid configuration";
}

// gemv_partial_res_ln_f32_gpu(xpart[Sx, K], xbias[K], res[1, K], gamma[K], beta[K], w[K, N]; eps)
//   -> (part[S, N], sum[1, K]); x = LN(sum), sum = slices of xpart + xbias + res
void runGemvPartialResLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t sx = a.ints[0], k = a.ints[1], n = a.ints[8];
  LK_REQUIRE(ctx, a.ints[2] == k && a.ints[3] == 1 && a.ints[4] == k && a.ints[5] == k && a.ints[6] == k &&
                      a.ints[7] == k && a.ints[9] == lk_hip_gemv_partial_slices(k) && a.ints[10] == n &&
                      a.ints[11] == 1 && a.ints[12] == k,
             "gemv_partial_res_ln: expected xpart [Sx, K], xbias [K], res [1, K], gamma [K], beta [K], w [K, N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_gemv_partial_f32(3, nullptr, P<float>(a, 0), P<float>(a, 1), sx, 0, P<float>(a, 2), P<float>(a, 3),
                              P<float>(a, 4), P<float>(a, 7), eps, P<float>(a, 5), P<float>(a, 6), n, k, ctx.stream))
    ctx.error = "gemv_partial_res_ln: K > 1024, K or N not a multiple of 4, or unaligned operands";
}

// gemv_partial_ln_f32_gpu(x[1, K], gamma[K], beta[K], w[K, N]; eps) -> (part[S, N], copy of x [1, K]); x' = LN(x)
void runGemvPartialLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t k = a.ints[1], n = a.ints[5];
  LK_REQUIRE(ctx, a.ints[0] == 1 && a.ints[2] == k && a.ints[3] == k && a.ints[4] == k &&
                      a.ints[6] == lk_hip_gemv_partial_slices(k) && a.ints[7] == n && a.ints[8] == 1 &&
                      a.ints[9] == k,
             "gemv_partial_ln: expected x [1, K], gamma [K], beta [K], w [K, N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_gemv_partial_f32(3, nullptr, nullptr, nullptr, 0, 0, P<float>(a, 0), P<float>(a, 1), P<float>(a, 2),
                              P<float>(a, 5), eps, P<float>(a, 3), P<float>(a, 4), n, k, ctx.stream))
    ctx.error = "gemv_partial_ln: K > 1024, K or N not a multiple of 4, or unaligned operands";
}

// attention_decode_part_f32_gpu(qkv_part[S, 3D], kc[cap, D], vc[cap, D], pos[1], bias[3D]; heads)
//   -> chunks[heads, ceil(cap / 64), 66]; writes row pos of kc, vc
void runAttnDecodePart(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], d3 = a.ints[1], cap = a.ints[2], d = a.ints[3];
  const int heads = static_cast<int>(a.ints[11]);
  LK_REQUIRE(ctx, d3 == 3 * d && d == 64 * heads && a.ints[4] == cap && a.ints[5] == d && a.ints[6] == 1 &&
                      a.ints[7] == d3 && a.ints[8] == heads && a.ints[9] == (cap + 63) / 64 && a.ints[10] == 66,
             "attention_decode_part: expected qkv_part [S, 3D], kc/vc [cap, D], pos [1], bias [3D], D = 64 heads");
  if (lk_hip_attention_decode_part_f32(P<float>(a, 0), s, P<float>(a, 1), P<float>(a, 2), P<int64_t>(a, 3),
                                       P<float>(a, 4), P<float>(a, 5), cap, heads, ctx.stream))
    ctx.error = "attention_decode_part: launch failed";
}

// gemv_partial_embed_ln_f32_gpu(table[V, K], id[1], table2[P, K], id2[1], gamma[K], beta[K], w[K, N]; eps)
//   -> (part[S, N], sum[1, K]); sum = table[id] + table2[id2], x = LN(sum)
void runGemvPartialEmbedLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t v = a.ints[0], k = a.ints[1], p = a.ints[3], n = a.ints[9];
  LK_REQUIRE(ctx, a.ints[2] == 1 && a.ints[4] == k && a.ints[5] == 1 && a.ints[6] == k && a.ints[7] == k &&
                      a.ints[8] == k && a.ints[10] == lk_hip_gemv_partial_slices(k) && a.ints[11] == n &&
                      a.ints[12] == 1 && a.ints[13] == k,
             "gemv_partial_embed_ln: expected table [V, K], id [1], table2 [P, K], id2 [1], gamma [K], beta [K], "
             "w [K, N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_gemv_partial_embed_ln_f32(P<float>(a, 0), P<int64_t>(a, 1), P<float>(a, 2), P<int64_t>(a, 3), v, p,
                                       P<float>(a, 4), P<float>(a, 5), eps, P<float>(a, 6), P<float>(a, 7),
                                       P<float>(a, 8), n, k, ctx.stream))
    ctx.error = "gemv_partial_embed_ln: K > 1024, K or N not a multiple of 4, or unaligned operands";
}

// lm_head_ln_argmax_f32_gpu(part[S, K], bias[K], res[1, K], gamma[K], beta[K], table[V, K]; eps)
//   -> (logits[1, V], argmax i64[1]); logits = LN(slices of part + bias + res) . table^T
void runLmHeadLnArgmax(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], k = a.ints[1], v = a.ints[7];
  LK_REQUIRE(ctx, a.ints[2] == k && a.ints[3] == 1 && a.ints[4] == k && a.ints[5] == k && a.ints[6] == k &&
                      a.ints[8] == k && a.ints[9] == 1 && a.ints[10] == v && a.ints[11] == 1,
             "lm_head_ln_argmax: expected part [S, K], bias [K], res [1, K], gamma [K], beta [K], table [V, K]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  const int rc = lk_hip_lm_head_ln_argmax_f32(P<float>(a, 0), s, P<float>(a, 1), P<float>(a, 2), P<float>(a, 3),
                                              P<float>(a, 4), eps, P<float>(a, 5), P<float>(a, 6), P<int64_t>(a, 7),
                                              v, k, ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes),
                                              ctx.stream);
  status(ctx, rc, rc == 3 ? "lm_head_ln_argmax: workspace too small"
                          : "lm_head_ln_argmax: K > 1024, K not a multiple of 4, or unaligned operands");
}

// reduce_bias_res_ln2_f32_gpu(part[S, N], bias[N], res[1, N], gamma[N], beta[N]; eps) -> (sum[1, N], ln[1, N])
void runReduceLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], n = a.ints[1];
  LK_REQUIRE(ctx, a.ints[2] == n && a.ints[3] == 1 && a.ints[4] == n && a.ints[5] == n && a.ints[6] == n,
             "reduce_bias_res_ln2: expected part [S, N], bias [N], res [1, N], gamma [N], beta [N]");
  const float eps = a.numFloats > 0 ? static_cast<float>(a.floats[0]) : 1e-5f;
  if (lk_hip_reduce_ln_f32(P<float>(a, 0), s, P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), P<float>(a, 4),
                           P<float>(a, 5), P<float>(a, 6), n, eps, ctx.stream))
    ctx.error = "reduce_bias_res_ln2: N > 1024";
}

}  // namespace

void registerDecodeFusedKernels() {
  const Device G = Device::Gpu;
  registerKernel({"gemv_partial_f32_gpu", G, runGemvPartial, 2, 1});
  registerKernel({"gemv_partial_gelu_f32_gpu", G, runGemvPartialGelu, 3, 1});
  registerKernel({"gemv_partial_attn_f32_gpu", G, runGemvPartialAttn, 2, 1});
  registerKernel({"gemv_partial_res_ln_f32_gpu", G, runGemvPartialResLn, 6, 2});
  registerKernel({"gemv_partial_ln_f32_gpu", G, runGemvPartialLn, 4, 2});
  registerKernel({"attention_decode_part_f32_gpu", G, runAttnDecodePart, 5, 1});
  registerKernel({"reduce_bias_res_ln2_f32_gpu", G, runReduceLn, 5, 2});
  registerKernel({"gemv_partial_embed_ln_f32_gpu", G, runGemvPartialEmbedLn, 7, 2});
  registerKernel({"lm_head_ln_argmax_f32_gpu", G, runLmHeadLnArgmax, 6, 2});
}

}  // namespace lkh
