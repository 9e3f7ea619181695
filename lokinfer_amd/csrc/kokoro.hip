// Kokoro frame-rate kernels, channel-last [L, C] (the generator / decoder / F0-N layout).
//
//   lk_hip_channel_stats_lc_f32   per-(128-row chunk, channel) (mean, M2), two passes
//                                 (reference channel_stats_lc_f32_gpu, kokoro_lc.metal:172-208)
//   lk_hip_adain_affine_lc_f32    chunk combine -> affine [3, C] = (mean, (1 + g) / sqrt(var + eps), b)
//                                 (adain_affine_lc_f32_gpu, kokoro_lc.metal:216-260)
//   lk_hip_act_lc_f32             snake / leaky with optional affine (snake_affine_lc / leaky[_affine]_lc,
//                                 kokoro_lc.metal:151-166)
//   lk_hip_convt_gather_lc_f32    ConvTranspose1d overlap-add of x . W[Ci, K*Co] (convt_gather_lc[_add],
//                                 kokoro_lc.metal:262-286)
//   lk_hip_dwconvt_lc_f32         depthwise ConvTranspose1d (dwconvt_lc, kokoro_lc.metal:333-348)
//   lk_hip_upsample2_lc_f32, lk_hip_concat_pad_lc_f32, lk_hip_lc_to_cf_f32, lk_hip_add3_scale_f32,
//   lk_hip_transpose_f32, lk_hip_add_f32, lk_hip_mul_f32           layout / elementwise glue
//   lk_hip_istft_lc_f32           iSTFT from channel-last logits (istft_logits_lc_f32_gpu, kokoro_lc.metal:362-398)
//
// All element-wise kernels are grid-stride over float4 where the channel count allows; the reductions read
// rows of 64 consecutive channels (256 B) per wave.
#include <cmath>

#include "common.h"

namespace lkd {

constexpr int kStatChunk = 128;

// Block = 64 channels x 4 row groups of one 128-row chunk. Pass 1: mean; pass 2: centred M2 (the chunk's rows are
// re-read from L2). Dilation d: the chunks of each residue class rho (rows rho + d i, i < ceil((L - rho) / d)), block
// y = rho chunks + k over rows rho + d (128 k + i), written to st[(rho chunks + k) C + c] (the Winograd GEMM's
// statistics layout; d = 1 is the plain 128-row layout). Chunks past a residue class's rows write nothing.
__global__ __launch_bounds__(256) void statsKernel(const float* __restrict__ x, float* __restrict__ st, int64_t l,
                                                  int64_t c, int d, int64_t chunks) {
  __shared__ float part[4][64];
  const int cl = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * 64 + cl;
  const int64_t s = blockIdx.y;
  const int64_t rho = s / chunks, k = s - rho * chunks;
  const int64_t lor = rho < l ? (l - rho + d - 1) / d : 0;  // rows of this residue class
  const int64_t t0 = k * kStatChunk;
  const int n = static_cast<int>(min<int64_t>(kStatChunk, lor - t0));
  if (n <= 0) return;  // uniform over the block
  const bool ok = ch < c;
  const int r0 = g * 32;
  const int64_t stride = static_cast<int64_t>(d) * c;
  const float* col = x + (rho + t0 * d) * c + (ok ? ch : 0);
  // the thread's 32 rows are loaded once (independent loads in flight) and kept for both passes
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = (ok && r0 + i < n) ? col[static_cast<int64_t>(r0 + i) * stride] : 0.0f;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) sum += v[i];
  part[g][cl] = sum;
  __syncthreads();
  const float mean = (part[0][cl] + part[1][cl] + part[2][cl] + part[3][cl]) / static_cast<float>(n);
  __syncthreads();
  float m2 = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float dv = v[i] - mean;
    if (r0 + i < n) m2 += dv * dv;
  }
  part[g][cl] = m2;
  __syncthreads();
  if (g == 0 && ok) {
    st[(s * c + ch) * 2] = mean;
    st[(s * c + ch) * 2 + 1] = part[0][cl] + part[1][cl] + part[2][cl] + part[3][cl];
  }
}

// AdaIN affine from channel_stats_lc statistics (128-row chunks), 4 channels x 64 chunk slices per workgroup.
__global__ __launch_bounds__(kAffineThreads) void adainAffineKernel(const float* __restrict__ st,
                                                                   const float* __restrict__ gb, float* __restrict__ af,
                                                                   int64_t l, int64_t c, int64_t creal, float eps) {
  adainAffineSlices(st, gb, af, l, c, 1, (l + kStatChunk - 1) / kStatChunk, creal, eps);
}

// act: 1 snake, 2 leaky (0: affine only).
__global__ void actKernel(const float* __restrict__ x, const float* __restrict__ af, const float* __restrict__ alpha,
                          float* __restrict__ out, int64_t n, int64_t c, int act, float slope) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t ch = i % c;
    float v = x[i];
    if (af) v = (v - af[ch]) * af[c + ch] + af[2 * c + ch];
    if (act == 1) {
      const float a = alpha[ch];
      v = v + (1.0f / a) * snakeSinSq(a * v);
    } else if (act == 2) {
      v = v >= 0.0f ? v : v * slope;
    }
    out[i] = v;
  }
}

// out[t, co] = bias + sum_{kk == t + pad (mod s)} y[(t + pad - kk) / s, kk * Co + co] (+ add[t, co]);
// reflect_left: out row 0 is convT row 1, row t is convT row t - 1.
__global__ void convtGatherKernel(const float* __restrict__ y, const float* __restrict__ bias,
                                  const float* __restrict__ add, float* __restrict__ out, int64_t lin, int64_t lout,
                                  int64_t co, int k, int stride, int pad, int reflectLeft) {
  const int64_t n = lout * co;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t tp = i / co, o = i - tp * co;
    const int64_t t = reflectLeft ? (tp == 0 ? 1 : tp - 1) : tp;
    float acc = bias[o];
    const int64_t tpad = t + pad;
    const int64_t ldy = static_cast<int64_t>(k) * co;
    for (int64_t kk = tpad % stride; kk < k; kk += stride) {
      const int64_t num = tpad - kk;
      if (num < 0) break;
      const int64_t j = num / stride;
      if (j < lin) acc += y[j * ldy + kk * co + o];
    }
    if (add) acc += add[i];
    out[i] = acc;
  }
}

__global__ void dwconvtKernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
                              float* __restrict__ out, int64_t lin, int64_t lout, int64_t c, int k, int stride,
                              int pad) {
  const int64_t n = lout * c;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / c, ch = i - t * c;
    float acc = bias[ch];
    const int64_t tpad = t + pad;
    for (int64_t kk = tpad % stride; kk < k; kk += stride) {
      const int64_t num = tpad - kk;
      if (num < 0) break;
      const int64_t j = num / stride;
      if (j < lin) acc += x[j * c + ch] * w[ch * k + kk];
    }
    out[i] = acc;
  }
}

__global__ void upsample2Kernel(const float* __restrict__ x, float* __restrict__ out, int64_t l, int64_t c) {
  const int64_t n = 2 * l * c;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / c, ch = i - t * c;
    out[i] = x[(t / 2) * c + ch];
  }
}

__global__ void concatPadKernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                                int64_t l, int64_t ca, int64_t cb, int64_t cout) {
  const int64_t n = l * cout;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / cout, ch = i - t * cout;
    float v = 0.0f;
    if (ch < ca) v = a[t * ca + ch];
    else if (ch < ca + cb) v = b[t * cb + (ch - ca)];
    out[i] = v;
  }
}

// 32x32 tiles through LDS: x [R, C] -> out [C, R] (rows of both sides coalesced). lc_to_cf is the same with a
// column limit and source stride.
__global__ __launch_bounds__(256) void transposeKernel(const float* __restrict__ x, float* __restrict__ out,
                                                      int64_t r, int64_t c, int64_t ldx) {
  __shared__ float tile[32][33];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 32, r0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int j = ty; j < 32; j += 8) {
    const int64_t rr = r0 + j, cc = c0 + tx;
    tile[j][tx] = (rr < r && cc < c) ? x[rr * ldx + cc] : 0.0f;
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int64_t cc = c0 + j, rr = r0 + tx;
    if (cc < c && rr < r) out[cc * r + rr] = tile[tx][j];
  }
}

// op: 0 add, 1 mul, 2 (a + b + c) * s
__global__ void ewKernel(const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ c,
                         float* __restrict__ out, int64_t n, int op, float s) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (op == 0) out[i] = a[i] + b[i];
    else if (op == 1) out[i] = a[i] * b[i];
    else out[i] = (a[i] + b[i] + c[i]) * s;
  }
}

// iSTFT from channel-last logits x [L, Cpad]: column k < K = nfft / 2 + 1 is the log-magnitude, K + k the phase
// logit of bin k; X_k = exp(mag) e^{i sin(phase)}. Per frame the window-folded inverse real DFT (backward norm
// 1/N), then overlap-add in ascending frame order divided by the window-square envelope (torch.istft with a
// periodic Hann window, center = True). A workgroup synthesises the frames its 256 * hop output samples touch
// (its own plus nfft / hop halo frames) into LDS.
constexpr int kIstftMaxN = 64;
constexpr int kIstftFrames = 256;
// NF > 0: nfft == NF at compile time, so a frame's 2 (NF / 2 + 1) logit loads are independent and in flight together
// (a runtime-length loop waits for each load in turn: 136 us at 293281 frames).
template <int NF>
__global__ __launch_bounds__(256) void istftKernel(const float* __restrict__ x, float* __restrict__ out, int64_t l,
                                                  int64_t cpad, int nfftArg, int hop) {
  extern __shared__ float smem[];
  __shared__ float tabRe[33 * kIstftMaxN], tabIm[33 * kIstftMaxN], win[kIstftMaxN];
  const int nfft = NF > 0 ? NF : nfftArg;
  const int bins = nfft / 2 + 1, pad = nfft / 2;
  for (int i = threadIdx.x; i < bins * nfft; i += blockDim.x) {
    const int k = i / nfft, m = i % nfft;
    const bool edge = k == 0 || 2 * k == nfft;
    const double wm = 0.5 - 0.5 * cos(2.0 * M_PI * static_cast<double>(m) / static_cast<double>(nfft));
    const double ang = 2.0 * M_PI * static_cast<double>((k * m) % nfft) / static_cast<double>(nfft);
    const double cc = (edge ? 1.0 : 2.0) * static_cast<double>(static_cast<float>(wm)) / static_cast<double>(nfft);
    tabRe[i] = static_cast<float>(cc * cos(ang));
    tabIm[i] = edge ? 0.0f : static_cast<float>(-cc * sin(ang));
  }
  for (int m = threadIdx.x; m < nfft; m += blockDim.x)
    win[m] = static_cast<float>(0.5 - 0.5 * cos(2.0 * M_PI * static_cast<double>(m) / static_cast<double>(nfft)));
  __syncthreads();
  const int64_t len = static_cast<int64_t>(hop) * (l - 1);
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kIstftFrames * hop;
  // Frames touched by samples [i0, i0 + 256 hop): t in [tFirst, tLast].
  const int64_t p0 = i0 + pad;
  const int64_t tFirst = p0 >= nfft ? (p0 - nfft) / hop + 1 : 0;
  const int nHalo = (nfft + hop - 1) / hop + 3;
  const int nFrames = kIstftFrames + nHalo;
  float* fr = smem;  // [nFrames][nfft]
  for (int f = threadIdx.x; f < nFrames; f += blockDim.x) {
    const int64_t t = tFirst + f;
    if (t >= l) continue;
    const float* xt = x + t * cpad;
    if constexpr (NF > 0) {
      constexpr int B = NF / 2 + 1;
      float lm[B], lp[B], re[B], im[B];
#pragma unroll
      for (int k = 0; k < B; ++k) {
        lm[k] = xt[k];
        lp[k] = xt[B + k];
      }
#pragma unroll
      for (int k = 0; k < B; ++k) {
        const float mag = expf(lm[k]);
        const float ph = sinf(lp[k]);
        re[k] = mag * cosf(ph);
        im[k] = mag * sinf(ph);
      }
#pragma unroll
      for (int m = 0; m < NF; ++m) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < B; ++k) v += re[k] * tabRe[k * NF + m] + im[k] * tabIm[k * NF + m];
        fr[f * NF + m] = v;
      }
    } else {
      float re[33], im[33];
      for (int k = 0; k < bins; ++k) {
        const float mag = expf(xt[k]);
        const float ph = sinf(xt[bins + k]);
        re[k] = mag * cosf(ph);
        im[k] = mag * sinf(ph);
      }
      for (int m = 0; m < nfft; ++m) {
        float v = 0.0f;
        for (int k = 0; k < bins; ++k) v += re[k] * tabRe[k * nfft + m] + im[k] * tabIm[k * nfft + m];
        fr[f * nfft + m] = v;
      }
    }
  }
  __syncthreads();
  for (int64_t i = i0 + threadIdx.x; i < min<int64_t>(len, i0 + static_cast<int64_t>(kIstftFrames) * hop);
       i += blockDim.x) {
    const int64_t p = pad + i;
    const int64_t tHi = min<int64_t>(l - 1, p / hop);
    const int64_t tLo = p >= nfft ? (p - nfft) / hop + 1 : 0;
    float y = 0.0f, env = 0.0f;
    for (int64_t t = tLo; t <= tHi; ++t) {
      const int m = static_cast<int>(p - t * hop);
      if (t < tFirst || t - tFirst >= nFrames) continue;  // unreachable by construction of nHalo
      y += fr[(t - tFirst) * nfft + m];
      env += win[m] * win[m];
    }
    out[i] = y / env;
  }
}

// n_fft = 20, hop = 5 (the model's): the same synthesis with a host-built table (the window-folded DFT and the
// window, double cos / sin rounded to f32, as the kernel above builds them), the sizes as constants (the divisions
// by hop become multiplies) and 32-bit indices (L hop < 2^31). A workgroup owns 249 hops of output, so it
// synthesizes exactly 256 frames (its own and the 7 halo frames), one per thread, in one pass.
struct IstftTable20 {
  float re[11 * 20], im[11 * 20], win[20];
};

__global__ __launch_bounds__(256) void istft20Kernel(const float* __restrict__ x, float* __restrict__ out, int l,
                                                    int cpad, IstftTable20 host) {
  constexpr int NF = 20, HOP = 5, B = 11, PAD = 10;
  constexpr int NHALO = (NF + HOP - 1) / HOP + 3;
  constexpr int NFR = 256, FRAMES = NFR - NHALO;  // one synthesized frame per thread: FRAMES hops of output each
  __shared__ float tabRe[B * NF], tabIm[B * NF], win[NF], fr[NFR * NF];
  for (int i = threadIdx.x; i < B * NF; i += blockDim.x) {
    tabRe[i] = host.re[i];
    tabIm[i] = host.im[i];
  }
  if (threadIdx.x < NF) win[threadIdx.x] = host.win[threadIdx.x];
  __syncthreads();
  const int len = HOP * (l - 1);
  const int i0 = blockIdx.x * FRAMES * HOP;
  // Frames touched by samples [i0, i0 + FRAMES hop): t in [tFirst, tFirst + NFR).
  const int p0 = i0 + PAD;
  const int tFirst = p0 >= NF ? (p0 - NF) / HOP + 1 : 0;
  for (int f = threadIdx.x; f < NFR; f += blockDim.x) {
    const int t = tFirst + f;
    if (t >= l) continue;
    const float* xt = x + static_cast<int64_t>(t) * cpad;
    float lm[B], lp[B], re[B], im[B];
#pragma unroll
    for (int k = 0; k < B; ++k) {
      lm[k] = xt[k];
      lp[k] = xt[B + k];
    }
#pragma unroll
    for (int k = 0; k < B; ++k) {
      const float mag = expf(lm[k]);
      const float ph = sinf(lp[k]);
      re[k] = mag * cosf(ph);
      im[k] = mag * sinf(ph);
    }
#pragma unroll
    for (int m = 0; m < NF; ++m) {
      float v = 0.0f;
#pragma unroll
      for (int k = 0; k < B; ++k) v += re[k] * tabRe[k * NF + m] + im[k] * tabIm[k * NF + m];
      fr[f * NF + m] = v;
    }
  }
  __syncthreads();
  const int iEnd = min(len, i0 + FRAMES * HOP);
  for (int i = i0 + threadIdx.x; i < iEnd; i += blockDim.x) {
    const int p = PAD + i;
    const int tHi = min(l - 1, p / HOP);
    const int tLo = p >= NF ? (p - NF) / HOP + 1 : 0;
    float y = 0.0f, env = 0.0f;
    for (int t = tLo; t <= tHi; ++t) {
      const int m = p - t * HOP;
      if (t < tFirst || t - tFirst >= NFR) continue;  // unreachable by construction of NHALO
      y += fr[(t - tFirst) * NF + m];
      env += win[m] * win[m];
    }
    out[i] = y / env;
  }
}

inline unsigned gridFor(int64_t n, int threads = 256) {
  const int64_t b = (n + threads - 1) / threads;
  return static_cast<unsigned>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace lkd

namespace lkh {
// Statistics per residue class of dilation d in 128-row chunks (chunks = ceil(ceil(L / d) / 128) per class), the
// Winograd GEMM's layout: the split-K path of the Winograd GEMM computes them from the summed output.
int residueStats(const float* x, float* st, int64_t l, int64_t c, int d, int64_t chunks, hipStream_t s) {
  if (l <= 0 || c <= 0 || d < 1 || chunks < 1) return 1;
  dim3 grid(static_cast<unsigned>(ceilDiv(c, 64)), static_cast<unsigned>(d * chunks));
  hipLaunchKernelGGL(lkd::statsKernel, grid, dim3(256), 0, s, x, st, l, c, d, chunks);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
}  // namespace lkh

#define LK_RET return hipGetLastError() == hipSuccess ? 0 : 2

extern "C" {

int lk_hip_channel_stats_lc_f32(const float* x, float* st, int64_t l, int64_t c, void* stream) {
  if (l <= 0 || c <= 0) return 1;
  const int64_t chunks = lkh::ceilDiv(l, lkd::kStatChunk);
  dim3 grid(lkh::ceilDiv(c, 64), chunks);
  hipLaunchKernelGGL(lkd::statsKernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), x, st, l, c, 1, chunks);
  LK_RET;
}

int lk_hip_adain_affine_lc_f32(const float* st, const float* gb, float* af, int64_t l, int64_t c, int64_t creal,
                               float eps, void* stream) {
  if (l <= 0 || c <= 0 || creal > c) return 1;
  hipLaunchKernelGGL(lkd::adainAffineKernel, dim3(lkh::ceilDiv(c, lkd::kAffineCh)), dim3(lkd::kAffineThreads), 0,
                     static_cast<hipStream_t>(stream), st, gb, af, l, c, creal, eps);
  LK_RET;
}

int lk_hip_act_lc_f32(const float* x, const float* af, const float* alpha, float* out, int64_t l, int64_t c, int act,
                      float slope, void* stream) {
  const int64_t n = l * c;
  if (n <= 0) return n == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::actKernel, dim3(lkd::gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream), x, af,
                     alpha, out, n, c, act, slope);
  LK_RET;
}

int lk_hip_convt_gather_lc_f32(const float* y, const float* bias, const float* add, float* out, int64_t lin,
                               int64_t lout, int64_t co, int k, int stride, int pad, int reflectLeft, void* stream) {
  const int64_t n = lout * co;
  if (n <= 0) return 1;
  hipLaunchKernelGGL(lkd::convtGatherKernel, dim3(lkd::gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     y, bias, add, out, lin, lout, co, k, stride, pad, reflectLeft);
  LK_RET;
}

int lk_hip_dwconvt_lc_f32(const float* x, const float* w, const float* bias, float* out, int64_t lin, int64_t lout,
                          int64_t c, int k, int stride, int pad, void* stream) {
  const int64_t n = lout * c;
  if (n <= 0) return 1;
  hipLaunchKernelGGL(lkd::dwconvtKernel, dim3(lkd::gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                     w, bias, out, lin, lout, c, k, stride, pad);
  LK_RET;
}

int lk_hip_upsample2_lc_f32(const float* x, float* out, int64_t l, int64_t c, void* stream) {
  hipLaunchKernelGGL(lkd::upsample2Kernel, dim3(lkd::gridFor(2 * l * c)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, out, l, c);
  LK_RET;
}

int lk_hip_concat_pad_lc_f32(const float* a, const float* b, float* out, int64_t l, int64_t ca, int64_t cb,
                             int64_t cout, void* stream) {
  if (cout < ca + cb) return 1;
  hipLaunchKernelGGL(lkd::concatPadKernel, dim3(lkd::gridFor(l * cout)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a, b, out, l, ca, cb, cout);
  LK_RET;
}

// x [R, ldx] (first C columns used) -> out [C, R].
int lk_hip_transpose_f32(const float* x, float* out, int64_t r, int64_t c, int64_t ldx, void* stream) {
  if (r <= 0 || c <= 0) return r == 0 || c == 0 ? 0 : 1;
  dim3 grid(lkh::ceilDiv(c, 32), lkh::ceilDiv(r, 32));
  hipLaunchKernelGGL(lkd::transposeKernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), x, out, r, c, ldx);
  LK_RET;
}

// op 0: a + b; 1: a * b; 2: (a + b + c) * s.
int lk_hip_elementwise_f32(const float* a, const float* b, const float* c, float* out, int64_t n, int op, float s,
                           void* stream) {
  if (n <= 0) return n == 0 ? 0 : 1;
  hipLaunchKernelGGL(lkd::ewKernel, dim3(lkd::gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream), a, b, c,
                     out, n, op, s);
  LK_RET;
}

int lk_hip_istft_lc_f32(const float* x, float* out, int64_t l, int64_t cpad, int nfft, int hop, void* stream) {
  if (nfft < 2 || nfft % 2 || nfft > lkd::kIstftMaxN || hop < 1 || l < 2 || cpad < nfft + 2) return 1;
  const int64_t len = static_cast<int64_t>(hop) * (l - 1);
  const unsigned blocks = lkh::ceilDiv(len, static_cast<int64_t>(lkd::kIstftFrames) * hop);
  const int nHalo = (nfft + hop - 1) / hop + 3;
  const size_t shm = static_cast<size_t>(lkd::kIstftFrames + nHalo) * nfft * sizeof(float);
  if (nfft == 20 && hop == 5 && len < (int64_t{1} << 30)) {  // the model's n_fft and hop
    static const lkd::IstftTable20 tab = [] {
      lkd::IstftTable20 t{};
      for (int i = 0; i < 11 * 20; ++i) {
        const int k = i / 20, m = i % 20;
        const bool edge = k == 0 || 2 * k == 20;
        const double wm = 0.5 - 0.5 * std::cos(2.0 * M_PI * static_cast<double>(m) / 20.0);
        const double ang = 2.0 * M_PI * static_cast<double>((k * m) % 20) / 20.0;
        const double cc = (edge ? 1.0 : 2.0) * static_cast<double>(static_cast<float>(wm)) / 20.0;
        t.re[i] = static_cast<float>(cc * std::cos(ang));
        t.im[i] = edge ? 0.0f : static_cast<float>(-cc * std::sin(ang));
      }
      for (int m = 0; m < 20; ++m)
        t.win[m] = static_cast<float>(0.5 - 0.5 * std::cos(2.0 * M_PI * static_cast<double>(m) / 20.0));
      return t;
    }();
    const unsigned b20 = static_cast<unsigned>(lkh::ceilDiv(len, int64_t{(256 - 7) * 5}));
    hipLaunchKernelGGL(lkd::istft20Kernel, dim3(b20), dim3(256), 0, static_cast<hipStream_t>(stream), x, out,
                       static_cast<int>(l), static_cast<int>(cpad), tab);
  } else if (nfft == 20) {
    hipLaunchKernelGGL(lkd::istftKernel<20>, dim3(blocks), dim3(256), shm, static_cast<hipStream_t>(stream), x, out, l,
                       cpad, nfft, hop);
  } else
    hipLaunchKernelGGL(lkd::istftKernel<0>, dim3(blocks), dim3(256), shm, static_cast<hipStream_t>(stream), x, out, l,
                       cpad, nfft, hop);
  LK_RET;
}

}  // extern "C"
