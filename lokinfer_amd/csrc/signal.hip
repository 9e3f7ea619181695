// Kokoro signal path on the GPU (the reference runs these as host CPU kernels, kernels/cpu/kokoro_signal.cpp):
//
//   lk_hip_harmonic_source_f32  hn-NSF source (SineGen, 9 harmonics) with explicit noise
//                               (harmonic_source_f32_cpu, kokoro_signal.cpp:89-192)
//   lk_hip_stft_magphase_lc_f32 STFT -> magnitude | phase, channel-last and zero-padded to a multiple of 16
//                               columns for the implicit-GEMM conv that consumes it
//                               (stft_magphase_f32_cpu, kokoro_signal.cpp:196-273)
//   lk_hip_conv1d_1ch_f32       single-channel strided conv1d (the decoder's F0_conv / N_conv, which the
//                               reference runs as conv1d_f32_cpu, models/kokoro/model.py:704-705)
//
// The harmonic source keeps the reference's f32 op order, which is PyTorch's: per frame j and harmonic h the
// phase increment rad = remainder(f0 (h + 1) / 24000, 1) is accumulated in double and rounded to f32, then
// ((phase * 2) * pi) * 300; the x300 linear upsample uses src = fma(1/300, i + 0.5, -0.5) and
// fma(t0, l0, t1 * l1); the merge is y += v * w[h] in harmonic order, then tanh(y + b). With the same F0 input
// the f32 phases are bit-identical to the CPU restatement, which matters because they reach ~1e6 rad.
#include "common.h"

#include <algorithm>
#include <cmath>

// Every fused multiply-add in this file is an explicit __builtin_fmaf; nothing else may be contracted.
#pragma clang fp contract(off)

namespace lkd {

constexpr int kHarm = 9;

__device__ __forceinline__ float torchRemainder1(float a) {
  float m = fmodf(a, 1.0f);
  if (m != 0.0f && m < 0.0f) m += 1.0f;
  return m;
}

// One wave per harmonic: wave-level inclusive scans of 64 frames in double plus a running carry (the sums of
// f32 increments in [0, 1) over <= 2^16 frames are exact in double, so the scan order does not change them).
// p300[j, h] = ((f32(acc) * 2) * pi) * 300.
__global__ __launch_bounds__(64 * kHarm) void harmonicPhaseKernel(const float* __restrict__ f0,
                                                                 float* __restrict__ p300, int64_t n) {
  const int h = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double carry = 0.0;
  const float hf = static_cast<float>(h + 1);
  for (int64_t j0 = 0; j0 < n; j0 += 64) {
    const int64_t j = j0 + lane;
    double v = 0.0;
    if (j < n) {
      const float fn = f0[j] * hf;
      v = static_cast<double>(torchRemainder1(fn / 24000.0f));
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const double u = __shfl_up(v, o, 64);
      if (lane >= o) v += u;
    }
    const double acc = carry + v;
    if (j < n) {
      const float phase = (static_cast<float>(acc) * 2.0f) * 3.14159265358979323846f;
      p300[j * kHarm + h] = phase * 300.0f;
    }
    carry += __shfl(v, 63, 64);
  }
}

// The same phases for n <= kHarmLds frames: one workgroup per harmonic (so the nine scans run on nine CUs), f0
// staged in LDS first; thread T walks the contiguous frames [T seg, (T + 1) seg), seg = ceil(n / 256): it sums its
// increments in double, a workgroup scan of the 256 sums (wave scans, then the wave totals through LDS) gives each
// thread its prefix, and the thread re-walks its frames with the running sum. The sums of f32 increments in [0, 1)
// are exact in double, so this order gives the values of the frame-by-frame scan above. (That scan, all nine
// harmonics in one workgroup, runs n / 64 dependent rounds of a global load and six shuffles: 57 us at n = 4888.)
constexpr int kHarmLds = 16384;
__global__ __launch_bounds__(256) void harmonicPhaseLdsKernel(const float* __restrict__ f0, float* __restrict__ p300,
                                                              int n) {
  __shared__ float f0s[kHarmLds];
  __shared__ double waveTotal[4];
  for (int j = threadIdx.x; j < n; j += blockDim.x) f0s[j] = f0[j];
  __syncthreads();
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float hf = static_cast<float>(h + 1);
  const int seg = (n + 255) / 256;
  const int j0 = min(n, tid * seg), j1 = min(n, j0 + seg);
  double sum = 0.0;
  for (int j = j0; j < j1; ++j) sum += static_cast<double>(torchRemainder1(f0s[j] * hf / 24000.0f));
  double pre = sum;  // inclusive scan within the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(pre, o, 64);
    if (lane >= o) pre += u;
  }
  if (lane == 63) waveTotal[wave] = pre;
  __syncthreads();
  double acc = 0.0;  // this thread's exclusive prefix: the earlier waves' totals, then the left neighbour's scan
  for (int w = 0; w < wave; ++w) acc += waveTotal[w];
  const double left = __shfl_up(pre, 1, 64);
  if (lane > 0) acc += left;
  for (int j = j0; j < j1; ++j) {
    acc += static_cast<double>(torchRemainder1(f0s[j] * hf / 24000.0f));
    const float phase = (static_cast<float>(acc) * 2.0f) * 3.14159265358979323846f;
    p300[static_cast<int64_t>(j) * kHarm + h] = phase * 300.0f;
  }
}

__global__ void harmonicSourceKernel(const float* __restrict__ f0, const float* __restrict__ p300,
                                     const float* __restrict__ noise, const float* __restrict__ w,
                                     const float* __restrict__ b, float* __restrict__ out, int64_t n) {
  const int64_t s = n * 300;
  const float scale = static_cast<float>(1.0 / 300.0);
  const float ampV = 0.003f, ampU = (1.0f * 0.1f) / 3.0f;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < s;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float real = __builtin_fmaf(scale, static_cast<float>(i) + 0.5f, -0.5f);
    real = fmaxf(real, 0.0f);
    int64_t i0 = static_cast<int64_t>(floorf(real));
    if (i0 > n - 1) i0 = n - 1;
    const float l1 = fminf(fmaxf(real - static_cast<float>(i0), 0.0f), 1.0f);
    const float l0 = 1.0f - l1;
    const int64_t i1 = i0 < n - 1 ? i0 + 1 : i0;
    const bool voiced = f0[i / 300] > 10.0f;
    const float uv = voiced ? 1.0f : 0.0f, amp = voiced ? ampV : ampU;
    float y = 0.0f;
#pragma unroll
    for (int h = 0; h < kHarm; ++h) {
      const float t0 = p300[i0 * kHarm + h], t1 = p300[i1 * kHarm + h];
      const float phase = __builtin_fmaf(t0, l0, t1 * l1);
      // sin and tanh in double, rounded once to f32: correctly rounded (up to ties ~2^-29 apart), so the source
      // is reproducible bit for bit by any implementation that rounds the same exact values.
      const float sine = static_cast<float>(sin(static_cast<double>(phase))) * 0.1f;
      const float v = sine * uv + amp * noise[i * kHarm + h];
      y = y + v * w[h];
    }
    out[i] = static_cast<float>(tanh(static_cast<double>(y + b[0])));
  }
}

// The DFT table for nfft = NF, built on the host (double cos / sin, rounded to f32) and passed by value.
template <int NF>
struct StftTable {
  float re[(NF / 2 + 1) * NF], im[(NF / 2 + 1) * NF];
};

// n_fft = 20 (the model's): one thread per (frame t, bin k), k fastest. An interior frame reads its 20 samples at
// immediate offsets from one base (only the first and last frames reflect); the bin's sums use the host-built
// table in LDS, accumulated over m in order as below; the thread writes the bin's magnitude (column k), phase
// (column 11 + k) and, for k < ldo - 22, the zero column 22 + k. 32-bit index math (s < 2^31).
__global__ __launch_bounds__(256) void stft20Kernel(const float* __restrict__ x, float* __restrict__ out, int s,
                                                   int frames, int hop, int ldo, StftTable<20> host) {
  constexpr int NF = 20, B = 11, PAD = 10;
  __shared__ float tabRe[B * NF], tabIm[B * NF];
  for (int i = threadIdx.x; i < B * NF; i += blockDim.x) {
    tabRe[i] = host.re[i];
    tabIm[i] = host.im[i];
  }
  __syncthreads();
  const int total = frames * B;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int t = i / B, k = i - t * B;
    const int base = t * hop - PAD;
    float fr[NF];
    if (base >= 0 && base + NF <= s) {
      const float* xb = x + base;
#pragma unroll
      for (int m = 0; m < NF; ++m) fr[m] = xb[m];
    } else {
#pragma unroll
      for (int m = 0; m < NF; ++m) {
        int q = base + m;
        if (q < 0) q = -q;
        if (q >= s) q = 2 * (s - 1) - q;
        fr[m] = x[q];
      }
    }
    float re = 0.0f, im = 0.0f;
#pragma unroll
    for (int m = 0; m < NF; ++m) {
      re += tabRe[k * NF + m] * fr[m];
      im += tabIm[k * NF + m] * fr[m];
    }
    // Real-input DFT: the DC and Nyquist bins are exactly real. So is every bin of frame 0: with center = True
    // and reflect padding that frame is even about its centre (as is the periodic Hann window), and its exact
    // imaginary parts are 0 rather than rounding noise whose sign would flip the phase between +pi and -pi.
    if (k == 0 || 2 * k == NF || t == 0) im = 0.0f;
    float* o = out + static_cast<int64_t>(t) * ldo;
    o[k] = sqrtf(__builtin_fmaf(re, re, im * im));
    o[B + k] = atan2f(im, re);
    for (int c = 2 * B + k; c < ldo; c += B) o[c] = 0.0f;
  }
}

// One thread per output element (frame t, column c; c fastest, so a wave's stores are contiguous): columns < bins
// hold the magnitude of bin c, bins .. 2 bins - 1 the phase of bin c - bins, the rest 0. A bin is the windowed DFT of
// the reflect-padded frame (center = True) by a table built like the reference's (double cos / sin, rounded to f32),
// accumulated over m in order; the magnitude and phase threads of a bin compute the same sums. Grid-stride, so the
// per-workgroup table build is amortized. (One thread per frame ran 114 us at 293281 samples: 230 workgroups and
// 32 strided stores per thread; most of it was the load latency below.)
// NF > 0: nfft == NF at compile time, so a frame's NF sample loads are independent and in flight together (a
// runtime-length loop issues one load per iteration and waits for it: 110 us at 293281 samples).
constexpr int kStftMaxN = 64;
template <int NF>
__global__ __launch_bounds__(256) void stftKernel(const float* __restrict__ x, float* __restrict__ out, int64_t s,
                                                 int64_t frames, int nfftArg, int hop, int64_t ldo,
                                                 StftTable<NF> host) {
  __shared__ float tabRe[33 * kStftMaxN], tabIm[33 * kStftMaxN];
  const int nfft = NF > 0 ? NF : nfftArg;
  const int bins = nfft / 2 + 1, pad = nfft / 2;
  for (int i = threadIdx.x; i < bins * nfft; i += blockDim.x) {
    if constexpr (NF > 0) {
      tabRe[i] = host.re[i];
      tabIm[i] = host.im[i];
    } else {
      const int k = i / nfft, m = i % nfft;
      const float win = static_cast<float>(0.5 - 0.5 * cos(2.0 * M_PI * static_cast<double>(m) / nfft));
      const double ang = 2.0 * M_PI * static_cast<double>((k * m) % nfft) / static_cast<double>(nfft);
      tabRe[i] = static_cast<float>(win * cos(ang));
      tabIm[i] = static_cast<float>(-win * sin(ang));
    }
  }
  __syncthreads();
  const int64_t total = frames * ldo;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / ldo;
    const int c = static_cast<int>(i - t * ldo);
    float v = 0.0f;
    if (c < 2 * bins) {
      const int k = c < bins ? c : c - bins;
      float re = 0.0f, im = 0.0f;
      if constexpr (NF > 0) {
        float fr[NF];
#pragma unroll
        for (int m = 0; m < NF; ++m) {
          int64_t q = t * hop + m - pad;
          if (q < 0) q = -q;
          if (q >= s) q = 2 * (s - 1) - q;
          fr[m] = x[q];
        }
#pragma unroll
        for (int m = 0; m < NF; ++m) {
          re += tabRe[k * NF + m] * fr[m];
          im += tabIm[k * NF + m] * fr[m];
        }
      } else {
        for (int m = 0; m < nfft; ++m) {
          int64_t q = t * hop + m - pad;
          if (q < 0) q = -q;
          if (q >= s) q = 2 * (s - 1) - q;
          const float xv = x[q];
          re += tabRe[k * nfft + m] * xv;
          im += tabIm[k * nfft + m] * xv;
        }
      }
      // Real-input DFT: the DC and Nyquist bins are exactly real. So is every bin of frame 0: with center = True
      // and reflect padding that frame is even about its centre (as is the periodic Hann window), and its exact
      // imaginary parts are 0 rather than rounding noise whose sign would flip the phase between +pi and -pi.
      if (k == 0 || 2 * k == nfft || t == 0) im = 0.0f;
      v = c < bins ? sqrtf(__builtin_fmaf(re, re, im * im)) : atan2f(im, re);
    }
    out[i] = v;
  }
}

__global__ void conv1chKernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
                              float* __restrict__ out, int64_t l, int64_t lo, int k, int stride, int pad) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= lo) return;
  float acc = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    const int64_t src = i * stride - pad + kk;
    if (src >= 0 && src < l) acc += x[src] * w[kk];
  }
  out[i] = acc + b[0];
}

}  // namespace lkd

extern "C" {

// f0 [n], noise [300 n, 9], w [9], b [1] -> out [300 n]; workspace >= n * 9 floats (the phase table).
int lk_hip_harmonic_source_f32(const float* f0, const float* noise, const float* w, const float* b, float* out,
                               int64_t n, void* workspace, int64_t workspaceBytes, void* stream) {
  if (n < 1) return 1;
  if (!workspace || workspaceBytes < n * lkd::kHarm * 4) return 3;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* p300 = static_cast<float*>(workspace);
  if (n <= lkd::kHarmLds)
    hipLaunchKernelGGL(lkd::harmonicPhaseLdsKernel, dim3(lkd::kHarm), dim3(256), 0, st, f0, p300,
                       static_cast<int>(n));
  else
    hipLaunchKernelGGL(lkd::harmonicPhaseKernel, dim3(1), dim3(64 * lkd::kHarm), 0, st, f0, p300, n);
  const int64_t s = n * 300;
  const int64_t blocks = std::min<int64_t>((s + 255) / 256, 65536);
  hipLaunchKernelGGL(lkd::harmonicSourceKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, f0, p300,
                     noise, w, b, out, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// x [S] -> out [frames, ldo], frames = S / hop + 1, columns 0..K-1 magnitude, K..2K-1 phase, rest 0.
int lk_hip_stft_magphase_lc_f32(const float* x, float* out, int64_t s, int nfft, int hop, int64_t ldo, void* stream) {
  if (nfft < 2 || nfft % 2 || nfft > lkd::kStftMaxN || hop < 1 || s <= nfft / 2 || ldo < nfft + 2) return 1;
  const int64_t frames = s / hop + 1;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(lkh::ceilDiv(frames * ldo, 256), 2048));
  if (nfft == 20) {  // the model's n_fft: the table built once on the host, as the kernel builds it otherwise
    static const lkd::StftTable<20> tab = [] {
      lkd::StftTable<20> t{};
      for (int i = 0; i < 11 * 20; ++i) {
        const int k = i / 20, m = i % 20;
        const float win = static_cast<float>(0.5 - 0.5 * std::cos(2.0 * M_PI * static_cast<double>(m) / 20));
        const double ang = 2.0 * M_PI * static_cast<double>((k * m) % 20) / 20.0;
        t.re[i] = static_cast<float>(win * std::cos(ang));
        t.im[i] = static_cast<float>(-win * std::sin(ang));
      }
      return t;
    }();
    if (s < (int64_t{1} << 30) && frames * 11 < (int64_t{1} << 30)) {
      const unsigned b20 = static_cast<unsigned>(std::min<int64_t>(lkh::ceilDiv(frames * 11, 256), 4096));
      hipLaunchKernelGGL(lkd::stft20Kernel, dim3(b20), dim3(256), 0, static_cast<hipStream_t>(stream), x, out,
                         static_cast<int>(s), static_cast<int>(frames), hop, static_cast<int>(ldo), tab);
    } else {
      hipLaunchKernelGGL(lkd::stftKernel<20>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, out, s,
                         frames, nfft, hop, ldo, tab);
    }
  } else {
    hipLaunchKernelGGL(lkd::stftKernel<0>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, out, s,
                       frames, nfft, hop, ldo, lkd::StftTable<0>{});
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_conv1d_1ch_f32(const float* x, const float* w, const float* b, float* out, int64_t l, int k, int stride,
                          int pad, void* stream) {
  const int64_t lo = (l + 2 * pad - k) / stride + 1;
  if (lo < 1 || stride < 1) return 1;
  hipLaunchKernelGGL(lkd::conv1chKernel, dim3(lkh::ceilDiv(lo, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, w, b, out, l, lo, k, stride, pad);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// harmonic_source_f32_gpu(f0[n], noise[300 n, 9], w[9], b[1]) -> [300 n]
void runHarmonic(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t n = a.ints[0];
  LK_REQUIRE(ctx, a.ints[1] == 300 * n && a.ints[2] == 9 && a.ints[3] == 9 && a.ints[4] == 1,
             "harmonic_source: expected f0 [n], noise [300 n, 9], w [9], b [1]");
  const int rc = lk_hip_harmonic_source_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3),
                                            P<float>(a, 4), n, ctx.workspace,
                                            static_cast<int64_t>(ctx.workspaceBytes), ctx.stream);
  if (rc) ctx.error = rc == 3 ? "harmonic_source: workspace too small" : "harmonic_source: failed";
}

// stft_magphase_lc_f32_gpu(x[S]; hop, n_fft) -> [S / hop + 1, Cpad]
void runStft(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t s = a.ints[0], ldo = a.ints[2];
  const int hop = static_cast<int>(a.ints[3]), nfft = static_cast<int>(a.ints[4]);
  LK_REQUIRE(ctx, a.ints[1] == s / hop + 1, "stft_magphase_lc: bad output rows");
  if (lk_hip_stft_magphase_lc_f32(P<float>(a, 0), P<float>(a, 1), s, nfft, hop, ldo, ctx.stream))
    ctx.error = "stft_magphase_lc: invalid configuration";
}

// conv1d_1ch_f32_gpu(x[L], w[K], b[1]; padding, stride) -> [Lo]
void runConv1ch(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t l = a.ints[0];
  const int k = static_cast<int>(a.ints[1]);
  const int pad = static_cast<int>(a.ints[4]), stride = static_cast<int>(a.ints[5]);
  if (lk_hip_conv1d_1ch_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), l, k, stride, pad,
                            ctx.stream))
    ctx.error = "conv1d_1ch: invalid configuration";
}

}  // namespace

void registerSignalKernels() {
  const Device G = Device::Gpu;
  registerKernel({"harmonic_source_f32_gpu", G, runHarmonic, 4, 1});
  registerKernel({"stft_magphase_lc_f32_gpu", G, runStft, 1, 1});
  registerKernel({"conv1d_1ch_f32_gpu", G, runConv1ch, 3, 1});
}

}  // namespace lkh
