// Kokoro token-rate sequence kernels on the GPU (the reference runs these on the host CPU inside its GPU graph):
//
//   lk_hip_lstm_bidir_f32      1-layer bidirectional nn.LSTM (gates i, f, g, o; b = b_ih + b_hh)
//                              (reference lstm_bidir_f32_cpu / lstm_bidir_t_f32_cpu, ops/kokoro.py:88-116,
//                              kernels/cpu/kokoro_lstm.cpp)
//   lk_hip_repeat_interleave_f32  x.repeat_interleave(dur, 0) (repeat_interleave_f32_cpu, kokoro_misc.cpp:253-265)
//   lk_hip_adalayernorm_f32    (1 + g) * LN_noaffine(x) + b (adalayernorm_f32_cpu, kokoro_norm.cpp:10-62)
//   lk_hip_concat_bcast_f32    [x | v] per row (concat_cols + broadcast_rows, ops/kokoro.py:141-173)
//
// LSTM design: the input projection of every step, G = x W_ih^T + b for both directions, is one MFMA GEMM; the
// recurrence then runs as one 4H-thread workgroup per direction. Thread i owns gate row i and reads column i
// of W_hh^T (layout [H, 8H], the reference's lstm_bidir_t weight) for k = 0..H-1, so a wave's 64 loads of one k
// are 256 contiguous bytes; h(t-1) is broadcast from LDS. After a barrier, threads j < H apply the cell update
// in the reference order (c = f c + i g, h = o tanh(c)). Both directions run concurrently on two CUs.
#include "common.h"
#include "lokinfer_hip.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>

namespace lkd {

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

// 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal (each within 1 ulp; absolute error of a few
// 1e-8); saturates to 0 / 1 for large |x|. tanh(x) = 2 sigmoid(2x) - 1 to the same absolute error, so one
// branch-free sequence serves every gate of an LSTM cell.
__device__ __forceinline__ float sigmoidHw(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float tanhHw(float x) { return fmaf(2.0f, sigmoidHw(2.0f * x), -1.0f); }

// g: [T, 8H] gate pre-activations (forward gates in columns 0..4H, backward 4H..8H); whhT: [H, 8H];
// out: [T, 2H] = [h_fwd | h_bwd]. blockIdx.x = direction, blockDim.x = 4H.
__global__ __launch_bounds__(1024) void lstmRecurrenceKernel(const float* __restrict__ g,
                                                            const float* __restrict__ whhT, float* __restrict__ out,
                                                            int64_t t, int h) {
  __shared__ float hs[256];
  __shared__ float gs[1024];
  const int dir = blockIdx.x, i = threadIdx.x;
  const int g4 = 4 * h, ld = 8 * h;
  float c = 0.0f;
  if (i < h) hs[i] = 0.0f;
  __syncthreads();
  const float* wcol = whhT + dir * g4 + i;
  for (int64_t step = 0; step < t; ++step) {
    const int64_t tt = dir == 0 ? step : t - 1 - step;
    float acc = g[tt * ld + dir * g4 + i];
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int k = 0;
    for (; k + 4 <= h; k += 4) {
      a0 += wcol[(k + 0) * ld] * hs[k + 0];
      a1 += wcol[(k + 1) * ld] * hs[k + 1];
      a2 += wcol[(k + 2) * ld] * hs[k + 2];
      a3 += wcol[(k + 3) * ld] * hs[k + 3];
    }
    for (; k < h; ++k) a0 += wcol[k * ld] * hs[k];
    acc += (a0 + a1) + (a2 + a3);
    gs[i] = acc;
    __syncthreads();
    if (i < h) {
      const float ig = sigmoidf(gs[i]), fg = sigmoidf(gs[h + i]);
      const float gg = tanhf(gs[2 * h + i]), og = sigmoidf(gs[3 * h + i]);
      c = fg * c + ig * gg;
      const float hv = og * tanhf(c);
      hs[i] = hv;
      out[tt * 2 * h + dir * h + i] = hv;
    }
    __syncthreads();
  }
}

// Persistent LSTM recurrence: 16 workgroups per direction, each owning 16 hidden units, i.e. 64 gate rows of
// W_hh held in registers for the whole sequence. Wave w of a workgroup owns k = KW w .. KW w + KW - 1 (KW = H /
// kLstmWaves) and lane r the gate row r = gate * 16 + unit, so a lane keeps KW weights and the wave needs only the
// KW values of h(t-1) that its own lanes polled: they pass through a wave-private LDS slice (no workgroup barrier
// before the dot products). The waves' partial sums meet at one barrier; then wave 0 applies one activation per
// lane (its gate row), gathers the four gates of each unit into row 0 with permlane swaps, updates the cell and
// publishes h(t) as 64-bit words {tag = step + 1, value} (single 8-byte stores, see storeWord). Every wave then polls its
// KW words of h(t) until the tags match. No fences, no counters: the tag orders each value on its own. The gate
// pre-activations of the next step are loaded while wave 0 polls.
// The words are double-buffered by step parity: a writer can be one step ahead of a reader (it only needs the
// reader's h of the current step, which the reader publishes before it gathers), so with a single buffer its
// step s+1 word could replace the step s word the reader has not read yet. With two buffers the step s+1 word
// replaces the step s-1 word, and every reader is past step s-1 once the writer holds all h(s).
// The exchange words are cleared by a fill kernel before every launch. Every poll is bounded: after
// kLstmSpinLimit polls the lane stops, writes NaN (which every later h inherits) and records the step in the GPU's
// error record (LK_DEVERR_EXCHANGE_TIMEOUT), so a missing peer (e.g. not co-resident) ends the kernel instead of
// hanging it, and the host reports it at the next synchronisation.
constexpr int kLstmWgs = 16;         // workgroups per direction
constexpr int kLstmUnits = 16;       // hidden units per workgroup (H = 256)
// waves per workgroup, each over H / kLstmWaves of k: 8 waves of 32 k run a step in 1.18 us, 4 of 64 k in 1.23 us,
// 16 of 16 k in 1.23 us (the 16-partial sum and the wider barrier cost what the shorter dot products save)
constexpr int kLstmWaves = 8;
constexpr int kLstmThreads = 64 * kLstmWaves;
constexpr long long kLstmSpinLimit = 1LL << 22;

__global__ void lstmClearKernel(unsigned long long* xbuf, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) xbuf[i] = 0ull;
}

// Row r (lanes 16 r .. 16 r + 15) of a wave holds gate r of 16 units; returns in row 0 the four gates of each
// unit. v_permlane16_swap(v, v) exchanges the odd rows of its first operand with the even rows of its second, so
// its second result holds rows {1, 1, 3, 3}; v_permlane32_swap(v, v) exchanges the halves the same way, its second
// result holding rows {2, 3, 2, 3}. Three VALU ops instead of LDS permutes.
__device__ __forceinline__ void gatherGates(float v, float& i, float& f, float& g, float& o) {
  const unsigned u = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const auto p32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const auto p3 = __builtin_amdgcn_permlane16_swap(p32[1], p32[1], false, false);
  i = v;
  f = __uint_as_float(p16[1]);
  g = __uint_as_float(p32[1]);
  o = __uint_as_float(p3[1]);
}

// Up to two independent LSTMs of the same length in one launch (2 kLstmWgs workgroups each): the Kokoro text
// encoder's BiLSTM runs beside the duration encoder's first one instead of as a launch of its own.
struct LstmJobs {
  const float* g[2];
  const float* whhT[2];
  float* out[2];
  unsigned long long* xbuf[2];
};

// Exchange word I/O. kXcd: every workgroup of a direction runs on one XCD, so the words meet in that XCD's L2.
// A non-temporal (nt) load does not allocate in, or hit, the CU's vector cache and is served by the L2 that the
// writer's store wrote through to; a plain or sc0 load can keep returning a stale vector-cache line. Measured
// round trip between two workgroups of one XCD: 0.55 us with nt words against 1.06 us with the agent-scope (sc1)
// accesses of kXcd = false, which stay coherent across XCDs (1.42 us between two XCDs; nt words are not).
template <bool kXcd>
__device__ __forceinline__ unsigned long long loadWord(const unsigned long long* p) {
  if constexpr (kXcd) {
    unsigned long long w;
    asm volatile("global_load_dwordx2 %0, %1, off nt\n\ts_waitcnt vmcnt(0)" : "=v"(w) : "v"(p) : "memory");
    return w;
  } else {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
template <bool kXcd>
__device__ __forceinline__ void storeWord(unsigned long long* p, unsigned long long w) {
  if constexpr (kXcd) asm volatile("global_store_dwordx2 %0, %1, off nt" : : "v"(p), "v"(w) : "memory");
  else __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kXcds = 8;              // XCDs of an MI355X
constexpr int kLstmXcdSlots = 32;     // workgroups launched per XCD and direction team (16 claim a unit slice)
constexpr int kLstmXbufWords = 4 * 256 + 24;  // [direction][parity][256] exchange words + team formation words

// kXcd = false: workgroup bid = blockIdx.x % (2 kLstmWgs) of job blockIdx.x / (2 kLstmWgs); the words live
// wherever the workgroups run. kXcd = true: a direction team is kLstmWgs workgroups of one XCD (read from the
// XCC_ID hardware register). Dispatch deals workgroups to the XCDs round robin from wherever the previous
// dispatch stopped, so the mapping is formed at run time: the first workgroup to arrive on an XCD takes the next
// team ticket (job = ticket / 2, direction = ticket % 2) and publishes it, the next kLstmWgs - 1 read it and take
// unit slices 1.., and every later arrival (or one whose XCD drew a ticket beyond the teams) exits. The grid
// launches kLstmXcdSlots workgroups per XCD, so every XCD that draws a ticket also receives its kLstmWgs members.
template <bool kXcd>
__global__ __launch_bounds__(kLstmThreads) void lstmPersistentKernel(LstmJobs jobs, unsigned long long* err,
                                                                    int64_t t, int teams) {
  constexpr int H = 256;
  constexpr int KW = H / kLstmWaves;  // k per wave
  __shared__ float4 hsw[kLstmWaves][KW / 4];  // wave w: h(t-1)[KW w .. KW w + KW - 1]
  // wave w's partial dot product of each gate row, double-buffered by step parity: a wave w >= 1 may finish step
  // s (it polls other workgroups' words only) and write step s + 1's partials before wave 0 has read step s's
  __shared__ float part[2][kLstmWaves][64];
  int job, dir, b;
  if constexpr (kXcd) {
    __shared__ int claim[2];
    unsigned long long* ctl = jobs.xbuf[0] + 4 * H;  // [0, 8): per-XCD arrivals, [8]: tickets, [16, 24): team + 1
    if (threadIdx.x == 0) {
      const int xcc = static_cast<int>(__builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11))) & 7;
      const int slot = static_cast<int>(
          __hip_atomic_fetch_add(ctl + xcc, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      int team = teams;  // none
      if (slot == 0) {
        team = static_cast<int>(__hip_atomic_fetch_add(ctl + 8, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        __hip_atomic_store(ctl + 16 + xcc, static_cast<unsigned long long>(team) + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      } else if (slot < kLstmWgs) {
        unsigned long long v = 0;
        for (long long spins = 0; (v = __hip_atomic_load(ctl + 16 + xcc, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)) == 0;)
          if (++spins > kLstmSpinLimit) {
            lkd::raiseDeviceError(err, LK_DEVERR_EXCHANGE_TIMEOUT, -1);
            break;
          }
        if (v) team = static_cast<int>(v - 1);
      }
      claim[0] = slot;
      claim[1] = team;
    }
    __syncthreads();
    if (claim[0] >= kLstmWgs || claim[1] >= teams) return;
    job = claim[1] / 2;
    dir = claim[1] % 2;
    b = claim[0];
  } else {
    job = blockIdx.x / (2 * kLstmWgs);
    const int bid = blockIdx.x % (2 * kLstmWgs);
    dir = bid / kLstmWgs;
    b = bid % kLstmWgs;
  }
  const float* __restrict__ g = jobs.g[job];
  const float* __restrict__ whhT = jobs.whhT[job];
  float* __restrict__ out = jobs.out[job];
  unsigned long long* xbuf = jobs.xbuf[job];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ld = 8 * H;
  const int gate = lane >> 4, unit = lane & 15;
  const int64_t col = dir * 4 * H + gate * H + b * kLstmUnits + unit;  // this lane's gate row in g / W_hh^T
  float w[KW];
#pragma unroll
  for (int i = 0; i < KW; ++i) w[i] = whhT[static_cast<int64_t>(KW * wave + i) * ld + col];
  // every weight in registers before the loop (the empty asm redefines each one), so the step's products carry
  // no per-load waits
#pragma unroll
  for (int i = 0; i < KW; ++i) asm volatile("" : "+v"(w[i]));
  reinterpret_cast<float*>(hsw[wave])[lane % KW] = 0.0f;
  unsigned long long* xdir = xbuf + dir * 2 * H;  // [parity][H]
  float c = 0.0f;
  bool ok = true;
  float gv = 0.0f;  // wave 0: this lane's gate pre-activation for the current step
  if (wave == 0) gv = g[(dir == 0 ? 0 : t - 1) * ld + col];
  for (int64_t step = 0; step < t; ++step) {
    const int64_t tt = dir == 0 ? step : t - 1 - step;
    float gnx = 0.0f;  // wave 0: the next step's pre-activation, loaded a whole dot product before the poll
    if (wave == 0 && step + 1 < t) gnx = g[(dir == 0 ? step + 1 : t - 2 - step) * ld + col];
    __builtin_amdgcn_wave_barrier();
    // all 16 broadcast reads in flight before the first product
    float4 hv[KW / 4];
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) hv[i] = hsw[wave][i];
    __builtin_amdgcn_sched_barrier(0);
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) {
      const float4 h = hv[i];
      a0 = fmaf(w[4 * i], h.x, a0);
      a1 = fmaf(w[4 * i + 1], h.y, a1);
      a2 = fmaf(w[4 * i + 2], h.z, a2);
      a3 = fmaf(w[4 * i + 3], h.w, a3);
    }
    part[step & 1][wave][lane] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    const unsigned tag = static_cast<unsigned>(step + 1);
    unsigned long long* xb = xdir + (step & 1) * H;
    if (wave == 0) {
      float pv[kLstmWaves];  // the waves' partials summed as a pairwise tree: ((p0 + p1) + (p2 + p3)) + ...
#pragma unroll
      for (int i = 0; i < kLstmWaves; ++i) pv[i] = part[step & 1][i][lane];
#pragma unroll
      for (int n = kLstmWaves; n > 1; n /= 2)
#pragma unroll
        for (int i = 0; i < n / 2; ++i) pv[i] = pv[2 * i] + pv[2 * i + 1];
      const float x = gv + pv[0];
      const float sg = sigmoidHw(gate == 2 ? 2.0f * x : x);
      const float act = gate == 2 ? fmaf(2.0f, sg, -1.0f) : sg;
      float ig, fg, gg, og;
      gatherGates(act, ig, fg, gg, og);
      if (lane < kLstmUnits) {
        c = fg * c + ig * gg;
        const float hv = ok ? og * tanhHw(c) : __builtin_nanf("");
        const unsigned long long word = (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(hv);
        storeWord<kXcd>(xb + b * kLstmUnits + lane, word);
        out[tt * 2 * H + dir * H + b * kLstmUnits + lane] = hv;
      }
    }
    // gather this wave's KW values of h(t): lane polls word KW w + lane % KW (with KW = 32 both wave halves poll
    // the same words and store the same values)
    {
      unsigned long long word = 0ull;
      long long spins = 0;
      while (ok) {
        word = loadWord<kXcd>(xb + KW * wave + lane % KW);
        if (static_cast<unsigned>(word >> 32) == tag) break;
        if (++spins > kLstmSpinLimit) {
          ok = false;
          lkd::raiseDeviceError(err, LK_DEVERR_EXCHANGE_TIMEOUT, step);
        }
      }
      // A lane that timed out keeps stepping (so every wave reaches the end) but stops waiting; its NaN
      // reaches every gate row through the next step's dot products.
      reinterpret_cast<float*>(hsw[wave])[lane % KW] =
          ok ? __uint_as_float(static_cast<unsigned>(word & 0xffffffffull)) : __builtin_nanf("");
    }
    gv = gnx;
  }
}

// The XCD-local exchange needs all eight XCDs of an MI355X in one device (256 CUs, SPX mode); LK_LSTM_EXCHANGE=agent
// selects the agent-scope exchange anyway (the two give identical bits: only the words' cache path differs).
inline bool lstmXcdLocal() {
  const char* e = getenv("LK_LSTM_EXCHANGE");
  if (e && strcmp(e, "agent") == 0) return false;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  static std::atomic<int> cached[64] = {};  // per device: 0 unknown, 1 XCD-local, 2 agent
  if (dev >= 0 && dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c) return c == 1;
  }
  const bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                  cus == kXcds * 32;
  if (dev >= 0 && dev < 64) cached[dev].store(ok ? 1 : 2, std::memory_order_relaxed);
  return ok;
}

inline void launchLstm(const LstmJobs& jobs, int njobs, int64_t t, hipStream_t s) {
  if (lstmXcdLocal())
    hipLaunchKernelGGL(lstmPersistentKernel<true>, dim3(kXcds * kLstmXcdSlots), dim3(kLstmThreads), 0, s, jobs,
                       lkh::deviceErrorRecord(), t, 2 * njobs);
  else
    hipLaunchKernelGGL(lstmPersistentKernel<false>, dim3(2 * njobs * kLstmWgs), dim3(kLstmThreads), 0, s, jobs,
                       lkh::deviceErrorRecord(), t, 2 * njobs);
}

// Each workgroup scans dur (T <= 8192) into LDS, then gathers its rows: row f copies x[token(f)], token(f) =
// the first i with cum[i] > f.
__global__ __launch_bounds__(256) void repeatInterleaveKernel(const float* __restrict__ x,
                                                             const int64_t* __restrict__ dur, float* __restrict__ out,
                                                             int64_t t, int64_t c, int64_t frames,
                                                             unsigned long long* err) {
  __shared__ int64_t cum[8192];
  __shared__ int64_t part[256];
  const int tid = threadIdx.x;
  const int64_t per = (t + 255) / 256;
  int64_t s = 0;
  for (int64_t i = tid * per; i < min<int64_t>(t, (tid + 1) * per); ++i) s += dur[i] > 0 ? dur[i] : 0;
  part[tid] = s;
  __syncthreads();
  if (tid == 0)
    for (int j = 1; j < 256; ++j) part[j] += part[j - 1];
  __syncthreads();
  int64_t run = tid == 0 ? 0 : part[tid - 1];
  for (int64_t i = tid * per; i < min<int64_t>(t, (tid + 1) * per); ++i) {
    run += dur[i] > 0 ? dur[i] : 0;
    cum[i] = run;
  }
  __syncthreads();
  const int64_t rowsPerBlock = (frames + gridDim.x - 1) / gridDim.x;
  const int64_t r0 = blockIdx.x * rowsPerBlock, r1 = min<int64_t>(frames, r0 + rowsPerBlock);
  for (int64_t f = r0; f < r1; ++f) {
    int64_t lo = 0, hi = t;  // first i with cum[i] > f
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (cum[mid] > f) hi = mid;
      else lo = mid + 1;
    }
    const bool ok = lo < t;
    if (!ok && tid == 0) raiseDeviceError(err, LK_DEVERR_DURATIONS, f);
    for (int64_t j = tid; j < c; j += 256) out[f * c + j] = ok ? x[lo * c + j] : __builtin_nanf("");
  }
}

__device__ __forceinline__ float blockSum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = waveSum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// (1 + gb[c]) * (x - mean) / sqrt(var + eps) + gb[C + c]; one 256-thread workgroup per row, C <= 2048.
__global__ __launch_bounds__(256) void adaLayerNormKernel(const float* __restrict__ x, const float* __restrict__ gb,
                                                         float* __restrict__ out, int64_t c, float eps) {
  __shared__ float scratch[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * c;
  float v[8];
  float s = 0.0f;
  int n = 0;
  for (int64_t j = threadIdx.x; j < c; j += 256, ++n) {
    v[n] = x[base + j];
    s += v[n];
  }
  const float mean = blockSum(s, scratch) / static_cast<float>(c);
  float q = 0.0f;
  for (int i = 0; i < n; ++i) q += (v[i] - mean) * (v[i] - mean);
  const float rstd = 1.0f / sqrtf(blockSum(q, scratch) / static_cast<float>(c) + eps);
  n = 0;
  for (int64_t j = threadIdx.x; j < c; j += 256, ++n)
    out[base + j] = (1.0f + gb[j]) * ((v[n] - mean) * rstd) + gb[c + j];
}

__global__ void concatBcastKernel(const float* __restrict__ x, const float* __restrict__ v, float* __restrict__ out,
                                  int64_t r, int64_t c1, int64_t c2) {
  const int64_t cw = c1 + c2, n = r * cw;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / cw, col = i - row * cw;
    out[i] = col < c1 ? x[row * c1 + col] : v[col - c1];
  }
}

}  // namespace lkd

extern "C" {

// x [T, I], w_ih [8H, I], w_hh_t [H, 8H], b [8H] -> out [T, 2H]; gates workspace: T * 8H floats.
int lk_hip_lstm_bidir_f32(const float* x, const float* wih, const float* whhT, const float* b, float* out, int64_t t,
                          int64_t in, int64_t h, void* workspace, int64_t workspaceBytes, void* stream) {
  if (h < 1 || h > 256 || t < 1) return 1;
  if (!workspace || workspaceBytes < t * 8 * h * 4) return 3;
  float* g = static_cast<float*>(workspace);
  int rc = lk_hip_gemm_f32(x, wih, b, nullptr, g, t, 8 * h, in, 1, 0, 1.0f, nullptr, 0, stream);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t gBytes = ((t * 8 * h * 4 + 255) / 256) * 256;
  const int64_t xBytes = lkd::kLstmXbufWords * 8;
  if (h == 256 && workspaceBytes >= gBytes + xBytes) {
    auto* xbuf = reinterpret_cast<unsigned long long*>(static_cast<char*>(workspace) + gBytes);
    hipLaunchKernelGGL(lkd::lstmClearKernel, dim3(5), dim3(256), 0, s, xbuf, lkd::kLstmXbufWords);
    const lkd::LstmJobs jobs{{g, g}, {whhT, whhT}, {out, out}, {xbuf, xbuf}};
    lkd::launchLstm(jobs, 1, t, s);
  } else {
    hipLaunchKernelGGL(lkd::lstmRecurrenceKernel, dim3(2), dim3(static_cast<unsigned>(4 * h)), 0, s, g, whhT, out,
                       t, static_cast<int>(h));
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Two bidirectional LSTMs of the same length T and H = 256 in one recurrence launch (4 x 16 workgroups); each
// one's arithmetic is lk_hip_lstm_bidir_f32's. Workspace: two gate planes and two exchange buffers.
int lk_hip_lstm_bidir2_f32(const float* x1, const float* wih1, const float* whhT1, const float* b1, float* out1,
                           int64_t in1, const float* x2, const float* wih2, const float* whhT2, const float* b2,
                           float* out2, int64_t in2, int64_t t, int64_t h, void* workspace, int64_t workspaceBytes,
                           void* stream) {
  if (h != 256 || t < 1) return 1;
  const int64_t gBytes = ((t * 8 * h * 4 + 255) / 256) * 256;
  const int64_t xBytes = lkd::kLstmXbufWords * 8;
  if (!workspace || workspaceBytes < 2 * gBytes + 2 * xBytes) return 3;
  char* ws = static_cast<char*>(workspace);
  float* g1 = reinterpret_cast<float*>(ws);
  float* g2 = reinterpret_cast<float*>(ws + gBytes);
  auto* xb1 = reinterpret_cast<unsigned long long*>(ws + 2 * gBytes);
  auto* xb2 = reinterpret_cast<unsigned long long*>(ws + 2 * gBytes + xBytes);
  int rc = lk_hip_gemm_f32(x1, wih1, b1, nullptr, g1, t, 8 * h, in1, 1, 0, 1.0f, nullptr, 0, stream);
  if (!rc) rc = lk_hip_gemm_f32(x2, wih2, b2, nullptr, g2, t, 8 * h, in2, 1, 0, 1.0f, nullptr, 0, stream);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(lkd::lstmClearKernel, dim3(9), dim3(256), 0, s, xb1, 2 * lkd::kLstmXbufWords);  // adjacent
  const lkd::LstmJobs jobs{{g1, g2}, {whhT1, whhT2}, {out1, out2}, {xb1, xb2}};
  lkd::launchLstm(jobs, 2, t, s);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_repeat_interleave_f32(const float* x, const int64_t* dur, float* out, int64_t t, int64_t c, int64_t frames,
                                 void* stream) {
  if (t < 1 || t > 8192 || frames < 0) return 1;
  if (frames == 0) return 0;
  const int64_t blocks = std::min<int64_t>(frames, 1024);
  hipLaunchKernelGGL(lkd::repeatInterleaveKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, dur, out, t, c, frames, lkh::deviceErrorRecord());
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_adalayernorm_f32(const float* x, const float* gb, float* out, int64_t r, int64_t c, float eps,
                            void* stream) {
  if (c < 1 || c > 2048 || r < 1) return 1;
  hipLaunchKernelGGL(lkd::adaLayerNormKernel, dim3(static_cast<unsigned>(r)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, gb, out, c, eps);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int lk_hip_concat_bcast_f32(const float* x, const float* v, float* out, int64_t r, int64_t c1, int64_t c2,
                            void* stream) {
  const int64_t n = r * (c1 + c2);
  if (n <= 0) return n == 0 ? 0 : 1;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(lkd::concatBcastKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, v, out, r, c1, c2);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

namespace lkh {

namespace {

// lstm2_bidir_t_f32_gpu(x1[T, I1], w_ih1[8H, I1], w_hh_t1[H, 8H], b1[8H], x2[T, I2], w_ih2[8H, I2],
//   w_hh_t2[H, 8H], b2[8H]) -> ([T, 2H], [T, 2H]) (MI355X backend: two lstm_bidir_t in one recurrence launch)
void runLstm2(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t t = a.ints[0], in1 = a.ints[1], h = a.ints[4], in2 = a.ints[8];
  LK_REQUIRE(ctx,
             a.ints[2] == 8 * h && a.ints[3] == in1 && a.ints[5] == 8 * h && a.ints[6] == 8 * h && a.ints[7] == t &&
                 a.ints[9] == 8 * h && a.ints[10] == in2 && a.ints[11] == h && a.ints[12] == 8 * h &&
                 a.ints[13] == 8 * h,
             "lstm2_bidir_t: expected two lstm_bidir_t operand sets of one length and hidden size");
  const int rc = lk_hip_lstm_bidir2_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), P<float>(a, 8),
                                        in1, P<float>(a, 4), P<float>(a, 5), P<float>(a, 6), P<float>(a, 7),
                                        P<float>(a, 9), in2, t, h, ctx.workspace,
                                        static_cast<int64_t>(ctx.workspaceBytes), ctx.stream);
  if (rc) ctx.error = rc == 3 ? "lstm2_bidir_t: workspace too small" : "lstm2_bidir_t: H must be 256, or launch failed";
}

// lstm_bidir_t_f32_gpu(x[T, I], w_ih[8H, I], w_hh_t[H, 8H], b[8H]) -> [T, 2H]
void runLstm(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t t = a.ints[0], in = a.ints[1];
  const int64_t h = a.ints[4];
  LK_REQUIRE(ctx, a.ints[2] == 8 * h && a.ints[3] == in && a.ints[5] == 8 * h && a.ints[6] == 8 * h,
             "lstm_bidir_t: expected w_ih [8H, I], w_hh_t [H, 8H], b [8H]");
  const int rc = lk_hip_lstm_bidir_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), P<float>(a, 3), P<float>(a, 4),
                                       t, in, h, ctx.workspace, static_cast<int64_t>(ctx.workspaceBytes), ctx.stream);
  if (rc) ctx.error = rc == 3 ? "lstm_bidir_t: workspace too small for the gate pre-activations" : "lstm: failed";
}

// repeat_interleave_f32_gpu(x[T, C], dur i64[T]; frames) -> [frames, C]
void runRepeatInterleave(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t t = a.ints[0], c = a.ints[1], frames = a.ints[3];
  if (lk_hip_repeat_interleave_f32(P<float>(a, 0), P<int64_t>(a, 1), P<float>(a, 2), t, c, frames, ctx.stream))
    ctx.error = "repeat_interleave: T must be in 1..8192";
}

// adalayernorm_f32_gpu(x[R, C], gb[2C]; eps) -> [R, C]
void runAdaLn(ExecCtx& ctx, const KernelArgs& a) {
  const int64_t r = a.ints[0], c = a.ints[1];
  LK_REQUIRE(ctx, a.ints[2] == 2 * c, "adalayernorm: gb must be f32[2C]");
  if (lk_hip_adalayernorm_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), r, c,
                              static_cast<float>(a.numFloats ? a.floats[0] : 1e-5), ctx.stream))
    ctx.error = "adalayernorm: C must be <= 2048";
}

// concat_bcast_f32_gpu(x[R, C1], v[C2]) -> [R, C1 + C2]
void runConcatBcast(ExecCtx& ctx, const KernelArgs& a) {
  if (lk_hip_concat_bcast_f32(P<float>(a, 0), P<float>(a, 1), P<float>(a, 2), a.ints[0], a.ints[1], a.ints[2],
                              ctx.stream))
    ctx.error = "concat_bcast: failed";
}

}  // namespace

void registerSequenceKernels() {
  const Device G = Device::Gpu;
  registerKernel({"lstm_bidir_t_f32_gpu", G, runLstm, 4, 1});
  registerKernel({"lstm2_bidir_t_f32_gpu", G, runLstm2, 8, 2});
  registerKernel({"repeat_interleave_f32_gpu", G, runRepeatInterleave, 2, 1});
  registerKernel({"adalayernorm_f32_gpu", G, runAdaLn, 2, 1});
  registerKernel({"concat_bcast_f32_gpu", G, runConcatBcast, 2, 1});
}

}  // namespace lkh
