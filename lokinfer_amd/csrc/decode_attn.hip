// Bandwidth-bound decode attention with the KV write fused (reference attention_decode_split_f32_gpu /
// attention_decode_kvw_f32_gpu, transformer_gpu.cpp:122-222, kokoro_tok.metal:637-876 in lariaus/lokinfer).
//
// One query (heads x 64) attends over cache rows 0..pos; row pos is k, v (+ bias) of this step and is written
// into both caches. Keys are split into 64-key chunks, one wave per (head, chunk):
//   scores  lane j owns key kb + j: a 64-float dot with q (16 independent float4 loads per lane)
//   softmax chunk max / sum with wave64 shuffles (base-e, q pre-scaled by 1/8 = 1/sqrt(64))
//   P.V     lane = (key group g in 0..3, dim quad d4 in 0..15): 16 keys per lane as float4 loads, then a 2-step
//           shuffle reduction over g
// Partials (m, l, acc[64]) go to the caller's workspace; a second launch merges the chunks of each head in
// chunk order (flash-decoding). Every load of a chunk is issued before its first use, so a wave waits on HBM
// twice (K rows, V rows) instead of once per key.
#include "common.h"
#include "lokinfer_hip.h"

#include <mutex>

namespace lkd {

constexpr int kHd = 64;
constexpr int kChunk = 64;

struct DecodeParams {
  const float* qkv;
  float* kc;
  float* vc;
  const int64_t* pos;
  const float* bias;
  float* out;
  float* partial;  // [heads, chunks, 66]
  int64_t cap;
  int heads;
  int chunks;
  int writeKv;
  unsigned long long* err;  // the GPU's error record
};

__global__ __launch_bounds__(64) void decodeChunkKernel(DecodeParams p) {
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int64_t D = static_cast<int64_t>(p.heads) * kHd;
  const int64_t pos = *p.pos;
  if (pos < 0 || pos >= p.cap) {  // out-of-range position: no cache write, recorded; the merge writes NaN
    if (h == 0 && s == 0 && lane == 0) raiseDeviceError(p.err, LK_DEVERR_POSITION, pos);
    return;
  }
  const int64_t kb = static_cast<int64_t>(s) * kChunk;
  const int64_t ke = min<int64_t>(pos + 1, kb + kChunk);
  float* part = p.partial + (static_cast<int64_t>(h) * p.chunks + s) * (kHd + 2);
  const float* qrow = p.qkv + h * kHd;
  const float* bq = p.bias + h * kHd;
  const float* bk = p.bias + D + h * kHd;
  const float* bv = p.bias + 2 * D + h * kHd;
  if (kb >= ke) {  // chunk past the live keys
    if (lane == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    part[2 + lane] = 0.0f;
    return;
  }
  const float knew = p.qkv[D + h * kHd + lane] + bk[lane];
  if (p.writeKv && pos >= kb && pos < kb + kChunk) {
    p.kc[pos * D + h * kHd + lane] = knew;
    p.vc[pos * D + h * kHd + lane] = p.qkv[2 * D + h * kHd + lane] + bv[lane];
  }
  const float snew = waveSum((qrow[lane] + bq[lane]) * 0.125f * knew);
  float q[kHd];
#pragma unroll
  for (int d = 0; d < kHd; ++d) q[d] = (qrow[d] + bq[d]) * 0.125f;

  // scores
  const int64_t j = kb + lane;
  float sc = -INFINITY;
  if (j < ke) {
    if (j == pos) {
      sc = snew;
    } else {
      const float4* kr = reinterpret_cast<const float4*>(p.kc + j * D + h * kHd);
      float4 kv[kHd / 4];
#pragma unroll
      for (int d4 = 0; d4 < kHd / 4; ++d4) kv[d4] = kr[d4];
      float dot = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < kHd / 4; ++d4)
        dot += q[4 * d4] * kv[d4].x + q[4 * d4 + 1] * kv[d4].y + q[4 * d4 + 2] * kv[d4].z + q[4 * d4 + 3] * kv[d4].w;
      sc = dot;
    }
  }
  const float m = waveMax(sc);
  const float pj = j < ke ? expf(sc - m) : 0.0f;
  const float l = waveSum(pj);

  // P.V: lane = (g, d4); keys kb + g + 4 i, i = 0..15
  const int g = lane >> 4, d4 = lane & 15;
  float4 vv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = kb + g + 4 * i;
    if (row < ke && row != pos) {
      vv[i] = reinterpret_cast<const float4*>(p.vc + row * D + h * kHd)[d4];
    } else if (row == pos) {
      const float* vq = p.qkv + 2 * D + h * kHd + 4 * d4;
      vv[i] = make_float4(vq[0] + bv[4 * d4], vq[1] + bv[4 * d4 + 1], vq[2] + bv[4 * d4 + 2], vq[3] + bv[4 * d4 + 3]);
    } else {
      vv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float w = __shfl(pj, g + 4 * i, 64);
    acc.x += w * vv[i].x;
    acc.y += w * vv[i].y;
    acc.z += w * vv[i].z;
    acc.w += w * vv[i].w;
  }
#pragma unroll
  for (int o = 16; o < 64; o <<= 1) {
    acc.x += __shfl_xor(acc.x, o, 64);
    acc.y += __shfl_xor(acc.y, o, 64);
    acc.z += __shfl_xor(acc.z, o, 64);
    acc.w += __shfl_xor(acc.w, o, 64);
  }
  if (lane == 0) {
    part[0] = m;
    part[1] = l;
  }
  if (g == 0) reinterpret_cast<float4*>(part + 2)[d4] = acc;
}

// Merge of one head's chunks: lane c holds chunk c's (m, l) (chunks <= 64 per pass, looped beyond),
// M = max m_c, w_c = e^{m_c - M}, out[d] = sum_c w_c acc_c[d] / sum_c w_c l_c, chunks in order.
__global__ __launch_bounds__(64) void decodeMergeKernel(const float* __restrict__ partial, float* __restrict__ out,
                                                        const int64_t* pos, int64_t cap, int chunks) {
  const int h = blockIdx.x, lane = threadIdx.x;
  const int64_t ps = *pos;
  if (ps < 0 || ps >= cap) {
    out[h * kHd + lane] = __builtin_nanf("");
    return;
  }
  const float* base = partial + static_cast<int64_t>(h) * chunks * (kHd + 2);
  float M = -INFINITY;
  for (int c0 = 0; c0 < chunks; c0 += 64) {
    const int c = c0 + lane;
    M = fmaxf(M, waveMax(c < chunks ? base[c * (kHd + 2)] : -INFINITY));
  }
  float L = 0.0f, A = 0.0f;
  for (int c0 = 0; c0 < chunks; c0 += 64) {
    const int c = c0 + lane;
    const float lc = c < chunks ? base[c * (kHd + 2) + 1] : 0.0f;
    const float wc = lc > 0.0f ? expf(base[c * (kHd + 2)] - M) : 0.0f;
    L += waveSum(lc * wc);
    const int n = min(64, chunks - c0);
    for (int i = 0; i < n; ++i) {
      const float w = __shfl(wc, i, 64);
      A += w * base[(c0 + i) * (kHd + 2) + 2 + lane];
    }
  }
  out[h * kHd + lane] = A / L;
}

}  // namespace lkd

extern "C" {

int64_t lk_hip_attention_decode_workspace_bytes(int heads, int64_t cap) {
  const int64_t chunks = (cap + lkd::kChunk - 1) / lkd::kChunk;
  return static_cast<int64_t>(heads) * chunks * (lkd::kHd + 2) * 4;
}

// qkv [1, 3D] (before bias), kc / vc [cap, D] (rows 0..pos-1 valid; row pos written when writeKv), pos device
// i64[1], bias [3D] -> out [1, D], D = 64 heads. The grid covers max_keys (<= cap) keys; chunks past pos exit
// early. pos outside [0, cap) writes nothing, yields NaN and is recorded as LK_DEVERR_POSITION.
int lk_hip_attention_decode_f32(const float* qkv, float* kc, float* vc, const int64_t* pos, const float* bias,
                                float* out, int64_t cap, int heads, int64_t maxKeys, int writeKv, void* workspace,
                                int64_t workspaceBytes, void* stream) {
  if (heads <= 0 || cap <= 0) return 1;
  if (maxKeys <= 0 || maxKeys > cap) maxKeys = cap;
  lkd::DecodeParams p{};
  p.qkv = qkv;
  p.kc = kc;
  p.vc = vc;
  p.pos = pos;
  p.bias = bias;
  p.out = out;
  p.cap = cap;
  p.heads = heads;
  p.writeKv = writeKv;
  p.err = lkh::deviceErrorRecord();
  p.chunks = static_cast<int>((maxKeys + lkd::kChunk - 1) / lkd::kChunk);
  if (!workspace || workspaceBytes < static_cast<int64_t>(heads) * p.chunks * (lkd::kHd + 2) * 4) return 3;
  p.partial = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(lkd::decodeChunkKernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(p.chunks)),
                     dim3(64), 0, s, p);
  hipLaunchKernelGGL(lkd::decodeMergeKernel, dim3(static_cast<unsigned>(heads)), dim3(64), 0, s, p.partial, out, pos,
                     cap, p.chunks);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"

// ---- allocation-free variant --------------------------------------------------------------------------------
// The chunk partials live in a fixed device array instead of a caller workspace, for callers that cannot allocate
// (HIP graph capture of a serving loop, harnesses that forbid hipMalloc). Each GPU holds its own copy of the array
// for the life of the process; its device address is looked up once per device and kept. The merge reads only
// partials the chunk launch of the same call wrote, so nothing needs clearing between calls, but two calls that
// overlap on one GPU (different streams) race on the array.
namespace {

constexpr int64_t kNoAllocScratchFloats = 512 * 1024;  // 2 MiB: heads x ceil(max_keys / 64) x 66 floats
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex gScratchMu;
float* gScratchPtr[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure).
float* scratchOnCurrentDevice() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(gScratchMu);
  if (!gScratchPtr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) {
      (void)hipGetLastError();  // do not leave the failure for a later launch check
      return nullptr;
    }
    gScratchPtr[dev] = static_cast<float*>(ptr);
  }
  return gScratchPtr[dev];
}

}  // namespace

extern "C" {

int64_t lk_hip_attention_decode_noalloc_max_floats(void) { return kNoAllocScratchFloats; }

int lk_hip_attention_decode_f32_noalloc(const float* qkv, float* kc, float* vc, const int64_t* pos, const float* bias,
                                        float* out, int64_t cap, int heads, int64_t maxKeys, int writeKv,
                                        void* stream) {
  if (heads <= 0 || cap <= 0) return 1;
  const int64_t keys = maxKeys <= 0 || maxKeys > cap ? cap : maxKeys;
  const int64_t need = static_cast<int64_t>(heads) * ((keys + lkd::kChunk - 1) / lkd::kChunk) * (lkd::kHd + 2);
  if (need > kNoAllocScratchFloats) return 4;  // beyond the fixed scratch array
  float* ptr = scratchOnCurrentDevice();
  if (!ptr) return 2;
  return lk_hip_attention_decode_f32(qkv, kc, vc, pos, bias, out, cap, heads, maxKeys, writeKv, ptr,
                                     kNoAllocScratchFloats * 4, stream);
}

}  // extern "C"
