// Bandwidth-bound decode attention with the KV write fused (reference attention_decode_split_f32_gpu /
// attention_decode_kvw_f32_gpu, transformer_gpu.cpp:122-222, kokoro_tok.metal:637-876 in lariaus/lokinfer).
//
// One query (heads x 64) attends over cache rows 0..pos; row pos is k, v (+ bias) of this step and is written
// into both caches. Keys are split into 64-key chunks, one wave per (head, chunk) (DecodeChunk: coalesced row
// loads, DPP row sums for the scores, softmax of q / 8 = q / sqrt(64) in log2 units, P.V in registers). Partials
// (m, l, acc[64]) go to the caller's workspace; a second launch merges the chunks of each head in chunk order
// (flash-decoding).
#include "common.h"
#include "decode_chunk.h"
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
  int chunks;  // partials per head: waves per head
  int sub;     // 64-key chunks per wave
  int writeKv;
  unsigned long long* err;  // the GPU's error record
};

__global__ __launch_bounds__(64) void decodeChunkKernel(DecodeParams p) {
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int64_t D = static_cast<int64_t>(p.heads) * kHd;
  const int64_t c4 = h * kHd + 4 * (lane & 15);  // this lane's 4 dims in a row of q, k or v
  const float4 q4 = *reinterpret_cast<const float4*>(p.qkv + c4);
  const float4 k4 = *reinterpret_cast<const float4*>(p.qkv + D + c4);
  const float4 v4 = *reinterpret_cast<const float4*>(p.qkv + 2 * D + c4);
  const float4 bq = *reinterpret_cast<const float4*>(p.bias + c4);
  const float4 bk = *reinterpret_cast<const float4*>(p.bias + D + c4);
  const float4 bv = *reinterpret_cast<const float4*>(p.bias + 2 * D + c4);
  const int64_t pos = *p.pos;
  DecodeChunk ch;
  ch.load<true>(p.kc, p.vc, pos, p.cap, s * p.sub, D, c4);
  // an out-of-range position writes no cache row and NaN partials, and is recorded; the merge writes NaN
  if (ch.badPos && h == 0 && s == 0 && lane == 0) raiseDeviceError(p.err, LK_DEVERR_POSITION, pos);
  const decF4 q = decF4{q4.x + bq.x, q4.y + bq.y, q4.z + bq.z, q4.w + bq.w} * (0.125f * kLog2e);
  const decF4 knew = {k4.x + bk.x, k4.y + bk.y, k4.z + bk.z, k4.w + bk.w};
  const decF4 vnew = {v4.x + bv.x, v4.y + bv.y, v4.z + bv.z, v4.w + bv.w};
  if (p.writeKv && ch.writesRow()) {
    *reinterpret_cast<decF4*>(p.kc + pos * D + c4) = knew;
    *reinterpret_cast<decF4*>(p.vc + pos * D + c4) = vnew;
  }
  DecodeChunk::Result r = ch.compute(q, knew, vnew);
  // a long cache: this wave also takes the next sub - 1 64-key chunks, combined online (stops at pos)
  for (int j = 1; j < p.sub && !ch.badPos && static_cast<int64_t>(s * p.sub + j) * kChunk <= pos; ++j) {
    DecodeChunk nx;
    nx.load<true>(p.kc, p.vc, pos, p.cap, s * p.sub + j, D, c4);
    if (p.writeKv && nx.writesRow()) {
      *reinterpret_cast<decF4*>(p.kc + pos * D + c4) = knew;
      *reinterpret_cast<decF4*>(p.vc + pos * D + c4) = vnew;
    }
    r = DecodeChunk::combine(r, nx.compute(q, knew, vnew));
  }
  ch.store(r, p.partial + (static_cast<int64_t>(h) * p.chunks + s) * (kHd + 2));
}

// Merge of one head's chunks (one workgroup of 16 waves per head), one pass: wave w takes chunks w, w + 16, ... in
// order, 8 chunks' loads at a time, keeping a running max M_w (log2 units) and sums rescaled to it,
// L_w = sum_c 2^{m_c - M_w} l_c, A_w[d] = sum_c 2^{m_c - M_w} acc_c[d]; then out[d] = sum_w 2^{M_w - M} A_w[d] /
// sum_w 2^{M_w - M} L_w with M = max M_w, the 16 waves in order. A long cache (128 chunks per head) costs one
// memory round trip.
constexpr int kMergeWaves = 16, kMergeBatch = 8;
__global__ __launch_bounds__(64 * kMergeWaves) void decodeMergeKernel(const float* __restrict__ partial,
                                                                      float* __restrict__ out, const int64_t* pos,
                                                                      int64_t cap, int chunks) {
  __shared__ float red[kMergeWaves][kHd];
  __shared__ float sM[kMergeWaves], sL[kMergeWaves];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t ps = *pos;
  if (ps < 0 || ps >= cap) {
    if (wv == 0) out[h * kHd + lane] = __builtin_nanf("");
    return;
  }
  const float* base = partial + static_cast<int64_t>(h) * chunks * (kHd + 2);
  float M = -INFINITY, a = 0.0f, l = 0.0f;  // M is the same in every lane of the wave (m, l are per chunk)
  for (int c0 = wv; c0 < chunks; c0 += kMergeWaves * kMergeBatch) {
    float mc[kMergeBatch], lc[kMergeBatch], ac[kMergeBatch];
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const int c = min(c0 + kMergeWaves * i, chunks - 1);
      mc[i] = base[c * (kHd + 2)];
      lc[i] = base[c * (kHd + 2) + 1];
      ac[i] = base[c * (kHd + 2) + 2 + lane];
    }
    float bm = M;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i)
      if (c0 + kMergeWaves * i < chunks && lc[i] > 0.0f) bm = fmaxf(bm, mc[i]);
    if (bm > M) {  // rescale the running sums to the new max
      const float r = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - bm);
      a *= r;
      l *= r;
      M = bm;
    }
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      if (c0 + kMergeWaves * i < chunks && lc[i] > 0.0f) {
        const float w = __builtin_amdgcn_exp2f(mc[i] - M);
        l += w * lc[i];
        a += w * ac[i];
      }
    }
  }
  red[wv][lane] = a;
  if (lane == 0) {
    sM[wv] = M;
    sL[wv] = l;
  }
  __syncthreads();
  if (wv == 0) {
    float Mx = sM[0];
#pragma unroll
    for (int w = 1; w < kMergeWaves; ++w) Mx = fmaxf(Mx, sM[w]);
    float A = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kMergeWaves; ++w) {
      const float r = sL[w] > 0.0f ? __builtin_amdgcn_exp2f(sM[w] - Mx) : 0.0f;
      A += r * red[w][lane];
      L += r * sL[w];
    }
    out[h * kHd + lane] = A / L;
  }
}

// Waves per head and 64-key chunks per wave for `keys` keys: one chunk per wave up to 128 chunks, beyond that
// as many chunks per wave as keep the waves (and the partials the merge reads) at 128 or fewer per head.
constexpr int64_t kMaxWavesPerHead = 128;
inline void decodeSplit(int64_t keys, int* waves, int* sub) {
  const int64_t c = (keys + kChunk - 1) / kChunk;
  const int64_t sb = c > kMaxWavesPerHead ? (c + kMaxWavesPerHead - 1) / kMaxWavesPerHead : 1;
  *sub = static_cast<int>(sb);
  *waves = static_cast<int>((c + sb - 1) / sb);
}

}  // namespace lkd

extern "C" {

int64_t lk_hip_attention_decode_workspace_bytes(int heads, int64_t cap) {
  int waves = 0, sub = 0;
  lkd::decodeSplit(cap, &waves, &sub);
  return static_cast<int64_t>(heads) * waves * (lkd::kHd + 2) * 4;
}

// qkv [1, 3D] (before bias), kc / vc [cap, D] (rows 0..pos-1 valid; row pos written when writeKv), pos device
// i64[1], bias [3D] -> out [1, D], D = 64 heads. The grid covers max_keys (<= cap) keys; chunks past pos store
// empty partials. pos outside [0, cap) writes nothing, yields NaN and is recorded as LK_DEVERR_POSITION.
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
  lkd::decodeSplit(maxKeys, &p.chunks, &p.sub);
  if (!workspace || workspaceBytes < static_cast<int64_t>(heads) * p.chunks * (lkd::kHd + 2) * 4) return 3;
  p.partial = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(lkd::decodeChunkKernel, dim3(static_cast<unsigned>(heads), static_cast<unsigned>(p.chunks)),
                     dim3(64), 0, s, p);
  hipLaunchKernelGGL(lkd::decodeMergeKernel, dim3(static_cast<unsigned>(heads)), dim3(64 * lkd::kMergeWaves), 0, s,
                     p.partial, out, pos, cap, p.chunks);
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

constexpr int64_t kNoAllocScratchFloats = 512 * 1024;  // 2 MiB: heads x (waves per head) x 66 floats
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
  int waves = 0, sub = 0;
  lkd::decodeSplit(keys, &waves, &sub);
  const int64_t need = static_cast<int64_t>(heads) * waves * (lkd::kHd + 2);
  if (need > kNoAllocScratchFloats) return 4;  // beyond the fixed scratch array
  float* ptr = scratchOnCurrentDevice();
  if (!ptr) return 2;
  return lk_hip_attention_decode_f32(qkv, kc, vc, pos, bias, out, cap, heads, maxKeys, writeKv, ptr,
                                     kNoAllocScratchFloats * 4, stream);
}

}  // extern "C"
