// One wave's share of batch-1 decode attention: head h, keys kb .. ke - 1 of a [cap, heads * 64] K / V cache
// (a 64-key chunk), with this step's key / value (row pos) taken from registers instead of the cache. Used by the
// split decode kernel (q, k, v from the qkv row) and by the fused decode-step kernel (q, k, v from GEMV partial
// rows). Scores are in log2 units (the caller scales q by log2(e) / sqrt(64)), so each exponential is one exp2.
//
// Layout: lane (g = lane / 16, d4 = lane % 16) owns dims 4 d4 .. 4 d4 + 3 of keys kb + g + 4 i, i = 0..15, so
// each load instruction reads 4 whole cache rows (coalesced), a score is a 16-lane row sum (DPP), and the softmax
// weights of a lane's keys are already in the lane for P.V. The chunk's rows are loaded unconditionally from rows
// clamped to 0 .. pos (row pos itself and rows past it are replaced by selects and never used), so the loads can
// be issued before the caller waits on anything else; a chunk past the live keys, or an invalid pos, still runs
// and stores its fixed result (m = -inf, l = 0, acc = 0; NaN for an invalid pos).
#pragma once

#include "common.h"

namespace lkd {

typedef float decF4 __attribute__((ext_vector_type(4)));

struct DecodeChunk {
  static constexpr int kKeys = 64;
  decF4 kr[16], vr[16];
  int64_t kb, ke, ps;
  bool badPos, dead;
  int g, d4;

  // pos: this step's row; cap: cache rows. Issues the 32 row loads of the chunk; NT: non-temporal loads (a cache
  // read once, not again in the next step)
  template <bool NT = false>
  __device__ __forceinline__ void load(const float* kc, const float* vc, int64_t pos, int64_t cap, int chunk,
                                       int64_t D, int64_t c4) {
    const int lane = threadIdx.x & 63;
    g = lane >> 4;
    d4 = lane & 15;
    ps = pos;
    badPos = pos < 0 || pos >= cap;
    const int64_t psc = badPos ? 0 : pos;
    kb = static_cast<int64_t>(chunk) * kKeys;
    ke = min<int64_t>(psc + 1, kb + kKeys);
    dead = kb >= ke;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t row = min<int64_t>(kb + g + 4 * i, ke - 1);
      if constexpr (NT) {
        kr[i] = __builtin_nontemporal_load(reinterpret_cast<const decF4*>(kc + row * D + c4));
        vr[i] = __builtin_nontemporal_load(reinterpret_cast<const decF4*>(vc + row * D + c4));
      } else {
        kr[i] = *reinterpret_cast<const decF4*>(kc + row * D + c4);
        vr[i] = *reinterpret_cast<const decF4*>(vc + row * D + c4);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // all 32 row loads issued here, not spread into the reduction
  }

  struct Result {
    float m, l;  // chunk max and sum of 2^{s - m} (-inf, 0 for a chunk past the live keys)
    decF4 acc;   // sum of 2^{s - m} v over the chunk, this lane's 4 dims (the same in every row of the wave)
  };

  // q (already scaled by log2(e) / sqrt(64)), knew, vnew: this lane's 4 dims.
  __device__ __forceinline__ Result compute(decF4 q, decF4 knew, decF4 vnew) const {
    const float snew = rowSum16((q.x * knew.x + q.y * knew.y) + (q.z * knew.z + q.w * knew.w));
    float sc[16];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t key = kb + g + 4 * i;
      const float dot = rowSum16((q.x * kr[i].x + q.y * kr[i].y) + (q.z * kr[i].z + q.w * kr[i].w));
      sc[i] = key < ke ? (key == ps ? snew : dot) : -INFINITY;
      m = fmaxf(m, sc[i]);
    }
    m = crossRowMax(m);
    float l = 0.0f;
    decF4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t key = kb + g + 4 * i;
      const float pj = key < ke ? __builtin_amdgcn_exp2f(sc[i] - m) : 0.0f;
      l += pj;
      const decF4 v = key < ke ? (key == ps ? vnew : vr[i]) : decF4{0.f, 0.f, 0.f, 0.f};
      acc += pj * v;
    }
    l = crossRowSum(l);
    acc.x = crossRowSum(acc.x);
    acc.y = crossRowSum(acc.y);
    acc.z = crossRowSum(acc.z);
    acc.w = crossRowSum(acc.w);
    if (dead) return Result{-INFINITY, 0.0f, decF4{0.f, 0.f, 0.f, 0.f}};
    return Result{m, l, acc};
  }

  // Stores (m, l, acc[64]) to part: lane 0 writes m, l, row 0 the 64 dims; NaN partials for an invalid pos.
  __device__ __forceinline__ void store(Result r, float* part) const {
    const int lane = threadIdx.x & 63;
    if (badPos) {
      const float nan = __builtin_nanf("");
      r = Result{nan, 1.0f, decF4{nan, nan, nan, nan}};
    }
    if (lane == 0) {
      part[0] = r.m;
      part[1] = r.l;
    }
    if (g == 0) reinterpret_cast<decF4*>(part + 2)[d4] = r.acc;
  }

  __device__ __forceinline__ void finish(decF4 q, decF4 knew, decF4 vnew, float* part) const {
    store(compute(q, knew, vnew), part);
  }

  // Online combination of two chunk results (the running one first): both rescaled to the larger max.
  __device__ __forceinline__ static Result combine(Result a, Result b) {
    const float m = fmaxf(a.m, b.m);
    const float wa = a.l > 0.0f ? __builtin_amdgcn_exp2f(a.m - m) : 0.0f;
    const float wb = b.l > 0.0f ? __builtin_amdgcn_exp2f(b.m - m) : 0.0f;
    return Result{m, a.l * wa + b.l * wb, a.acc * wa + b.acc * wb};
  }

  // true for the lanes that write this lane's 4 dims of row pos (row 0 of the chunk that holds pos)
  __device__ __forceinline__ bool writesRow() const { return !badPos && g == 0 && ps >= kb && ps < kb + kKeys; }
};

}  // namespace lkd
