// Q/K RMSNorm + NeoX RoPE (+ BF16 KV store) with one wave per head vector, for launches
// with few tokens (a decode step): lane l holds reference threads l and l + 64 of the
// head's 128-thread block (qk_rope_store_exact.cuh:27-44), i.e. features l and l + 64.
//
//  - Thread t's compensated sum is (x_t^2, 0) (one Accumulate from zero,
//    inference.cu:103-109).  Warp w's shuffle-down tree (inference.cu:111-119) runs on the
//    32 lanes that hold its threads: warps 0 and 1 in the first register of lanes 0-31 and
//    32-63, warps 2 and 3 in the second.  Level 16 is a ds_swizzle exchange inside each
//    32-lane half, levels 8..1 are DPP row shifts.
//  - The four warp partials then fold as (w0 + w2) + (w1 + w3), the order the quad layout
//    (qk_quad.h) replays: lane 0 holds w0 and w2, lane 32 w1 and w3.
//  - RoPE pairs feature f < 64 with f + 64: both sit in the same lane.
// The quad layout (qk_quad.h) spends 32 features per lane and wins when the grid fills the
// GPU; with a few hundred heads each quad wave runs alone on its SIMD and its ~900
// dependent instructions set the launch's time, while here a wave has two features per
// lane and about a fifth of the instructions.
#pragma once
#include <type_traits>

#include "qk_heads.h"

namespace padra {

// Value of lane (lane ^ 16) inside each 32-lane half (ds_swizzle bit mode: and 0x1f,
// or 0, xor 0x10).
__device__ __forceinline__ float swizzle_xor16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

// One 32-thread warp tree on the partial (s, e) of every lane: after it, lane 32h of each
// half holds its warp's (sum, error).  Lanes whose partner lies outside the warp read
// values the tree never consumes.
__device__ __forceinline__ void warp_tree_lanes(float &s, float &e) {
  {
    const float s2 = swizzle_xor16(s), e2 = swizzle_xor16(e);
    fold(s2, e2, s, e);
  }
  {
    const float s2 = lane_down<8>(s), e2 = lane_down<8>(e);
    fold(s2, e2, s, e);
  }
  {
    const float s2 = lane_down<4>(s), e2 = lane_down<4>(e);
    fold(s2, e2, s, e);
  }
  {
    const float s2 = lane_down<2>(s), e2 = lane_down<2>(e);
    fold(s2, e2, s, e);
  }
  {
    const float s2 = lane_down<1>(s), e2 = lane_down<1>(e);
    fold(s2, e2, s, e);
  }
}

template <class T> __device__ __forceinline__ float head_load(const T *p) {
  if constexpr (std::is_same<T, uint16_t>::value)
    return __uint_as_float((uint32_t)*p << 16);
  else
    return *p;
}
template <class T> __device__ __forceinline__ void head_store(T *p, float v) {
  if constexpr (std::is_same<T, uint16_t>::value)
    *p = (uint16_t)(__float_as_uint(v) >> 16);
  else
    *p = v;
}

// Head vector `hv` of the flat index space (q heads, k heads, v heads).  FMT: -1 (no
// cache) or PADRA_KV_BF16.  Every lane of the wave takes part (the exchanges need them).
template <class T, int FMT>
__device__ __forceinline__ void qk_head_wave(const QKArgs<T> &a, unsigned hv) {
  static_assert(FMT <= PADRA_KV_BF16, "the per-head layout stores BF16 caches only");
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned total = nq + nk + (FMT >= 0 ? nk : 0u);
  if (hv >= total)
    return; // wave-uniform
  const int role = hv < nq ? 0 : (hv < nq + nk ? 1 : 2); // 0 q, 1 k, 2 v
  const unsigned idx = role == 0 ? hv : (role == 1 ? hv - nq : hv - nq - nk);
  const unsigned heads = role == 0 ? (unsigned)a.hq : (unsigned)a.hkv;
  const int t = (int)(idx / heads);
  const int hh = (int)(idx - (unsigned)t * heads);
  // The control record first, then the head's two features, then the position.
  const PosState ps = fetch_state(a.pos, t);
  const T *src = head_src(a, hv, nq, nk);
  const float x0 = head_load(src + lane), x1 = head_load(src + 64 + lane);
  bool ok = false;
  const int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first, false, ok);
  ok = ok && pos >= 0 && pos < a.table_rows;
  if (!ok) {
    if (lane == 0)
      raise_bad(a.bad);
    return; // wave-uniform
  }
  const int features = a.hkv * D;
  const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
  const bool store = FMT == PADRA_KV_BF16 && role >= 1 && t >= a.first;
  const long long row = store ? (seq * a.seq_stride + ring_slot(pos, a.cap)) * features + hh * D : 0;
  if (role == 2) { // V head: its BF16 row into the cache
    if (store) {
      uint16_t *vc = static_cast<uint16_t *>(a.vc) + row;
      vc[lane] = (uint16_t)(pack2(0.f, x0) >> 16);
      vc[64 + lane] = (uint16_t)(pack2(0.f, x1) >> 16);
    }
    return;
  }
  const uint16_t *w = (role == 1 ? a.kn : a.qn);
  const float w0 = head_load(w + lane), w1 = head_load(w + 64 + lane);
  const uint16_t *trow = a.table + (size_t)pos * D;
  const float c = head_load(trow + lane), sn = head_load(trow + 64 + lane);

  // Threads l and l + 64: (x^2, 0), then the warp trees and the partials' fold.
  float s0 = x0 * x0, e0 = 0.f, s1 = x1 * x1, e1 = 0.f;
  warp_tree_lanes(s0, e0);
  warp_tree_lanes(s1, e1);
  fold(s1, e1, s0, e0); // lane 0: w0 + w2; lane 32: w1 + w3
  float S = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s0), 0));
  float E = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), 0));
  const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s0), 32));
  const float e2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), 32));
  fold(s2, e2, S, E);
  const float sum = S + E;
  const float inv = 1.f / sqrtf(sum / (float)D + a.eps);
  // A = B(B(x * inv) * w); lo = B(B(a c) + B((-b) s)), hi = B(B(b c) + B(a s)).
  const float an = B(B(x0 * inv) * w0), bn = B(B(x1 * inv) * w1);
  const float lo = B(B(an * c) + B((-bn) * sn));
  const float hi = B(B(bn * c) + B(an * sn));
  const bool fine = isfinite(sum) && bf16_finite_after_round(lo) && bf16_finite_after_round(hi);
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
  T *dst = const_cast<T *>(src);
  head_store(dst + lane, lo);
  head_store(dst + 64 + lane, hi);
  if (role == 1 && store) {
    uint16_t *kc = static_cast<uint16_t *>(a.kc) + row;
    kc[lane] = (uint16_t)(__float_as_uint(lo) >> 16);
    kc[64 + lane] = (uint16_t)(__float_as_uint(hi) >> 16);
  }
}

// Waves of a per-head launch: one per head vector (q, k and, with a cache, v).
template <int FMT>
__host__ __device__ inline long long qk_head_waves(int tokens, int q_heads, int kv_heads) {
  return (long long)tokens * (q_heads + kv_heads * (FMT >= 0 ? 2 : 1));
}

} // namespace padra
