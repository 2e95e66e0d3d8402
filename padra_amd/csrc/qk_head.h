// Q/K RMSNorm + NeoX RoPE (+ BF16 KV store) with one wave per head vector, for launches
// with few tokens (a decode step): lane l holds reference threads l and l + 64 of the
// head's 128-thread block (qk_rope_store_exact.cuh:27-44), i.e. features l and l + 64.
//
//  - Thread t's compensated sum is (x_t^2, 0) (one Accumulate from zero,
//    inference.cu:103-109).  Warp w's shuffle-down tree (inference.cu:111-119) runs on the
//    32 lanes that hold its threads: warps 0 and 1 in the first register of lanes 0-31 and
//    32-63, warps 2 and 3 in the second.  Level 16 is a v_permlane16_swap exchange
//    between the 16-lane rows of each 32-lane half, levels 8..1 are DPP row shifts.
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

// One 32-thread warp tree on the partial (s, e) of every lane: after it, lane 32h of each
// half holds its warp's (sum, error).  Lanes whose partner lies outside the warp read
// values the tree never consumes.
__device__ __forceinline__ void warp_tree_lanes(float &s, float &e) {
  {
    const float s2 = lane_xor<16>(s), e2 = lane_xor<16>(e);
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

// The stages on feature bits 0..5 (bit 0 first) of the N values of a lane.
template <int N> __device__ __forceinline__ void hadamard64_lanes(float (&x)[N], int lane) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<1>(x[i], lane);
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<2>(x[i], lane);
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<4>(x[i], lane);
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<8>(x[i], lane);
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<16>(x[i], lane);
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = hadamard_lane<32>(x[i], lane);
}
// Maximum over the 32-lane half (S = 16) or over the wave (S = 32).
template <int S> __device__ __forceinline__ float lanes_max(float m) {
  return xor_reduce<S>(m, [](float x, float y) { return fmaxf(x, y); });
}

// The quantized codes of one head vector held by a wave, lane l holding features l and
// l + 64 in x0 and x1: computed, not stored (kv_q8.cuh:56-73, kv_q8_native.cuh:76-100).
//  - `bad`: a non-finite value (q8: or a value that is not BF16-exact) in this lane.
//  - q8: scale = amax/127 over the head (1 for a zero head), codes RNE(x / scale) clamped
//    to +-127: the reciprocal form where q8_fast_ok admits it, else the division.
//  - q8_0: the rotation for the rotated format (K: stages on feature bits 0..6, scale
//    1/sqrt(128); V: bits 0..5, scale 1/8), then blocks of 32 features: x0 is in block
//    l / 32, x1 in block 2 + l / 32, so a block is a 32-lane half of one register;
//    d = half(amax/127), codes roundf(x * (1/d_fp32)) clamped; `fail0` / `fail1` when the
//    block's amax or d is not finite.
struct LaneCodes {
  uint32_t c0, c1;
  float scale;     // q8
  uint32_t d0, d1; // q8_0: fp16 bits of the blocks' scales
  bool bad, fail0, fail1;
};
template <int FMT, bool ISV>
__device__ __forceinline__ LaneCodes lane_codes(float x0, float x1, int lane) {
  LaneCodes r;
  r.bad = !isfinite(x0) || !isfinite(x1);
  if constexpr (FMT == PADRA_KV_Q8)
    r.bad = r.bad || ((__float_as_uint(x0) | __float_as_uint(x1)) & 0xffffu) != 0;
  r.fail0 = r.fail1 = false;
  r.d0 = r.d1 = 0;
  r.scale = 1.f;
  if constexpr (FMT == PADRA_KV_Q8) {
    const float m = lanes_max<32>(fmaxf(fabsf(x0), fabsf(x1)));
    const float scale = m == 0.f ? 1.f : m / 127.f, inverse = 1.f / scale;
    r.scale = scale;
    if (q8_fast_ok(scale)) { // wave-uniform: the divisions stay off the common path
      r.c0 = q8_code_fast(x0, scale, inverse);
      r.c1 = q8_code_fast(x1, scale, inverse);
    } else {
      r.c0 = q8_code(x0, scale);
      r.c1 = q8_code(x1, scale);
    }
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      float x[2] = {x0, x1};
      hadamard64_lanes(x, lane);
      if constexpr (ISV) {
        x0 = x[0] * .125f;
        x1 = x[1] * .125f;
      } else {
        x0 = (x[0] + x[1]) * .08838834764831845f;
        x1 = (x[0] - x[1]) * .08838834764831845f;
      }
    }
    const float a0 = lanes_max<16>(fabsf(x0)), a1 = lanes_max<16>(fabsf(x1));
    const float d0 = a0 / 127.f, d1 = a1 / 127.f;
    const __half h0 = __float2half(d0), h1 = __float2half(d1);
    r.fail0 = !isfinite(a0) || !isfinite(__half2float(h0));
    r.fail1 = !isfinite(a1) || !isfinite(__half2float(h1));
    r.d0 = __half_as_ushort(h0);
    r.d1 = __half_as_ushort(h1);
    r.c0 = q8_0_code(x0, d0 == 0.f ? 0.f : 1.f / d0);
    r.c1 = q8_0_code(x1, d1 == 0.f ? 0.f : 1.f / d1);
  }
  return r;
}

// Stores the codes of one (token, KV head) pair into cache row `slot`, by the rules of the
// reference's one warp per pair (kv_q8.cuh:41-73, kv_q8_native.cuh:52-101), as the quad
// encoder does:
//  - a bad value in K or V raises the flag and neither row is written;
//  - q8: codes of both, then the (k, v) scale pair as one 8-byte store;
//  - q8_0: block r of K and V is written for every r before the first block whose K or V
//    scale fails; the flag is raised at a failing block.
template <int FMT, class A>
__device__ __forceinline__ void store_pair_lanes(const A &a, const LaneCodes &k,
                                                 const LaneCodes &v, long long slot, int h,
                                                 int lane) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  if (__ballot(k.bad || v.bad) != 0) { // wave-uniform
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  if constexpr (FMT == PADRA_KV_Q8) {
    uint8_t *kq = static_cast<uint8_t *>(a.kc) + slot * features + h * D;
    uint8_t *vq = static_cast<uint8_t *>(a.vc) + slot * features + h * D;
    kq[lane] = (uint8_t)k.c0;
    kq[64 + lane] = (uint8_t)k.c1;
    vq[lane] = (uint8_t)v.c0;
    vq[64 + lane] = (uint8_t)v.c1;
    if (lane == 0)
      reinterpret_cast<float2 *>(a.scales)[slot * a.hkv + h] = make_float2(k.scale, v.scale);
  } else {
    const int half = lane >> 5;
    // First failing block (4 = none): block `half` in the first registers, half + 2 in
    // the second.
    const int mine = (k.fail0 || v.fail0) ? half : ((k.fail1 || v.fail1) ? half + 2 : 4);
    const int stop = min(mine, lane_xor<32>(mine));
    if (stop < 4 && lane == 0)
      raise_bad(a.bad);
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    uint8_t *kr = static_cast<uint8_t *>(a.kc) + slot * row_bytes;
    uint8_t *vr = static_cast<uint8_t *>(a.vc) + slot * row_bytes;
    const int qoff = 2 * (features / 32) + h * D;
    uint16_t *kd = reinterpret_cast<uint16_t *>(kr) + h * 4;
    uint16_t *vd = reinterpret_cast<uint16_t *>(vr) + h * 4;
    if (half < stop) {
      kr[qoff + lane] = (uint8_t)k.c0;
      vr[qoff + lane] = (uint8_t)v.c0;
      if ((lane & 31) == 0) { // lanes 0 and 32: the scales of blocks 0 and 1
        kd[half] = (uint16_t)k.d0;
        vd[half] = (uint16_t)v.d0;
      }
    }
    if (half + 2 < stop) {
      kr[qoff + 64 + lane] = (uint8_t)k.c1;
      vr[qoff + 64 + lane] = (uint8_t)v.c1;
      if ((lane & 31) == 0) {
        kd[half + 2] = (uint16_t)k.d1;
        vd[half + 2] = (uint16_t)v.d1;
      }
    }
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

// RMSNorm + NeoX RoPE of the head vector held by a wave (features l and l + 64 in x0
// and x1; w the norm weights and c, sn the table entries of the lane's pair index):
// the rotated BF16 values lo and hi; false when the sum of squares or a result is not
// finite.
//  - Threads l and l + 64 start from (x^2, 0); the warp trees, then the partials' fold.
//  - A = B(B(x * inv) * w); lo = B(B(a c) + B((-b) s)), hi = B(B(b c) + B(a s))
//    (qk_rope_store_exact.cuh:39-44).
__device__ __forceinline__ bool head_norm_rope(float x0, float x1, float w0, float w1, float c,
                                               float sn, float eps, float &lo, float &hi) {
  constexpr int D = 128;
  // The order-free sum (sumsq_margin), or (rarely; wave-uniform) the reference's tree.
  float sum;
  if (!certified_sum(wave_sum64(sq64_rn(x1, sq64_rn(x0, 0.0))), sumsq_margin(1, 8), sum)) {
    float s0 = x0 * x0, e0 = 0.f, s1 = x1 * x1, e1 = 0.f;
    warp_tree_lanes(s0, e0);
    warp_tree_lanes(s1, e1);
    fold(s1, e1, s0, e0); // lane 0: w0 + w2; lane 32: w1 + w3
    float S = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s0), 0));
    float E = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), 0));
    const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s0), 32));
    const float e2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), 32));
    fold(s2, e2, S, E);
    sum = S + E;
  }
  const float inv = 1.f / sqrtf(sum / (float)D + eps);
  const float an = B(B(x0 * inv) * w0), bn = B(B(x1 * inv) * w1);
  lo = B(B(an * c) + B((-bn) * sn));
  hi = B(B(bn * c) + B(an * sn));
  return isfinite(sum) && bf16_finite_after_round(lo) && bf16_finite_after_round(hi);
}

// Head vector `hv` of the flat index space (q heads, k heads, v heads).  FMT: -1 (no
// cache) or PADRA_KV_BF16; with a quantized format only Q heads come here, whose position
// must admit the ring as the pair's does.  Every lane of the wave takes part (the
// exchanges need them).
template <class T, int FMT>
__device__ __forceinline__ void qk_head_wave_plain(const QKArgs<T> &a, unsigned hv) {
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
  // The norm weights before the position check, so that they are in flight with the data.
  const uint16_t *w = (role == 1 ? a.kn : a.qn);
  const float w0 = head_load(w + lane), w1 = head_load(w + 64 + lane);
  bool ok = false;
  const int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first,
                                   FMT > PADRA_KV_BF16, ok);
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
  const uint16_t *trow = a.table + (size_t)pos * D;
  const float c = head_load(trow + lane), sn = head_load(trow + 64 + lane);
  float lo, hi;
  const bool fine = head_norm_rope(x0, x1, w0, w1, c, sn, a.eps, lo, hi);
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

// K head `kidx` (token kidx / hkv, head kidx % hkv) with a quantized cache: the K norm and
// RoPE, and the codes of the (token, KV head) pair, the wave having loaded V head kidx
// too.  V's codes are computed before K's norm, in the same straight-line code, so that
// the two dependent chains interleave; the flag checks and the stores come last.
template <class T, int FMT>
__device__ __forceinline__ void qk_pair_wave(const QKArgs<T> &a, unsigned kidx) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int t = (int)(kidx / (unsigned)a.hkv);
  const int hh = (int)(kidx - (unsigned)t * (unsigned)a.hkv);
  const PosState ps = fetch_state(a.pos, t);
  const T *src = a.k + (size_t)kidx * D, *vsrc = a.v + (size_t)kidx * D;
  const float x0 = head_load(src + lane), x1 = head_load(src + 64 + lane);
  const float v0 = head_load(vsrc + lane), v1 = head_load(vsrc + 64 + lane);
  const float w0 = head_load(a.kn + lane), w1 = head_load(a.kn + 64 + lane);
  bool ok = false;
  const int pos = resolve_position(a.pos, ps, t, a.cap, a.first, true, ok);
  ok = ok && pos >= 0 && pos < a.table_rows;
  if (!ok) {
    if (lane == 0)
      raise_bad(a.bad);
    return; // wave-uniform
  }
  const uint16_t *trow = a.table + (size_t)pos * D;
  const float c = head_load(trow + lane), sn = head_load(trow + 64 + lane);
  const LaneCodes cv = lane_codes<FMT, true>(v0, v1, lane);
  float lo, hi;
  const bool fine = head_norm_rope(x0, x1, w0, w1, c, sn, a.eps, lo, hi);
  const LaneCodes ck = lane_codes<FMT, false>(lo, hi, lane);
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
  T *dst = const_cast<T *>(src);
  head_store(dst + lane, lo);
  head_store(dst + 64 + lane, hi);
  if (t >= a.first) {
    const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
    store_pair_lanes<FMT>(a, ck, cv, seq * a.seq_stride + ring_slot(pos, a.cap), hh, lane);
  }
}

// Head vector `hv` of the flat index space (q heads, k heads and, with a BF16 cache,
// v heads).  With a quantized cache the wave of K head (t, h) also encodes V head (t, h).
template <class T, int FMT>
__device__ __forceinline__ void qk_head_wave(const QKArgs<T> &a, unsigned hv) {
  if constexpr (FMT > PADRA_KV_BF16) {
    const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
    if (hv < nq)
      qk_head_wave_plain<T, FMT>(a, hv); // a Q head: no cache work
    else if (hv < nq + (unsigned)a.tokens * (unsigned)a.hkv)
      qk_pair_wave<T, FMT>(a, hv - nq);
  } else {
    qk_head_wave_plain<T, FMT>(a, hv);
  }
}

// Waves of a per-head launch: one per head vector (q, k and, with a BF16 cache, v).
template <int FMT>
__host__ __device__ inline long long qk_head_waves(int tokens, int q_heads, int kv_heads) {
  return (long long)tokens * (q_heads + kv_heads * (FMT == PADRA_KV_BF16 ? 2 : 1));
}

} // namespace padra
