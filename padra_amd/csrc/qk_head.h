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

// Value of lane (lane ^ M) for M a power of two below 64: DPP quad permutes for 1 and 2,
// ds_swizzle (xor inside 32-lane halves) for 4..16, a lane permute for 32.
template <int M> __device__ __forceinline__ float lane_xor(float v) {
  const int i = __float_as_int(v);
  if constexpr (M == 1)
    return __int_as_float(__builtin_amdgcn_mov_dpp(i, 0xb1 /* quad_perm [1,0,3,2] */, 0xf, 0xf, true));
  else if constexpr (M == 2)
    return __int_as_float(__builtin_amdgcn_mov_dpp(i, 0x4e /* quad_perm [2,3,0,1] */, 0xf, 0xf, true));
  else if constexpr (M < 32)
    return __int_as_float(__builtin_amdgcn_ds_swizzle(i, 0x1F | (M << 10)));
  else
    return __shfl_xor(v, 32, 64);
}

// One Hadamard stage on feature bit log2(M), the feature's bit being the lane's:
// lower' = lower + upper, upper' = lower - upper (kv_q8_native.cuh:24-31).
template <int M> __device__ __forceinline__ float hadamard_lane(float v, int lane) {
  const float o = lane_xor<M>(v);
  return (lane & M) ? o - v : v + o;
}
// The stages on feature bits 0..5 (bit 0 first) of the four values of a lane.
__device__ __forceinline__ void hadamard64_lanes(float (&x)[4], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<1>(x[i], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<2>(x[i], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<4>(x[i], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<8>(x[i], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<16>(x[i], lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = hadamard_lane<32>(x[i], lane);
}
// Maximum over the 32-lane half (S = 16) or over the wave (S = 32).
template <int S> __device__ __forceinline__ float lanes_max(float m) {
  m = fmaxf(m, lane_xor<1>(m));
  m = fmaxf(m, lane_xor<2>(m));
  m = fmaxf(m, lane_xor<4>(m));
  m = fmaxf(m, lane_xor<8>(m));
  m = fmaxf(m, lane_xor<16>(m));
  if constexpr (S == 32)
    m = fmaxf(m, lane_xor<32>(m));
  return m;
}

// Quantized encoding of one (token, KV head) pair held by a wave: x = {K feature l,
// K feature l + 64, V feature l, V feature l + 64} in lane l, K the normalized, rotated
// BF16 head.  The reference's one warp per pair (kv_q8.cuh:41-73,
// kv_q8_native.cuh:52-101), with the same rules as the quad encoder:
//  - a non-finite value in K or V (q8: or a value that is not BF16-exact) raises the flag
//    and neither row is written;
//  - q8: scale = amax/127 per head (1 for a zero head), codes RNE(x / scale) clamped to
//    +-127, the (k, v) scale pair as one 8-byte store;
//  - q8_0: the rotation for the rotated format (K: stages on feature bits 0..6, scale
//    1/sqrt(128); V: bits 0..5, scale 1/8), then blocks of 32 features (block l / 32 in
//    x[0], 2 + l / 32 in x[1]; the same for V): d = half(amax/127), codes
//    roundf(x * (1/d_fp32)); block r of K and V is written for every r before the first
//    block whose K or V scale fails, and the flag is raised at a failing block.
template <int FMT, class A>
__device__ __forceinline__ void encode_pair_head(const A &a, float (&x)[4], long long slot,
                                                 int h, int lane) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  bool invalid = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    invalid |= !isfinite(x[i]);
    if constexpr (FMT == PADRA_KV_Q8)
      invalid |= (__float_as_uint(x[i]) & 0xffffu) != 0;
  }
  if (__ballot(invalid) != 0) { // wave-uniform
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  if constexpr (FMT == PADRA_KV_Q8) {
    const float mk = lanes_max<32>(fmaxf(fabsf(x[0]), fabsf(x[1])));
    const float mv = lanes_max<32>(fmaxf(fabsf(x[2]), fabsf(x[3])));
    const float sk = mk == 0.f ? 1.f : mk / 127.f, sv = mv == 0.f ? 1.f : mv / 127.f;
    const float ik = 1.f / sk, iv = 1.f / sv;
    uint32_t c[4];
    if (q8_fast_ok(sk) && q8_fast_ok(sv)) { // wave-uniform
      c[0] = q8_code_fast(x[0], sk, ik);
      c[1] = q8_code_fast(x[1], sk, ik);
      c[2] = q8_code_fast(x[2], sv, iv);
      c[3] = q8_code_fast(x[3], sv, iv);
    } else {
      c[0] = q8_code(x[0], sk);
      c[1] = q8_code(x[1], sk);
      c[2] = q8_code(x[2], sv);
      c[3] = q8_code(x[3], sv);
    }
    uint8_t *kq = static_cast<uint8_t *>(a.kc) + slot * features + h * D;
    uint8_t *vq = static_cast<uint8_t *>(a.vc) + slot * features + h * D;
    kq[lane] = (uint8_t)c[0];
    kq[64 + lane] = (uint8_t)c[1];
    vq[lane] = (uint8_t)c[2];
    vq[64 + lane] = (uint8_t)c[3];
    if (lane == 0)
      reinterpret_cast<float2 *>(a.scales)[slot * a.hkv + h] = make_float2(sk, sv);
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      hadamard64_lanes(x, lane);
      const float k0 = x[0], k1 = x[1];
      x[0] = (k0 + k1) * .08838834764831845f;
      x[1] = (k0 - k1) * .08838834764831845f;
      x[2] *= .125f;
      x[3] *= .125f;
    }
    float d[4];
    uint32_t c[4];
    bool fail_lo = false, fail_hi = false; // blocks half and half + 2 of K or V
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float am = lanes_max<16>(fabsf(x[i]));
      const float ad = am / 127.f;
      const __half dh = __float2half(ad);
      d[i] = __uint_as_float((uint32_t)__half_as_ushort(dh));
      const bool f = !isfinite(am) || !isfinite(__half2float(dh));
      if (i & 1)
        fail_hi |= f;
      else
        fail_lo |= f;
      c[i] = q8_0_code(x[i], ad == 0.f ? 0.f : 1.f / ad);
    }
    const int half = lane >> 5;
    const int mine = fail_lo ? half : (fail_hi ? half + 2 : 4); // first failing block, 4 = none
    const int stop = min(mine, __shfl_xor(mine, 32, 64));
    if (stop < 4 && lane == 0)
      raise_bad(a.bad);
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    uint8_t *kr = static_cast<uint8_t *>(a.kc) + slot * row_bytes;
    uint8_t *vr = static_cast<uint8_t *>(a.vc) + slot * row_bytes;
    const int qoff = 2 * (features / 32) + h * D;
    if (half < stop) {
      kr[qoff + lane] = (uint8_t)c[0];
      vr[qoff + lane] = (uint8_t)c[2];
    }
    if (half + 2 < stop) {
      kr[qoff + 64 + lane] = (uint8_t)c[1];
      vr[qoff + 64 + lane] = (uint8_t)c[3];
    }
    if ((lane & 31) == 0) { // lanes 0 and 32: the block scales of their blocks
      uint16_t *kd = reinterpret_cast<uint16_t *>(kr) + h * 4;
      uint16_t *vd = reinterpret_cast<uint16_t *>(vr) + h * 4;
      if (half < stop) {
        kd[half] = (uint16_t)__float_as_uint(d[0]);
        vd[half] = (uint16_t)__float_as_uint(d[2]);
      }
      if (half + 2 < stop) {
        kd[half + 2] = (uint16_t)__float_as_uint(d[1]);
        vd[half + 2] = (uint16_t)__float_as_uint(d[3]);
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

// Head vector `hv` of the flat index space (q heads, k heads, v heads).  FMT: -1 (no
// cache), PADRA_KV_BF16, or a quantized format: then there are no V waves, and the wave
// of K head (t, h) also loads V head (t, h) and encodes the pair (encode_pair_head).
// Every lane of the wave takes part (the exchanges need them).
template <class T, int FMT>
__device__ __forceinline__ void qk_head_wave(const QKArgs<T> &a, unsigned hv) {
  constexpr int D = 128;
  constexpr bool QUANT = FMT > PADRA_KV_BF16;
  const int lane = threadIdx.x & 63;
  const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned total = nq + nk + (FMT == PADRA_KV_BF16 ? nk : 0u);
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
  float v0 = 0.f, v1 = 0.f;
  if (QUANT && role == 1) {
    const T *vsrc = a.v + (size_t)idx * D;
    v0 = head_load(vsrc + lane);
    v1 = head_load(vsrc + 64 + lane);
  }
  bool ok = false;
  const int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first, QUANT, ok);
  ok = ok && pos >= 0 && pos < a.table_rows;
  if (!ok) {
    if (lane == 0)
      raise_bad(a.bad);
    return; // wave-uniform
  }
  const int features = a.hkv * D;
  const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
  const bool store = FMT >= 0 && role >= 1 && t >= a.first;
  const long long slot = store ? seq * a.seq_stride + ring_slot(pos, a.cap) : 0;
  const long long row = slot * features + hh * D;
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
    if constexpr (QUANT) {
      float pair[4] = {lo, hi, v0, v1};
      encode_pair_head<FMT>(a, pair, slot, hh, lane);
    } else {
      uint16_t *kc = static_cast<uint16_t *>(a.kc) + row;
      kc[lane] = (uint16_t)(__float_as_uint(lo) >> 16);
      kc[64 + lane] = (uint16_t)(__float_as_uint(hi) >> 16);
    }
  }
}

// Waves of a per-head launch: one per head vector (q, k and, with a BF16 cache, v).
template <int FMT>
__host__ __device__ inline long long qk_head_waves(int tokens, int q_heads, int kv_heads) {
  return (long long)tokens * (q_heads + kv_heads * (FMT == PADRA_KV_BF16 ? 2 : 1));
}

} // namespace padra
