// Helpers of the per-head Q/K RMSNorm + NeoX RoPE + KV-cache store: the in-lane warp
// tree, the Hadamard stages, and the lane-pair K/V encoders of the store-only kernel
// (padra_KVStore), which holds a head in two lanes.  The Q/K kernels themselves hold a
// head in four lanes (qk_quad.h).
//
// Reference: QKNormRopeStoreControlled (qk_rope_store_exact.cuh:4-49), QKNormRope
// (qknorm_rope.cuh:4-50), QKNormRopePair64 (qknorm_rope_pair64.cuh:3-83).  The reference
// block has 128 threads, one feature each; warp w (features 32w..32w+31) reduces its
// squares with a shuffle-down tree and the four warp partials reduce as
// ((w0 + w2) + (w1 + w3)).  A lane holding warp w's 32 features runs that warp's whole
// tree in-lane (warp_sumsq32).  The first tree level adds two squares with zero error
// terms; it is written out directly (its error fold is an exact no-op).
#pragma once
#include <type_traits>

#include "common.h"
#include "norm_rows.h"

namespace padra {

template <class T> struct QKArgs {
  T *q, *k;
  const T *v;
  const uint16_t *qn, *kn, *table;
  int table_rows, tokens, hq, hkv;
  float eps;
  PosSrc pos;
  // KV binding (format is a template parameter).
  void *kc, *vc, *scales;
  int cap, first;
  long long seq_stride;
  int *bad;
};

// Compensated sum of squares of one warp's 32 features, in the reference tree order
// (shuffle-down levels 16, 8, 4, 2, 1 of inference.cu:111-119).
__device__ __forceinline__ void warp_sumsq32(const float (&x)[32], float &S, float &E) {
  float s[16], e[16];
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    const float a2 = x[f] * x[f], b2 = x[f + 16] * x[f + 16];
    s[f] = a2 + b2;
    e[f] = (fmaxf(a2, b2) - s[f]) + fminf(a2, b2);
  }
#pragma unroll
  for (int f = 0; f < 8; ++f)
    fold(s[f + 8], e[f + 8], s[f], e[f]);
#pragma unroll
  for (int f = 0; f < 4; ++f)
    fold(s[f + 4], e[f + 4], s[f], e[f]);
#pragma unroll
  for (int f = 0; f < 2; ++f)
    fold(s[f + 2], e[f + 2], s[f], e[f]);
  fold(s[1], e[1], s[0], e[0]);
  S = s[0];
  E = e[0];
}

template <class T>
__device__ __forceinline__ void store32(T *p, const uint32_t (&w)[16]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t c[4] = {w[4 * m], w[4 * m + 1], w[4 * m + 2], w[4 * m + 3]};
    ActIO<T>::store8(p + 8 * m, c);
  }
}
__device__ __forceinline__ void store32_bf16(uint16_t *p, const uint32_t (&w)[16]) {
  store32<uint16_t>(p, w);
}

// Hadamard butterflies on the 32 in-lane features (feature bits 0..4), in stage order
// bit 0 first: lower' = lower + upper, upper' = lower - upper (kv_q8_native.cuh:24-31).
__device__ __forceinline__ void hadamard32(float (&x)[32]) {
#pragma unroll
  for (int bit = 1; bit < 32; bit *= 2)
#pragma unroll
    for (int f = 0; f < 32; ++f)
      if (!(f & bit)) {
        const float lower = x[f], upper = x[f | bit];
        x[f] = lower + upper;
        x[f | bit] = lower - upper;
      }
}
// Stage on feature bit 5 (features f and f + 32 live in the two lanes of the pair).
__device__ __forceinline__ void hadamard_cross(float (&x)[32], int half) {
#pragma unroll
  for (int f = 0; f < 32; ++f) {
    const float other = shfl_xor(x[f], 1);
    x[f] = half ? other - x[f] : x[f] + other;
  }
}

__device__ __forceinline__ void store_codes32(int8_t *p, const uint32_t (&w)[8]) {
  st_nt(reinterpret_cast<uint4 *>(p), make_uint4(w[0], w[1], w[2], w[3]));
  st_nt(reinterpret_cast<uint4 *>(p) + 1, make_uint4(w[4], w[5], w[6], w[7]));
}

// Q8 / Q8_0 encoding of one head vector of the K cache (ISV false: the rotated K row)
// or the V cache (ISV true), held by the two lanes of a pair: this lane has features
// 32*half + i in xa and 64 + 32*half + i in xb.  Writes codes and scales to row `slot`.
// The pair at lane ^ 32 holds the same head's other vector and is active with this one.
// As in the reference's one warp per (token, head) (kv_q8.cuh:41-73,
// kv_q8_native.cuh:70-100), an invalid K or V vector (non-finite, or for q8 not
// BF16-exact) raises the flag and writes neither, and a q8_0 block that fails in K or in
// V ends the writes of both.
template <int FMT, class A>
__device__ __forceinline__ void encode_head_q(const A &a, float (&xa)[32], float (&xb)[32],
                                              long long slot, int h, int half, bool isv) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  bool invalid = false;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    invalid |= !isfinite(xa[i]) || !isfinite(xb[i]);
    if constexpr (FMT == PADRA_KV_Q8) // q8 also rejects values that are not BF16-exact
      invalid |= (__float_as_uint(xa[i]) & 0xffffu) != 0 || (__float_as_uint(xb[i]) & 0xffffu) != 0;
  }
  // Both exchanges run in every lane (a lane that skipped one would leave its value
  // unreadable to the partner).
  const int pair_bad = __shfl_xor((int)invalid, 1, 64);
  invalid = invalid || pair_bad != 0;
  const int other_bad = __shfl_xor((int)invalid, 32, 64);
  invalid = invalid || other_bad != 0;
  if (invalid) {
    if (half == 0)
      raise_bad(a.bad);
    return;
  }
  if constexpr (FMT == PADRA_KV_Q8) {
    // kv_q8::Encode (kv_q8.cuh:56-73): scale = amax/127 (1 for an all-zero head), codes
    // RNE(x / scale) clamped to +-127.
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      m = fmaxf(m, fmaxf(fabsf(xa[i]), fabsf(xb[i])));
    m = fmaxf(m, shfl_xor(m, 1));
    const float scale = m == 0.f ? 1.f : m / 127.f;
    int8_t *codes = static_cast<int8_t *>(isv ? a.vc : a.kc) + slot * features + h * D;
    const float inverse = 1.f / scale;
    const bool fast = q8_fast_ok(scale); // pair-uniform
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      auto code = [&](float x) { return fast ? q8_code_fast(x, scale, inverse) : q8_code(x, scale); };
      w0[i] = pack_codes4(code(xa[4 * i]), code(xa[4 * i + 1]), code(xa[4 * i + 2]),
                          code(xa[4 * i + 3]));
      w1[i] = pack_codes4(code(xb[4 * i]), code(xb[4 * i + 1]), code(xb[4 * i + 2]),
                          code(xb[4 * i + 3]));
    }
    store_codes32(codes + 32 * half, w0);
    store_codes32(codes + 64 + 32 * half, w1);
    if (half == 0)
      reinterpret_cast<float *>(a.scales)[(slot * a.hkv + h) * 2 + (isv ? 1 : 0)] = scale;
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      // q8_native::Rotate (kv_q8_native.cuh:22-45): stages on feature bits 0..4 in lane,
      // bit 5 across the pair, and for K bit 6 between the lane's two groups.
      hadamard32(xa);
      hadamard32(xb);
      hadamard_cross(xa, half);
      hadamard_cross(xb, half);
      // K: the stage on feature bit 6 (xa with xb) and the 1/sqrt(128) scale; V: the 1/8
      // scale.  Lanes of both halves run this loop with per-lane operands: for V,
      // lower + 0 and lower - 0 leave each value (a zero's sign aside, which no code or
      // scale sees).
      const float sc = isv ? .125f : .08838834764831845f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const float lower = xa[i], upper = isv ? 0.f : xb[i];
        xa[i] = (lower + upper) * sc;
        xb[i] = (isv ? xb[i] : lower - upper) * sc;
      }
    }
    // Blocks (kv_q8_native.cuh:84-99): this lane holds block `half` (xa) and block
    // `half + 2` (xb); d = half(amax/127), codes roundf(x * (1/d_fp32)).
    float am = 0.f, bm = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      am = fmaxf(am, fabsf(xa[i]));
      bm = fmaxf(bm, fabsf(xb[i]));
    }
    const float ad = am / 127.f, bd = bm / 127.f;
    const __half ah = __float2half(ad), bh = __float2half(bd);
    // A failing block stops the reference at that block: blocks before the first failing
    // one are written, later ones are not.
    const bool fa = !isfinite(am) || !isfinite(__half2float(ah));
    const bool fb = !isfinite(bm) || !isfinite(__half2float(bh));
    const int mine = fa ? half : (fb ? half + 2 : 4);
    int stop = min(mine, __shfl_xor(mine, 1, 64)); // first failing block, 4 = none
    stop = min(stop, __shfl_xor(stop, 32, 64));      // of K and V together
    if (stop < 4 && half == 0)
      raise_bad(a.bad);
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    uint8_t *row = static_cast<uint8_t *>(isv ? a.vc : a.kc) + slot * row_bytes;
    int8_t *qs = reinterpret_cast<int8_t *>(row + 2 * (features / 32) + h * D);
    uint16_t *d = reinterpret_cast<uint16_t *>(row) + h * 4;
    const float ai = ad == 0.f ? 0.f : 1.f / ad, bi = bd == 0.f ? 0.f : 1.f / bd;
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w0[i] = pack_codes4(q8_0_code(xa[4 * i], ai), q8_0_code(xa[4 * i + 1], ai),
                          q8_0_code(xa[4 * i + 2], ai), q8_0_code(xa[4 * i + 3], ai));
      w1[i] = pack_codes4(q8_0_code(xb[4 * i], bi), q8_0_code(xb[4 * i + 1], bi),
                          q8_0_code(xb[4 * i + 2], bi), q8_0_code(xb[4 * i + 3], bi));
    }
    const uint16_t a16 = __half_as_ushort(ah), b16 = __half_as_ushort(bh);
    if (stop == 4) {
      // The head's four block scales go out as one 8-byte store from lane 0 of the pair:
      // d[0] = block 0 (lane 0, a), d[1] = block 1 (lane 1, a), d[2], d[3] the b blocks.
      const uint32_t mine_d = (uint32_t)a16 | ((uint32_t)b16 << 16);
      const uint32_t other = __shfl_xor(mine_d, 1, 64);
      if (half == 0)
        *reinterpret_cast<uint2 *>(d) = make_uint2((mine_d & 0xffffu) | (other << 16),
                                                   (mine_d >> 16) | (other & 0xffff0000u));
      store_codes32(qs + 32 * half, w0);
      store_codes32(qs + 64 + 32 * half, w1);
    } else {
      if (half < stop) {
        d[half] = a16;
        store_codes32(qs + 32 * half, w0);
      }
      if (half + 2 < stop) {
        d[half + 2] = b16;
        store_codes32(qs + 64 + 32 * half, w1);
      }
    }
  }
}

// 32 consecutive activations of one lane, kept packed: 4 x 16 B of BF16 or 8 x 16 B of
// fp32.  get(i) unpacks on use, so the packed words are all that stays live.
template <class T> struct Act32;
template <> struct Act32<uint16_t> {
  uint4 w[4];
  __device__ __forceinline__ void load(const uint16_t *p) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      w[m] = ld_nt(reinterpret_cast<const uint4 *>(p) + m);
  }
  __device__ __forceinline__ uint32_t word(int i) const {
    const uint4 &v = w[i / 4];
    return (i & 3) == 0 ? v.x : (i & 3) == 1 ? v.y : (i & 3) == 2 ? v.z : v.w;
  }
  __device__ __forceinline__ float get(int i) const {
    return i & 1 ? hi16(word(i / 2)) : lo16(word(i / 2));
  }
};
template <> struct Act32<float> {
  float4 f[8];
  __device__ __forceinline__ void load(const float *p) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const uint4 v = ld_nt(reinterpret_cast<const uint4 *>(p) + m);
      f[m] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                         __uint_as_float(v.w));
    }
  }
  __device__ __forceinline__ float get(int i) const {
    const float4 &v = f[i / 4];
    return (i & 3) == 0 ? v.x : (i & 3) == 1 ? v.y : (i & 3) == 2 ? v.z : v.w;
  }
};

// Eight consecutive BF16 values of a cached (re-read) vector: norm weights, table rows.
struct Bf8 {
  uint4 w;
  __device__ __forceinline__ void load(const uint16_t *p) { w = *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ uint32_t word(int i) const {
    return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
  }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t v = word(i / 2);
    return i & 1 ? hi16(v) : lo16(v);
  }
};

template <class X>
__device__ __forceinline__ void group_sumsq(const X &x, float &S, float &E) {
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    v[i] = x.get(i);
  warp_sumsq32(v, S, E);
}

// The source row of head vector hv of the flat index space (q heads, k heads, v heads).
template <class A>
__device__ __forceinline__ auto head_src(const A &a, unsigned hv, unsigned nq, unsigned nk) {
  constexpr int D = 128;
  return hv < nq ? a.q + (size_t)hv * D
                 : (hv < nq + nk ? a.k + (size_t)(hv - nq) * D : a.v + (size_t)(hv - nq - nk) * D);
}

} // namespace padra
