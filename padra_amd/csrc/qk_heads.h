// Helpers of the Q/K RMSNorm + NeoX RoPE + KV-cache store kernels (qk_quad.h, qk_head.h)
// and the store-only kernels (kv_codec.hip): the argument block, the in-lane warp tree,
// the in-lane Hadamard stages, and packed activation and code stores.
//
// Reference: QKNormRopeStoreControlled (qk_rope_store_exact.cuh:4-49), QKNormRope
// (qknorm_rope.cuh:4-50), QKNormRopePair64 (qknorm_rope_pair64.cuh:3-83).  The reference
// block has 128 threads, one feature each; warp w (features 32w..32w+31) reduces its
// squares with a shuffle-down tree and the four warp partials reduce as
// ((w0 + w2) + (w1 + w3)).  A lane holding warp w's 32 features runs that warp's whole
// tree in-lane (warp_tree_node).  The first tree level adds two squares with zero error
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
// (shuffle-down levels 16, 8, 4, 2, 1 of inference.cu:111-119): after level d, slot f < d
// holds slot f of level 2d folded with slot f + d of level 2d, and level 16 pairs features
// f and f + 16.  Evaluated depth first (slot f of level d from its two children), so that
// at most one partial per level is live: the tree is the rarely taken branch of the Q/K
// waves, and a breadth-first form (16 partials at once) set the kernel's register count.
template <int F, int D, class X>
__device__ __forceinline__ void warp_tree_node(const X &x, float &s, float &e) {
  if constexpr (D == 16) {
    const float a = x.get(F), b = x.get(F + 16);
    const float a2 = a * a, b2 = b * b;
    s = a2 + b2;
    e = (fmaxf(a2, b2) - s) + fminf(a2, b2);
  } else {
    float s2, e2;
    warp_tree_node<F, 2 * D>(x, s, e);
    warp_tree_node<F + D, 2 * D>(x, s2, e2);
    fold(s2, e2, s, e);
  }
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
// The q8_0 codes of a lane's 32-value block, packed four to a word: without the clamp
// when every active lane of the wave has a finite inverse (wave-uniform test).
__device__ __forceinline__ void q8_0_codes32(const float (&x)[32], float inverse,
                                             uint32_t (&w)[8]) {
  if (__ballot(!isfinite(inverse)) == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w[i] = pack_codes4(q8_0_code_in_range(x[4 * i], inverse),
                         q8_0_code_in_range(x[4 * i + 1], inverse),
                         q8_0_code_in_range(x[4 * i + 2], inverse),
                         q8_0_code_in_range(x[4 * i + 3], inverse));
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w[i] = pack_codes4(q8_0_code(x[4 * i], inverse), q8_0_code(x[4 * i + 1], inverse),
                         q8_0_code(x[4 * i + 2], inverse), q8_0_code(x[4 * i + 3], inverse));
  }
}

__device__ __forceinline__ void store_codes32(int8_t *p, const uint32_t (&w)[8]) {
  st_nt(reinterpret_cast<uint4 *>(p), make_uint4(w[0], w[1], w[2], w[3]));
  st_nt(reinterpret_cast<uint4 *>(p) + 1, make_uint4(w[4], w[5], w[6], w[7]));
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

// The same tree evaluated breadth first (16 partials at once): the form the tree-only
// waves use (it schedules better there).
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

template <class X>
__device__ __forceinline__ void group_sumsq(const X &x, float &S, float &E) {
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    v[i] = x.get(i);
  warp_sumsq32(v, S, E);
}
template <class X>
__device__ __forceinline__ void group_sumsq_df(const X &x, float &S, float &E) {
  warp_tree_node<0, 1>(x, S, E);
}
// The source row of head vector hv of the flat index space (q heads, k heads, v heads).
template <class A>
__device__ __forceinline__ auto head_src(const A &a, unsigned hv, unsigned nq, unsigned nk) {
  constexpr int D = 128;
  return hv < nq ? a.q + (size_t)hv * D
                 : (hv < nq + nk ? a.k + (size_t)(hv - nq) * D : a.v + (size_t)(hv - nq - nk) * D);
}

} // namespace padra
