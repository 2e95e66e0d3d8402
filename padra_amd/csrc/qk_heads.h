// Per-head Q/K RMSNorm + NeoX RoPE, and the KV-cache store of the rotated K row and
// the V row in BF16, q8 or q8_0 form, with two lanes per 128-wide head vector and 32 head
// vectors per wavefront: the fp32-activation path, and the lane-pair encoders the
// store-only kernel (padra_KVStore) uses.  BF16 activations take the four-lane layout of
// qk_quad.h, which builds on the helpers here.
//
// Reference: QKNormRopeStoreControlled (qk_rope_store_exact.cuh:4-49), QKNormRope
// (qknorm_rope.cuh:4-50), QKNormRopePair64 (qknorm_rope_pair64.cuh:3-83).  The reference
// block has 128 threads, one feature each; warp w (features 32w..32w+31) reduces its
// squares with a shuffle-down tree and the four warp partials reduce as
// ((w0 + w2) + (w1 + w3)).  Here lane `half` of a pair holds the features of warps
// `half` and `half + 2` (features 32*half + i and 64 + 32*half + i, i < 32), so:
//  - each warp's whole tree runs inside one lane;
//  - w0 + w2 and w1 + w3 are also in-lane, and the last fold is one lane exchange;
//  - every RoPE pair (i, i + 64) is in one lane, with no exchange at all.
// The first tree level adds two squares with zero error terms; it is written out
// directly (its error fold is an exact no-op).
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
__device__ __forceinline__ void load32(const T *p, float (&x)[32]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float c[8];
    ActIO<T>::load8(p + 8 * m, c);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      x[8 * m + i] = c[i];
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
// The reference encodes K and V of a head in one warp (kv_q8.cuh:41-73,
// kv_q8_native.cuh:70-100); here they are encoded by different waves, so when one of them
// is invalid (non-finite input, the error flag is raised) the other is still written.
template <int FMT, bool ISV, class A>
__device__ __forceinline__ void encode_head_q(const A &a, float (&xa)[32], float (&xb)[32],
                                              long long slot, int h, int half) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  bool invalid = false;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    invalid |= !isfinite(xa[i]) || !isfinite(xb[i]);
    if constexpr (FMT == PADRA_KV_Q8) // q8 also rejects values that are not BF16-exact
      invalid |= (__float_as_uint(xa[i]) & 0xffffu) != 0 || (__float_as_uint(xb[i]) & 0xffffu) != 0;
  }
  invalid = invalid || __shfl_xor((int)invalid, 1, 64);
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
    int8_t *codes = static_cast<int8_t *>(ISV ? a.vc : a.kc) + slot * features + h * D;
    const float inverse = 1.f / scale;
    const bool fast = q8_fast_ok(scale); // pair-uniform
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w0[i] = w1[i] = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        w0[i] |= (fast ? q8_code_fast(xa[4 * i + b], scale, inverse) : q8_code(xa[4 * i + b], scale)) << (8 * b);
        w1[i] |= (fast ? q8_code_fast(xb[4 * i + b], scale, inverse) : q8_code(xb[4 * i + b], scale)) << (8 * b);
      }
    }
    store_codes32(codes + 32 * half, w0);
    store_codes32(codes + 64 + 32 * half, w1);
    if (half == 0)
      reinterpret_cast<float *>(a.scales)[(slot * a.hkv + h) * 2 + (ISV ? 1 : 0)] = scale;
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      // q8_native::Rotate (kv_q8_native.cuh:22-45): stages on feature bits 0..4 in lane,
      // bit 5 across the pair, and for K bit 6 between the lane's two groups.
      hadamard32(xa);
      hadamard32(xb);
      hadamard_cross(xa, half);
      hadamard_cross(xb, half);
      if constexpr (!ISV) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const float lower = xa[i], upper = xb[i];
          xa[i] = (lower + upper) * .08838834764831845f;
          xb[i] = (lower - upper) * .08838834764831845f;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          xa[i] = xa[i] * .125f;
          xb[i] = xb[i] * .125f;
        }
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
    const int stop = min(mine, __shfl_xor(mine, 1, 64)); // first failing block, 4 = none
    if (stop < 4 && half == 0)
      raise_bad(a.bad);
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    uint8_t *row = static_cast<uint8_t *>(ISV ? a.vc : a.kc) + slot * row_bytes;
    int8_t *qs = reinterpret_cast<int8_t *>(row + 2 * (features / 32) + h * D);
    uint16_t *d = reinterpret_cast<uint16_t *>(row) + h * 4;
    const float ai = ad == 0.f ? 0.f : 1.f / ad, bi = bd == 0.f ? 0.f : 1.f / bd;
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w0[i] = w1[i] = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        w0[i] |= q8_0_code(xa[4 * i + b], ai) << (8 * b);
        w1[i] |= q8_0_code(xb[4 * i + b], bi) << (8 * b);
      }
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

// One wave = 32 head vectors, two lanes each (the fp32-activation path).  The flat index
// space is the T*Hq query heads, then the T*Hkv key heads, then (with a cache binding) the
// T*Hkv value heads, whose lanes only move the V row into the cache.
//
// The wave's 32 heads (16 KB of fp32) move through an LDS image: sixteen coalesced 1 KB
// loads per lane in, each lane reads its two 128-byte halves (features 32*half .. and
// 64 + 32*half ..), and the rotated query and key heads go back through the image to
// sixteen coalesced 1 KB stores.  (Reading the halves straight from memory, each
// instruction touched 64 separate 16-byte pieces 128 or 512 bytes apart: 47 us for a
// 2048-token chunk, against 10 us through the image.)  Chunk ci (16 bytes) of head jj sits
// at slot 32*jj + ((ci + jj) & 31): both the transposing writes and the half reads are
// free of bank conflicts.
__device__ __forceinline__ int direct_slot(int jj, int ci) { return 32 * jj + ((ci + jj) & 31); }

template <class T, int FMT>
__device__ __forceinline__ void qk_heads_wave_direct(const QKArgs<T> &a, long long wave,
                                                     uint4 *image) {
  static_assert(std::is_same<T, float>::value, "BF16 activations take the quad layout");
  constexpr int D = 128;
  __shared__ int head_live[32]; // 1: the head's rotated values go back to its activation
  const int lane = threadIdx.x & 63, half = lane & 1, jj = lane >> 1;
  const unsigned block0 = (unsigned)wave * 32u;
  const unsigned hv = block0 + (unsigned)jj;
  const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned total = nq + nk + (FMT >= 0 ? nk : 0u);
  const bool live = hv < total;
  const int role = hv < nq ? 0 : (hv < nq + nk ? 1 : 2); // 0 q, 1 k, 2 v
  const unsigned idx = role == 0 ? hv : (role == 1 ? hv - nq : hv - nq - nk);
  const unsigned heads = role == 0 ? (unsigned)a.hq : (unsigned)a.hkv;
  const int t = live ? (int)(idx / heads) : 0, h = live ? (int)(idx % heads) : 0;
  const PosState ps = fetch_state(a.pos, t);
  auto src_of = [&](unsigned hc) -> const float * {
    return hc < nq ? a.q + (size_t)hc * D
                   : (hc < nq + nk ? a.k + (size_t)(hc - nq) * D : a.v + (size_t)(hc - nq - nk) * D);
  };

  // 1. The block into the image: sixteen 1 KB loads per lane, in two batches of eight.
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    uint4 in[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int c = 64 * (8 * b + m) + lane;
      const unsigned hc = min(block0 + (unsigned)(c >> 5), total - 1u);
      in[m] = ld_nt(reinterpret_cast<const uint4 *>(src_of(hc)) + (c & 31));
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int c = 64 * (8 * b + m) + lane;
      image[direct_slot(c >> 5, c & 31)] = in[m];
    }
  }
  bool ok = false;
  const int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first,
                                   FMT > PADRA_KV_BF16, ok);
  ok = ok && live && pos >= 0 && pos < a.table_rows;
  if (live && !ok && half == 0)
    raise_bad(a.bad);
  __syncthreads();
  // This lane's halves: chunks 8*half .. (xa) and 16 + 8*half .. (xb) of its head.
  Act32<T> xa, xb;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const uint4 va = image[direct_slot(jj, 8 * half + p)];
    const uint4 vb = image[direct_slot(jj, 16 + 8 * half + p)];
    xa.f[p] = make_float4(__uint_as_float(va.x), __uint_as_float(va.y), __uint_as_float(va.z),
                          __uint_as_float(va.w));
    xb.f[p] = make_float4(__uint_as_float(vb.x), __uint_as_float(vb.y), __uint_as_float(vb.z),
                          __uint_as_float(vb.w));
  }
  const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
  const long long slot = seq * a.seq_stride + (ok ? ring_slot(pos, max(a.cap, 1)) : 0);
  bool store_act = false;
  uint32_t lo[16], hi[16];

  if (FMT >= 0 && role == 2) {
    // V row: the unchanged values go to the cache (StorePrefillControlled,
    // prefill_control.cuh:36-37; QKNormRopeStoreControlled, qk_rope_store_exact.cuh:47).
    if constexpr (FMT >= 0) {
      if (ok && t >= a.first) {
        if constexpr (FMT == PADRA_KV_BF16) {
          uint16_t *vc = static_cast<uint16_t *>(a.vc) + slot * (a.hkv * D) + h * D;
          uint32_t pa[16], pb[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            pa[i] = pack2(xa.get(2 * i), xa.get(2 * i + 1));
            pb[i] = pack2(xb.get(2 * i), xb.get(2 * i + 1));
          }
          store32_bf16(vc + 32 * half, pa);
          store32_bf16(vc + 64 + 32 * half, pb);
        } else {
          float fa[32], fb[32];
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            fa[i] = xa.get(i);
            fb[i] = xb.get(i);
          }
          encode_head_q<FMT, true>(a, fa, fb, slot, h, half);
        }
      }
    }
  } else if (ok) {
    const bool isk = role == 1;
    const uint16_t *w = isk ? a.kn : a.qn;
    const uint16_t *row = a.table + (size_t)pos * D;

    float S, E, S2, E2;
    group_sumsq(xa, S, E);
    group_sumsq(xb, S2, E2);
    fold(S2, E2, S, E); // w_half + w_{half+2}
    const float So = shfl_xor(S, 1), Eo = shfl_xor(E, 1);
    float bs = half ? So : S, be = half ? Eo : E;
    fold(half ? S : So, half ? E : Eo, bs, be); // (w0 + w2) + (w1 + w3)
    const float sum = bs + be;
    const float inv = 1.f / sqrtf(sum / (float)D + a.eps);

    // Normalize and rotate pairs (i, i + 64), eight at a time: every BF16 rounding of the
    // reference is one half of a packed conversion of the pair.
    bool fine = isfinite(sum);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      Bf8 wa, wb, c8, s8;
      wa.load(w + 32 * half + 8 * m);
      wb.load(w + 64 + 32 * half + 8 * m);
      c8.load(row + 32 * half + 8 * m);
      s8.load(row + 64 + 32 * half + 8 * m);
#pragma unroll
      for (int q = 0; q < 8; q += 2) {
        float l2[2], h2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i = 8 * m + q + u;
          const uint32_t p1 = pack2(xa.get(i) * inv, xb.get(i) * inv);
          const uint32_t p2 = pack2(lo16(p1) * wa.get(q + u), hi16(p1) * wb.get(q + u));
          const float A = lo16(p2), Bv = hi16(p2), c = c8.get(q + u), sn = s8.get(q + u);
          const uint32_t p3 = pack2(A * c, Bv * c);
          const uint32_t p4 = pack2((-Bv) * sn, A * sn);
          l2[u] = lo16(p3) + lo16(p4);
          h2[u] = hi16(p3) + hi16(p4);
          fine = fine && bf16_finite_after_round(l2[u]) && bf16_finite_after_round(h2[u]);
        }
        lo[(8 * m + q) / 2] = pack2(l2[0], l2[1]);
        hi[(8 * m + q) / 2] = pack2(h2[0], h2[1]);
      }
    }
    store_act = true;
    if (!fine)
      raise_bad(a.bad);

    if constexpr (FMT >= 0) {
      if (isk && t >= a.first) {
        if constexpr (FMT == PADRA_KV_BF16) {
          uint16_t *kc = static_cast<uint16_t *>(a.kc) + slot * (a.hkv * D) + h * D;
          store32_bf16(kc + 32 * half, lo);
          store32_bf16(kc + 64 + 32 * half, hi);
        } else {
          float ka[32], kb[32];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            ka[2 * i] = lo16(lo[i]);
            ka[2 * i + 1] = hi16(lo[i]);
            kb[2 * i] = lo16(hi[i]);
            kb[2 * i + 1] = hi16(hi[i]);
          }
          encode_head_q<FMT, false>(a, ka, kb, slot, h, half);
        }
      }
    }
  }

  // 2. Rotated query and key heads back through the image (as fp32), then sixteen 1 KB
  // stores per lane.  Each lane rewrites only the slots it read.
  if (store_act) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t *l = lo + 4 * p, *g = hi + 4 * p;
      image[direct_slot(jj, 8 * half + 2 * p)] =
          make_uint4(l[0] << 16, l[0] & 0xffff0000u, l[1] << 16, l[1] & 0xffff0000u);
      image[direct_slot(jj, 8 * half + 2 * p + 1)] =
          make_uint4(l[2] << 16, l[2] & 0xffff0000u, l[3] << 16, l[3] & 0xffff0000u);
      image[direct_slot(jj, 16 + 8 * half + 2 * p)] =
          make_uint4(g[0] << 16, g[0] & 0xffff0000u, g[1] << 16, g[1] & 0xffff0000u);
      image[direct_slot(jj, 16 + 8 * half + 2 * p + 1)] =
          make_uint4(g[2] << 16, g[2] & 0xffff0000u, g[3] << 16, g[3] & 0xffff0000u);
    }
  }
  if (half == 0)
    head_live[jj] = store_act ? 1 : 0;
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int c = 64 * m + lane, j = c >> 5;
    if (!head_live[j])
      continue;
    const unsigned hc = block0 + (unsigned)j;
    float *dst = const_cast<float *>(src_of(hc));
    st_nt(reinterpret_cast<uint4 *>(dst) + (c & 31), image[direct_slot(j, c & 31)]);
  }
}

// The source row of head vector hv of the flat index space (q heads, k heads, v heads).
template <class A>
__device__ __forceinline__ const uint16_t *head_src(const A &a, unsigned hv, unsigned nq,
                                                    unsigned nk) {
  constexpr int D = 128;
  return hv < nq ? a.q + (size_t)hv * D
                 : (hv < nq + nk ? a.k + (size_t)(hv - nq) * D : a.v + (size_t)(hv - nq - nk) * D);
}

} // namespace padra
