// Per-head Q/K RMSNorm + NeoX RoPE, and the KV-cache store of the rotated K row and
// the V row in BF16, q8 or q8_0 form.  Two lanes per 128-wide head vector, 32 head
// vectors per wavefront.
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

// q8 code (kv_q8.cuh:12-14): RNE of the correctly rounded quotient, clamped to +-127.
__device__ __forceinline__ uint32_t q8_code(float value, float scale) {
  const int c = max(-127, min(127, (int)rintf(value / scale)));
  return (uint32_t)(c & 0xff);
}
// q8_0 code (kv_q8_native.cuh:46-48): roundf (half away from zero) of v * inverse.
__device__ __forceinline__ uint32_t q8_0_code(float value, float inverse) {
  const int c = max(-127, min(127, (int)roundf(value * inverse)));
  return (uint32_t)(c & 0xff);
}
__device__ __forceinline__ void store_codes32(int8_t *p, const uint32_t (&w)[8]) {
  reinterpret_cast<uint4 *>(p)[0] = make_uint4(w[0], w[1], w[2], w[3]);
  reinterpret_cast<uint4 *>(p)[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

template <class T, int FMT>
__device__ __forceinline__ void qk_heads_wave(const QKArgs<T> &a, long long wave) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, half = lane & 1;
  const long long hv = wave * 32 + (lane >> 1);
  const long long nq = (long long)a.tokens * a.hq;
  const long long total = nq + (long long)a.tokens * a.hkv;
  if (hv >= total)
    return; // both lanes of a pair leave together
  const bool isk = hv >= nq;
  const long long kvi = hv - nq;
  const int t = isk ? (int)(kvi / a.hkv) : (int)(hv / a.hq);
  const int h = isk ? (int)(kvi % a.hkv) : (int)(hv % a.hq);
  T *const base = isk ? a.k + kvi * D : a.q + hv * D;

  bool ok;
  const int pos = resolve_position(a.pos, t, FMT >= 0 ? a.cap : 0, a.first,
                                   FMT > PADRA_KV_BF16, ok);
  if (!ok || pos < 0 || pos >= a.table_rows) {
    if (half == 0)
      raise_bad(a.bad);
    return;
  }

  float xa[32], xb[32];
  load32<T>(base + 32 * half, xa);
  load32<T>(base + 64 + 32 * half, xb);
  float S, E, S2, E2;
  warp_sumsq32(xa, S, E);
  warp_sumsq32(xb, S2, E2);
  fold(S2, E2, S, E); // w_half + w_{half+2}
  const float So = shfl_xor(S, 1), Eo = shfl_xor(E, 1);
  float bs = half ? So : S, be = half ? Eo : E;
  fold(half ? S : So, half ? E : Eo, bs, be); // (w0 + w2) + (w1 + w3)
  const float sum = bs + be;
  const float inv = 1.f / sqrtf(sum / (float)D + a.eps);

  const uint16_t *w = isk ? a.kn : a.qn;
  const uint16_t *row = a.table + (size_t)pos * D;
  uint32_t lo[16], hi[16];
  bool fine = true;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float wa[8], wb[8], c[8], sn[8];
    load8_bf16(w + 32 * half + 8 * m, wa);
    load8_bf16(w + 64 + 32 * half + 8 * m, wb);
    load8_bf16(row + 32 * half + 8 * m, c);
    load8_bf16(row + 64 + 32 * half + 8 * m, sn);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float l2[2], h2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 8 * m + 2 * p + u, ii = 2 * p + u;
        const float A = B(B(xa[i] * inv) * wa[ii]);
        const float Bv = B(B(xb[i] * inv) * wb[ii]);
        l2[u] = B(A * c[ii]) + B((-Bv) * sn[ii]);
        h2[u] = B(Bv * c[ii]) + B(A * sn[ii]);
        fine = fine && bf16_finite_after_round(l2[u]) && bf16_finite_after_round(h2[u]);
      }
      lo[4 * m + p] = pack2(l2[0], l2[1]);
      hi[4 * m + p] = pack2(h2[0], h2[1]);
    }
  }
  store32<T>(base + 32 * half, lo);
  store32<T>(base + 64 + 32 * half, hi);
  if (!fine)
    raise_bad(a.bad);

  if constexpr (FMT >= 0) {
    if (!isk || t < a.first)
      return;
    const int features = a.hkv * D;
    const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
    const long long slot = seq * a.seq_stride + pos % a.cap;
    const T *vsrc = a.v + kvi * D;
    if constexpr (FMT == PADRA_KV_BF16) {
      uint16_t *kc = static_cast<uint16_t *>(a.kc) + slot * features + h * D;
      uint16_t *vc = static_cast<uint16_t *>(a.vc) + slot * features + h * D;
      store32_bf16(kc + 32 * half, lo);
      store32_bf16(kc + 64 + 32 * half, hi);
      float va[32], vb[32];
      load32<T>(vsrc + 32 * half, va);
      load32<T>(vsrc + 64 + 32 * half, vb);
      uint32_t pa[16], pb[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pa[i] = pack2(va[2 * i], va[2 * i + 1]);
        pb[i] = pack2(vb[2 * i], vb[2 * i + 1]);
      }
      store32_bf16(vc + 32 * half, pa);
      store32_bf16(vc + 64 + 32 * half, pb);
    } else {
      // Rotated K (BF16-exact) and V values of this lane's two feature groups.
      float ka[32], kb[32], va[32], vb[32];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        ka[2 * i] = lo16(lo[i]);
        ka[2 * i + 1] = hi16(lo[i]);
        kb[2 * i] = lo16(hi[i]);
        kb[2 * i + 1] = hi16(hi[i]);
      }
      load32<T>(vsrc + 32 * half, va);
      load32<T>(vsrc + 64 + 32 * half, vb);
      // The encoders reject heads with non-finite values (kv_q8.cuh:49-54,
      // kv_q8_native.cuh:79-83); q8 also rejects values that are not BF16-exact.
      bool invalid = false;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        invalid |= !isfinite(ka[i]) || !isfinite(kb[i]) || !isfinite(va[i]) || !isfinite(vb[i]);
        if constexpr (FMT == PADRA_KV_Q8)
          invalid |= (__float_as_uint(va[i]) & 0xffffu) != 0 ||
                     (__float_as_uint(vb[i]) & 0xffffu) != 0;
      }
      invalid = invalid || __shfl_xor((int)invalid, 1, 64);
      if (invalid) {
        if (half == 0)
          raise_bad(a.bad);
        return;
      }
      if constexpr (FMT == PADRA_KV_Q8) {
        float km = 0.f, vm = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          km = fmaxf(km, fmaxf(fabsf(ka[i]), fabsf(kb[i])));
          vm = fmaxf(vm, fmaxf(fabsf(va[i]), fabsf(vb[i])));
        }
        km = fmaxf(km, shfl_xor(km, 1));
        vm = fmaxf(vm, shfl_xor(vm, 1));
        const float ks = km == 0.f ? 1.f : km / 127.f, vs = vm == 0.f ? 1.f : vm / 127.f;
        int8_t *ck = static_cast<int8_t *>(a.kc) + slot * features + h * D;
        int8_t *cv = static_cast<int8_t *>(a.vc) + slot * features + h * D;
        uint32_t w0[8], w1[8], w2[8], w3[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          w0[i] = w1[i] = w2[i] = w3[i] = 0u;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            w0[i] |= q8_code(ka[4 * i + b], ks) << (8 * b);
            w1[i] |= q8_code(kb[4 * i + b], ks) << (8 * b);
            w2[i] |= q8_code(va[4 * i + b], vs) << (8 * b);
            w3[i] |= q8_code(vb[4 * i + b], vs) << (8 * b);
          }
        }
        store_codes32(ck + 32 * half, w0);
        store_codes32(ck + 64 + 32 * half, w1);
        store_codes32(cv + 32 * half, w2);
        store_codes32(cv + 64 + 32 * half, w3);
        if (half == 0)
          reinterpret_cast<padra_Q8KVScalePair *>(a.scales)[slot * a.hkv + h] = {ks, vs};
      } else {
        if constexpr (FMT == PADRA_KV_Q8_0) {
          // K: 128-point transform, stages bit 0..4 in lane, bit 5 across the pair,
          // bit 6 between the lane's two groups; V: two 64-point transforms (bits 0..5).
          hadamard32(ka);
          hadamard32(kb);
          hadamard_cross(ka, half);
          hadamard_cross(kb, half);
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            const float lower = ka[i], upper = kb[i];
            ka[i] = (lower + upper) * .08838834764831845f;
            kb[i] = (lower - upper) * .08838834764831845f;
          }
          hadamard32(va);
          hadamard32(vb);
          hadamard_cross(va, half);
          hadamard_cross(vb, half);
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            va[i] = va[i] * .125f;
            vb[i] = vb[i] * .125f;
          }
        }
        // Blocks: this lane holds block `half` (ka, va) and block `half + 2` (kb, vb).
        float kam = 0.f, kbm = 0.f, vam = 0.f, vbm = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          kam = fmaxf(kam, fabsf(ka[i]));
          kbm = fmaxf(kbm, fabsf(kb[i]));
          vam = fmaxf(vam, fabsf(va[i]));
          vbm = fmaxf(vbm, fabsf(vb[i]));
        }
        const float kad = kam / 127.f, kbd = kbm / 127.f, vad = vam / 127.f, vbd = vbm / 127.f;
        const __half kah = __float2half(kad), kbh = __float2half(kbd);
        const __half vah = __float2half(vad), vbh = __float2half(vbd);
        // A failing block stops the reference at that block (kv_q8_native.cuh:84-96):
        // blocks before the first failing one are written, later ones are not.
        const bool fa = !isfinite(kam) || !isfinite(vam) || !isfinite(__half2float(kah)) ||
                        !isfinite(__half2float(vah));
        const bool fb = !isfinite(kbm) || !isfinite(vbm) || !isfinite(__half2float(kbh)) ||
                        !isfinite(__half2float(vbh));
        const int mine = fa ? half : (fb ? half + 2 : 4);
        const int stop = min(mine, __shfl_xor(mine, 1, 64)); // first failing block, 4 = none
        if (stop < 4 && half == 0)
          raise_bad(a.bad);
        const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
        uint8_t *rk = static_cast<uint8_t *>(a.kc) + slot * row_bytes;
        uint8_t *rv = static_cast<uint8_t *>(a.vc) + slot * row_bytes;
        int8_t *qk = reinterpret_cast<int8_t *>(rk + 2 * (features / 32) + h * D);
        int8_t *qv = reinterpret_cast<int8_t *>(rv + 2 * (features / 32) + h * D);
        uint16_t *dk = reinterpret_cast<uint16_t *>(rk) + h * 4;
        uint16_t *dv = reinterpret_cast<uint16_t *>(rv) + h * 4;
        const float kai = kad == 0.f ? 0.f : 1.f / kad, kbi = kbd == 0.f ? 0.f : 1.f / kbd;
        const float vai = vad == 0.f ? 0.f : 1.f / vad, vbi = vbd == 0.f ? 0.f : 1.f / vbd;
        uint32_t w0[8], w1[8], w2[8], w3[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          w0[i] = w1[i] = w2[i] = w3[i] = 0u;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            w0[i] |= q8_0_code(ka[4 * i + b], kai) << (8 * b);
            w1[i] |= q8_0_code(kb[4 * i + b], kbi) << (8 * b);
            w2[i] |= q8_0_code(va[4 * i + b], vai) << (8 * b);
            w3[i] |= q8_0_code(vb[4 * i + b], vbi) << (8 * b);
          }
        }
        const uint16_t ka16 = __half_as_ushort(kah), kb16 = __half_as_ushort(kbh);
        const uint16_t va16 = __half_as_ushort(vah), vb16 = __half_as_ushort(vbh);
        if (stop == 4) {
          // Gather the four block scales of the head into lane 0 of the pair: one 8-byte
          // store per tensor.
          const uint32_t kmine = (uint32_t)ka16 | ((uint32_t)kb16 << 16);
          const uint32_t vmine = (uint32_t)va16 | ((uint32_t)vb16 << 16);
          const uint32_t kother = __shfl_xor(kmine, 1, 64), vother = __shfl_xor(vmine, 1, 64);
          if (half == 0) {
            // d[0] = block 0 (lane 0, a), d[1] = block 1 (lane 1, a), d[2], d[3] the b's.
            const uint2 kd = make_uint2((kmine & 0xffffu) | (kother << 16),
                                        (kmine >> 16) | (kother & 0xffff0000u));
            const uint2 vd = make_uint2((vmine & 0xffffu) | (vother << 16),
                                        (vmine >> 16) | (vother & 0xffff0000u));
            *reinterpret_cast<uint2 *>(dk) = kd;
            *reinterpret_cast<uint2 *>(dv) = vd;
          }
          store_codes32(qk + 32 * half, w0);
          store_codes32(qk + 64 + 32 * half, w1);
          store_codes32(qv + 32 * half, w2);
          store_codes32(qv + 64 + 32 * half, w3);
        } else {
          if (half < stop) {
            dk[half] = ka16;
            dv[half] = va16;
            store_codes32(qk + 32 * half, w0);
            store_codes32(qv + 32 * half, w2);
          }
          if (half + 2 < stop) {
            dk[half + 2] = kb16;
            dv[half + 2] = vb16;
            store_codes32(qk + 64 + 32 * half, w1);
            store_codes32(qv + 64 + 32 * half, w3);
          }
        }
      }
    }
  }
}

} // namespace padra
