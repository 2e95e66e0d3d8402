// Decode attention over a BF16 or q8 KV cache: split-K partial softmax, then a per-head merge.
//
// Reference: gqa8_fragment_validation::SplitBF16 (attention_gqa8_fragment_validation.cuh:
// 79-214) with attention_perhead_exact::Merge (attention_perhead_exact.cuh:7-38); for q8
// caches gqa8_q8_attention::SplitBF16 (attention_gqa8_q8.cuh:112-277), which reads the
// tiles through kv_q8::Decode.  Any number of query heads per KV head up to 8 (the
// reference fixes 8).  One token per sequence, at its DecodeState position; keys are the
// last n positions (n = position + 1, or at most 1024 for a local ring), read from cache
// row (first + offset) % cap.
//
// Split kernel (k_attn_mx): one wave per (sequence, KV head, split), over that split's
// 32-key tiles, QK and PV on the matrix cores; the reference's online softmax per row
// (tile maximum, fp32 probabilities for the denominator fmaf(den, alpha, total), BF16
// probabilities for the PV product, scale 1/sqrt(128) applied after the dot product).
// Merge kernel: one wave per (sequence, query head): weights exp(lse_s - max) / sum, then
// out = B(sum_s w_s * partial_s) in split order.
//
// Not bit-identical to the reference: its QK and PV products run on tensor-core MMA with an
// unspecified accumulation order, and its expf/logf are CUDA's.  Products of two BF16
// values are exact in fp32, so only the order of the fp32 sums and the exp/log ulps differ.
#include <stdio.h>

#include <algorithm>

#include "common.h"

using namespace padra;

namespace {

constexpr int kD = 128, kKeys = 32;
constexpr float kScoreScale = .08838834764831845f;

int launched(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fprintf(stderr, "padra: %s launch failed: %s\n", what, hipGetErrorString(e));
    return PADRA_INTERNAL;
  }
  return PADRA_OK;
}
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct AttnArgs {
  const void *q; // [seqs][hq][128], activation type
  const uint16_t *kc, *vc;
  void *out; // [seqs][hq][128]
  float *partial, *lse;
  const padra_DecodeState *decode;
  int seqs, hq, hkv, cap, local, splits, maximum, vocab;
  long long seq_stride; // cache rows between sequences
  int *bad;
  // q8_0 caches: the coded query (int8 [seqs][hq][128]) and its block scales
  // (fp32 [seqs][hq][4]), both in the scratch.
  int8_t *qcodes;
  float *qscale;
  const float *kvscales; // q8 caches: (k, v) scale pair per row and KV head
};

// The sequence's admission and key window (Admitted, attention_gqa8_fragment_validation.cuh:
// 49-55, with the split count a parameter): n keys from position `first`.
__device__ __forceinline__ bool attn_window(const AttnArgs &a, int seq, int &n, int &first) {
  const padra_DecodeState st = load_state(a.decode + seq);
  const bool ok = decode_ready(st, a.maximum, a.vocab) && a.cap <= st.capacity &&
                  (a.local ? a.cap == min(1024, st.capacity) : a.cap == st.capacity);
  n = a.local ? min(st.position + 1, 1024) : st.position + 1;
  first = st.position + 1 - n;
  return ok;
}

__device__ __forceinline__ float xor_max32(float v) {
#pragma unroll
  for (int d = 16; d >= 1; d /= 2)
    v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}
__device__ __forceinline__ float xor_sum32(float v) {
#pragma unroll
  for (int d = 16; d >= 1; d /= 2)
    v = v + __shfl_xor(v, d, 64);
  return v;
}

template <class T> __device__ __forceinline__ float act_value(const void *p, size_t i) {
  if constexpr (std::is_same<T, uint16_t>::value)
    return __uint_as_float((uint32_t) static_cast<const uint16_t *>(p)[i] << 16);
  else
    return static_cast<const float *>(p)[i];
}

// ---- Split kernel on the matrix cores --------------------------------------------------
// QK and PV on v_mfma_f32_16x16x32_bf16 (the reference runs both on tensor-core MMA).  One
// wave per (sequence, KV head, split); query rows are the 16 MFMA columns (rows past G are
// zero).
//  - QK: S[key][row] = K[key][:] . Q[row][:] for the tile's two 16-key halves, 4 K-steps of
//    32 dimensions each.  Lane l then holds row l % 16, keys 16 h + 4 (l / 16) + i.
//  - Softmax: the row's tile maximum and probability sum are the lane's 8 values plus two
//    exchanges between the four lanes of the row.
//  - PV: O[row][dim] += P[row][key] V[key][dim] with P straight from the score registers
//    (K-slot i of lane group g is key 4g + i, then 16 + 4g + i - 4) and V staged in LDS as
//    4-key groups per dimension, so that each B operand is two 8-byte LDS reads.  Lane l
//    holds rows 4 (l / 16) + i of dimension 16 b + l % 16.
//  - The accumulators are rescaled only when some row's maximum moved (alpha == 1 exactly
//    otherwise).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Whether every code * scale of a q8 row is finite in BF16 and the scale is valid; rows
// that fail it (huge or invalid scales) check each decoded value instead.
__device__ __forceinline__ bool q8_scale_fast(float scale) {
  return scale > 0.f && (pack2(127.f * scale, 0.f) & 0x7f80u) != 0x7f80u;
}

// 16 codes (4 words) of one row: nonzero when a byte is 0x80 (code -128), from the
// zero-byte test of the words with the sign bits flipped.
__device__ __forceinline__ uint32_t q8_minus128(uint4 c) {
  const uint32_t x0 = c.x ^ 0x80808080u, x1 = c.y ^ 0x80808080u, x2 = c.z ^ 0x80808080u,
                 x3 = c.w ^ 0x80808080u;
  return (((x0 - 0x01010101u) & ~x0) | ((x1 - 0x01010101u) & ~x1) | ((x2 - 0x01010101u) & ~x2) |
          ((x3 - 0x01010101u) & ~x3)) &
         0x80808080u;
}

// The 16 values code * scale of a code chunk (kv_q8::Decode), and with `fine` cleared when
// the row's scale fails q8_scale_fast and a value is not finite in BF16 (or the scale is
// invalid).  Keys past the window decode zero codes with a unit scale, as the reference
// stages them.
__device__ __forceinline__ void q8_values16(uint4 c, float scale, bool inside, float (&f)[16],
                                            uint32_t &m128, bool &fine) {
  if (!inside) {
    c = make_uint4(0, 0, 0, 0);
    scale = 1.f;
  }
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      f[4 * i + b] = (float)(int8_t)((w[i] >> (8 * b)) & 0xffu) * scale;
  m128 |= q8_minus128(c);
  if (!q8_scale_fast(scale)) {
    bool ok = isfinite(scale) && scale > 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      ok = ok && (pack2(f[e], 0.f) & 0x7f80u) != 0x7f80u;
    fine = fine && ok;
  }
}

template <int G, class T, bool Q8>
__global__ __launch_bounds__(64) void k_attn_mx(AttnArgs a) {
  constexpr int KW = kD / 2 + 4; // K row stride in words (padding spreads the banks)
  constexpr int VW = kD + 16;    // V group stride in uint2
  __shared__ uint32_t ks[kKeys][KW];
  __shared__ uint2 vq[kKeys / 4][VW]; // (V[4j][d], V[4j+1][d]), (V[4j+2][d], V[4j+3][d])
  const int split = blockIdx.x, kv = blockIdx.y, seq = blockIdx.z, lane = threadIdx.x;
  const int col = lane & 15, grp = lane >> 4;
  int n, first;
  if (!attn_window(a, seq, n, first)) {
    if (split == 0 && kv == 0 && lane == 0)
      raise_bad(a.bad);
    return;
  }
  const int tiles = (n + kKeys - 1) / kKeys, active = min(a.splits, tiles);
  if (split >= active)
    return; // block-uniform
  const int begin = tiles * split / active, end = tiles * (split + 1) / active;
  const int features = a.hkv * kD;
  const size_t head_off = (size_t)seq * a.seq_stride * features + kv * kD;
  const uint16_t *kc = a.kc + head_off, *vc = a.vc + head_off;
  const int8_t *k8 = reinterpret_cast<const int8_t *>(a.kc) + head_off;
  const int8_t *v8 = reinterpret_cast<const int8_t *>(a.vc) + head_off;
  const float2 *sc = reinterpret_cast<const float2 *>(a.kvscales) +
                     (size_t)seq * a.seq_stride * a.hkv + kv;

  // Query operand: row col (zero past G), dimensions 32 t + 8 grp + e; finite and
  // BF16-exact, as the reference requires of its fp32 input.
  uint4 qb[4];
  bool fine = true;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t w[4] = {0, 0, 0, 0};
    if (col < G) {
      const size_t o = ((size_t)seq * a.hq + kv * G + col) * kD + 32 * t + 8 * grp;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = act_value<T>(a.q, o + 2 * e), x1 = act_value<T>(a.q, o + 2 * e + 1);
        fine = fine && isfinite(x0) && isfinite(x1) && (__float_as_uint(x0) & 0xffffu) == 0 &&
               (__float_as_uint(x1) & 0xffffu) == 0;
        w[e] = (__float_as_uint(x0) >> 16) | (__float_as_uint(x1) & 0xffff0000u);
      }
    }
    qb[t] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
  fine = true;

  // Tile loads, each instruction covering whole rows (256 B BF16 rows on 16 lanes, 128 B q8
  // rows on 8 lanes).  K: key c / 16 (q8: c / 8) of chunk c = lane + 64 m, dimensions in
  // chunk order.  V: lane keeps 4 consecutive keys of the same dimensions:
  //  BF16: m = 4 h + p is key 16 h + 4 grp + p, dimensions 8 col ..;
  //  q8:   m = p is key 4 (lane / 8) + p, dimensions 16 (lane % 8) ...
  // Rows past the window load a valid row and are zeroed (the reference zero-fills them).
  constexpr int CH = Q8 ? 4 : 8;
  float ksc[CH], vsc[CH];
  auto row_of = [&](int tile, int key) {
    const int o = tile * kKeys + key;
    return (size_t)((first + (o < n ? o : 0)) % a.cap);
  };
  auto vkey = [&](int m) { return Q8 ? 4 * (lane >> 3) + m : 16 * (m >> 2) + 4 * grp + (m & 3); };
  auto load_tile = [&](int tile, uint4 (&kw)[8], uint4 (&vw)[8]) {
#pragma unroll
    for (int m = 0; m < CH; ++m) {
      const int c = lane + 64 * m;
      const size_t kr = row_of(tile, c >> (Q8 ? 3 : 4)), vr = row_of(tile, vkey(m));
      if constexpr (Q8) {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(k8 + kr * features) + (c & 7));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(v8 + vr * features) + (lane & 7));
        ksc[m] = sc[kr * a.hkv].x;
        vsc[m] = sc[vr * a.hkv].y;
      } else {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(kc + kr * features) + (c & 15));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(vc + vr * features) + col);
      }
    }
  };

  float maximum = -INFINITY, den = 0.f;
  f32x4_t o[8];
#pragma unroll
  for (int b = 0; b < 8; ++b)
    o[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4 kw[8], vw[8];
  load_tile(begin, kw, vw);
  for (int tile = begin; tile < end; ++tile) {
    const int left = n - tile * kKeys; // keys of this tile inside the window (may be >= 32)
    // Stage K rows and V key groups as BF16.
    if constexpr (Q8) {
      uint32_t m128 = 0;
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        const int c = lane + 64 * m, key = c >> 3, part = c & 7;
        float f[16];
        q8_values16(kw[m], ksc[m], key < left, f, m128, fine);
        uint32_t w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          w[e] = pack2(f[2 * e], f[2 * e + 1]);
        *reinterpret_cast<uint4 *>(&ks[key][part * 8]) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint4 *>(&ks[key][part * 8 + 4]) = make_uint4(w[4], w[5], w[6], w[7]);
      }
      float fv[4][16];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        q8_values16(vw[m], vsc[m], vkey(m) < left, fv[m], m128, fine);
      fine = fine && m128 == 0;
      uint2 *dst = &vq[lane >> 3][16 * (lane & 7)];
#pragma unroll
      for (int e = 0; e < 16; e += 2)
        *reinterpret_cast<uint4 *>(dst + e) =
            make_uint4(pack2(fv[0][e], fv[1][e]), pack2(fv[2][e], fv[3][e]),
                       pack2(fv[0][e + 1], fv[1][e + 1]), pack2(fv[2][e + 1], fv[3][e + 1]));
    } else {
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int c = lane + 64 * m;
        if ((c >> 4) >= left)
          kw[m] = make_uint4(0, 0, 0, 0);
        if (vkey(m) >= left)
          vw[m] = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4 *>(&ks[c >> 4][(c & 15) * 4]) = kw[m];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 *p = &vw[4 * h];
        const uint32_t w0[4] = {p[0].x, p[0].y, p[0].z, p[0].w}, w1[4] = {p[1].x, p[1].y, p[1].z, p[1].w},
                       w2[4] = {p[2].x, p[2].y, p[2].z, p[2].w}, w3[4] = {p[3].x, p[3].y, p[3].z, p[3].w};
        uint2 *dst = &vq[4 * h + grp][8 * col];
#pragma unroll
        for (int e = 0; e < 4; ++e) // dimensions 2e, 2e + 1 of the chunk
          *reinterpret_cast<uint4 *>(dst + 2 * e) = make_uint4(
              __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u),
              __builtin_amdgcn_perm(w3[e], w2[e], 0x05040100u),
              __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u),
              __builtin_amdgcn_perm(w3[e], w2[e], 0x07060302u));
      }
    }
    __syncthreads();
    // The next tile's loads are in flight during this tile's arithmetic (the last tile
    // reloads itself, keeping the loads unconditional).
    load_tile(min(tile + 1, end - 1), kw, vw);

    // Scores: lane holds row col, keys 16 h + 4 grp + i.
    f32x4_t s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s[h] = mfma_bf16(*reinterpret_cast<const uint4 *>(&ks[16 * h + col][16 * t + 4 * grp]),
                         qb[t], s[h]);
    }
    float sv[8], tmax = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = s[h][i] * kScoreScale;
        if (16 * h + 4 * grp + i < left)
          fine = fine && isfinite(v);
        else
          v = -INFINITY;
        sv[4 * h + i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float next = fmaxf(maximum, tmax);
    const float alpha = isfinite(maximum) ? expf(maximum - next) : 0.f;
    float p[8], total = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      p[k] = isfinite(sv[k]) ? expf(sv[k] - next) : 0.f;
      total += p[k];
    }
    total += __shfl_xor(total, 16, 64);
    total += __shfl_xor(total, 32, 64);
    den = __builtin_fmaf(den, alpha, total);
    maximum = next;
    const uint4 pa = make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]),
                                pack2(p[6], p[7]));
    if (__ballot(alpha != 1.f) != 0) { // wave-uniform
      float ar[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ar[i] = __shfl(alpha, 4 * grp + i, 64);
#pragma unroll
      for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[b][i] *= ar[i];
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint2 v0 = vq[grp][16 * b + col], v1 = vq[4 + grp][16 * b + col];
      o[b] = mfma_bf16(pa, make_uint4(v0.x, v0.y, v1.x, v1.y), o[b]);
    }
    __syncthreads();
  }
  // Rows 4 grp + i: this lane's dimension 16 b + col of each.
  const int head0 = kv * G;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * grp + i;
    const float d = __shfl(den, r, 64), mx = __shfl(maximum, r, 64);
    if (r < G) {
      float *dst = a.partial + (((size_t)seq * a.splits + split) * a.hq + head0 + r) * kD + col;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const float v = o[b][i] / d;
        fine = fine && isfinite(v);
        dst[16 * b] = v;
      }
      if (col == 0) {
        const float l = mx + logf(d);
        fine = fine && isfinite(l);
        a.lse[((size_t)seq * a.splits + split) * a.hq + head0 + r] = l;
      }
    }
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
}

template <class T> __global__ __launch_bounds__(64) void k_attn_merge(AttnArgs a) {
  __shared__ float weights[32];
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  int n, first;
  if (!attn_window(a, seq, n, first))
    return; // the split kernel raised the flag
  const int active = min(a.splits, (n + kKeys - 1) / kKeys);
  const float v = lane < active ? a.lse[((size_t)seq * a.splits + lane) * a.hq + head] : -INFINITY;
  const float mx = xor_max32(v);
  const float w = lane < active ? expf(v - mx) : 0.f;
  const float total = xor_sum32(w);
  bool fine = true;
  if (lane < active) {
    weights[lane] = w / total;
    fine = isfinite(weights[lane]);
  }
  __syncthreads();
  float s0 = 0.f, s1 = 0.f;
  for (int sp = 0; sp < active; ++sp) {
    const float2 p = *reinterpret_cast<const float2 *>(
        a.partial + (((size_t)seq * a.splits + sp) * a.hq + head) * kD + 2 * lane);
    s0 = __builtin_fmaf(weights[sp], p.x, s0);
    s1 = __builtin_fmaf(weights[sp], p.y, s1);
  }
  const uint32_t word = pack2(s0, s1);
  fine = fine && ((word & 0x7f80u) != 0x7f80u) && ((word & 0x7f800000u) != 0x7f800000u);
  const size_t o = ((size_t)seq * a.hq + head) * kD + 2 * lane;
  if constexpr (std::is_same<T, uint16_t>::value)
    static_cast<uint32_t *>(a.out)[o / 2] = word;
  else
    *reinterpret_cast<float2 *>(static_cast<float *>(a.out) + o) =
        make_float2(lo16(word), hi16(word));
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
}


// ---- q8_0 caches ------------------------------------------------------------------------
//
// q8_native::EncodeQuery, Split, Merge (kv_q8_native.cuh:103-148, 198-363).  The query is
// rotated like the K rows (128-point Hadamard, bit 0 first) and coded per 32-block with an
// fp32 scale; a score is the integer dot product of codes, block by block, scaled by
// RN(k_scale * q_scale):  four partial sums P_sub over the 4-code groups sub and sub + 4 of
// each block (fmaf in block order), then ((P0 + P1) + (P2 + P3)), times 1/sqrt(128).  Each
// 128-key tile runs as four 32-key online-softmax streams (slice s: keys 32 s .. 32 s + 31),
// each key lane keeping its own denominator; PV multiplies V codes by p * v_scale.  The four
// streams join per split; the merge rotates the result back (two 64-point transforms).
// Here one half-wave (32 lanes) serves one query head: lane = key for the scores, lane =
// four dimensions for PV; the tile of 128 K and V rows is staged in LDS once for the G heads.

constexpr int kQ8Tile = 128, kRowBytes = 544;

template <class T> __global__ __launch_bounds__(64) void k_q8_0_query(AttnArgs a) {
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  const size_t base = ((size_t)seq * a.hq + head) * kD;
  float x0 = act_value<T>(a.q, base + lane), x1 = act_value<T>(a.q, base + 64 + lane);
  if (__ballot(!isfinite(x0) || !isfinite(x1)) != 0) {
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  // features lane and lane + 64: stages on bits 0..5 across lanes, bit 6 in the lane
#pragma unroll
  for (int bit = 1; bit < 64; bit *= 2) {
    const float o0 = __shfl_xor(x0, bit, 64), o1 = __shfl_xor(x1, bit, 64);
    x0 = (lane & bit) ? o0 - x0 : x0 + o0;
    x1 = (lane & bit) ? o1 - x1 : x1 + o1;
  }
  const float y0 = (x0 + x1) * .08838834764831845f, y1 = (x0 - x1) * .08838834764831845f;
  // blocks lane / 32 (feature lane) and 2 + lane / 32 (feature lane + 64)
  float m0 = fabsf(y0), m1 = fabsf(y1);
#pragma unroll
  for (int d = 16; d >= 1; d /= 2) {
    m0 = fmaxf(m0, __shfl_xor(m0, d, 64));
    m1 = fmaxf(m1, __shfl_xor(m1, d, 64));
  }
  const float d0 = m0 / 127.f, d1 = m1 / 127.f;
  if (__ballot(!isfinite(d0) || !isfinite(d1)) != 0) {
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  a.qcodes[base + lane] = (int8_t)q8_0_code(y0, d0 == 0.f ? 0.f : 1.f / d0);
  a.qcodes[base + 64 + lane] = (int8_t)q8_0_code(y1, d1 == 0.f ? 0.f : 1.f / d1);
  if ((lane & 31) == 0) {
    a.qscale[((size_t)seq * a.hq + head) * 4 + lane / 32] = d0;
    a.qscale[((size_t)seq * a.hq + head) * 4 + 2 + lane / 32] = d1;
  }
}

__device__ __forceinline__ float f16_bits(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
}

template <int G> __global__ __launch_bounds__(32 * G < 64 ? 64 : 32 * G) void k_q8_0_split(AttnArgs a) {
  constexpr int NT = 32 * G < 64 ? 64 : 32 * G;
  // Half a tile (two 32-key slices) is staged at a time: 20 KB of LDS per workgroup.
  constexpr int HK = kQ8Tile / 2;
  __shared__ uint32_t kq[HK][36]; // K codes, rows padded to 36 words
  __shared__ uint32_t vq[HK][32]; // V codes
  __shared__ float ksc[HK][4];
  __shared__ float vsc[4][HK];    // V block scales, by block then key
  __shared__ float pr[G][32];            // this slice's probabilities, per head
  const int split = blockIdx.x, kv = blockIdx.y, seq = blockIdx.z, tid = threadIdx.x;
  const int hg = tid >> 5, lane = tid & 31, head = kv * G + (hg < G ? hg : G - 1);
  int n, first;
  if (!attn_window(a, seq, n, first) || (a.local && a.cap != 1024)) {
    if (split == 0 && kv == 0 && tid == 0)
      raise_bad(a.bad);
    return;
  }
  const int tiles = (n + kQ8Tile - 1) / kQ8Tile, active = min(a.splits, tiles);
  if (split >= active)
    return; // block-uniform
  const int begin = tiles * split / active, end = tiles * (split + 1) / active;
  const int features = a.hkv * kD, dbytes = 2 * (features / 32);
  const uint8_t *krows = static_cast<const uint8_t *>(static_cast<const void *>(a.kc)) +
                         (size_t)seq * a.seq_stride * kRowBytes;
  const uint8_t *vrows = static_cast<const uint8_t *>(static_cast<const void *>(a.vc)) +
                         (size_t)seq * a.seq_stride * kRowBytes;
  // this head's coded query
  int qi[32];
  float qd[4];
  {
    const int *src = reinterpret_cast<const int *>(a.qcodes + ((size_t)seq * a.hq + head) * kD);
#pragma unroll
    for (int i = 0; i < 32; ++i)
      qi[i] = src[i];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      qd[b] = a.qscale[((size_t)seq * a.hq + head) * 4 + b];
  }
  float mx[4], den[4], acc[4][4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
    mx[sl] = -INFINITY;
    den[sl] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[sl][i] = 0.f;
  }
  for (int step = begin * 2; step < end * 2; ++step) {
    const int tile = step >> 1, h0 = (step & 1) * HK;
    // Stage keys h0 .. h0 + 63 of the tile: codes as 16-byte chunks (8 per row and tensor),
    // scales 8 bytes per row.
    for (int c = tid; c < HK * 8; c += NT) {
      const int key = c >> 3, part = c & 7, o = tile * kQ8Tile + h0 + key;
      uint4 kw = make_uint4(0, 0, 0, 0), vw = make_uint4(0, 0, 0, 0);
      if (o < n) {
        const size_t row = (size_t)(a.local ? (first + o) & 1023 : first + o) * kRowBytes;
        kw = ld_nt(reinterpret_cast<const uint4 *>(krows + row + dbytes + kv * kD) + part);
        vw = ld_nt(reinterpret_cast<const uint4 *>(vrows + row + dbytes + kv * kD) + part);
      }
      *reinterpret_cast<uint4 *>(&kq[key][4 * part]) = kw;
      *reinterpret_cast<uint4 *>(&vq[key][4 * part]) = vw;
    }
    for (int key = tid; key < HK; key += NT) {
      const int o = tile * kQ8Tile + h0 + key;
      uint2 kd = make_uint2(0, 0), vd = make_uint2(0, 0);
      if (o < n) {
        const size_t row = (size_t)(a.local ? (first + o) & 1023 : first + o) * kRowBytes;
        kd = *reinterpret_cast<const uint2 *>(krows + row + 8 * kv);
        vd = *reinterpret_cast<const uint2 *>(vrows + row + 8 * kv);
      }
      ksc[key][0] = f16_bits(kd.x & 0xffffu);
      ksc[key][1] = f16_bits(kd.x >> 16);
      ksc[key][2] = f16_bits(kd.y & 0xffffu);
      ksc[key][3] = f16_bits(kd.y >> 16);
      vsc[0][key] = f16_bits(vd.x & 0xffffu);
      vsc[1][key] = f16_bits(vd.x >> 16);
      vsc[2][key] = f16_bits(vd.y & 0xffffu);
      vsc[3][key] = f16_bits(vd.y >> 16);
    }
    __syncthreads();
    if (hg < G) {
#pragma unroll
      for (int hs = 0; hs < 2; ++hs) {
        const int sl = (step & 1) * 2 + hs; // the online-softmax stream of this slice
        const int key = hs * 32 + lane, o = tile * kQ8Tile + h0 + key;
        int kw[32];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const uint4 w = *reinterpret_cast<const uint4 *>(&kq[key][4 * m]);
          kw[4 * m] = (int)w.x;
          kw[4 * m + 1] = (int)w.y;
          kw[4 * m + 2] = (int)w.z;
          kw[4 * m + 3] = (int)w.w;
        }
        float part[4];
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          float dot = 0.f;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            int sum = __builtin_amdgcn_sdot4(kw[b * 8 + sub], qi[b * 8 + sub], 0, false);
            sum = __builtin_amdgcn_sdot4(kw[b * 8 + sub + 4], qi[b * 8 + sub + 4], sum, false);
            dot = __builtin_fmaf((float)sum, ksc[key][b] * qd[b], dot);
          }
          part[sub] = dot;
        }
        const float dot = (part[0] + part[1]) + (part[2] + part[3]);
        const float own = o < n ? dot * kScoreScale : -INFINITY;
        float top = own;
#pragma unroll
        for (int d = 16; d >= 1; d /= 2)
          top = fmaxf(top, __shfl_xor(top, d, 32));
        const float next = fmaxf(mx[sl], top);
        const float alpha = isfinite(mx[sl]) ? expf(mx[sl] - next) : 0.f;
        const float p = isfinite(own) ? expf(own - next) : 0.f;
        mx[sl] = next;
        den[sl] = __builtin_fmaf(den[sl], alpha, p);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[sl][i] *= alpha;
        // The half-wave's probabilities go through LDS (its own row of pr; a half-wave
        // executes in lockstep with its writes, so no barrier is needed for it).
        pr[hg][lane] = p;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll 2
        for (int k4 = 0; k4 < 32; k4 += 4) {
          const float4 p4 = *reinterpret_cast<const float4 *>(&pr[hg][k4]);
          const float4 s4 = *reinterpret_cast<const float4 *>(&vsc[lane >> 3][hs * 32 + k4]);
          const float pk[4] = {p4.x, p4.y, p4.z, p4.w}, sk[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float factor = pk[j] * sk[j];
            const uint32_t codes = vq[hs * 32 + k4 + j][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[sl][i] = __builtin_fmaf(factor, (float)(int8_t)(codes >> (8 * i)), acc[sl][i]);
          }
        }
        __builtin_amdgcn_wave_barrier(); // pr is rewritten by the next slice
      }
    }
    __syncthreads();
  }
  if (hg >= G)
    return;
  float top = -INFINITY;
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
    float d = den[sl];
#pragma unroll
    for (int o = 16; o >= 1; o /= 2)
      d = d + __shfl_xor(d, o, 32);
    mx[sl] = d > 0.f ? mx[sl] + logf(d) : -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[sl][i] = d > 0.f ? acc[sl][i] / d : 0.f;
    top = fmaxf(top, mx[sl]);
  }
  top = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
  float total = 0.f, sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
    const float w = isfinite(mx[sl]) ? expf(mx[sl] - top) : 0.f;
    total += w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sum[i] = __builtin_fmaf(w, acc[sl][i], sum[i]);
  }
  if (!(total > 0.f) || !isfinite(total)) {
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  float *dst = a.partial + (((size_t)seq * a.splits + split) * a.hq + head) * kD + 4 * lane;
  *reinterpret_cast<float4 *>(dst) =
      make_float4(sum[0] / total, sum[1] / total, sum[2] / total, sum[3] / total);
  if (lane == 0)
    a.lse[((size_t)seq * a.splits + split) * a.hq + head] = top + logf(total);
}

template <class T> __global__ __launch_bounds__(64) void k_q8_0_merge(AttnArgs a) {
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  int n, first;
  if (!attn_window(a, seq, n, first) || (a.local && a.cap != 1024))
    return; // the split kernel raised the flag
  const int active = min(a.splits, (n + kQ8Tile - 1) / kQ8Tile), l32 = lane & 31;
  const float v = l32 < active ? a.lse[((size_t)seq * a.splits + l32) * a.hq + head] : -INFINITY;
  float mxv = v;
#pragma unroll
  for (int d = 16; d >= 1; d /= 2)
    mxv = fmaxf(mxv, __shfl_xor(mxv, d, 32));
  const float p = l32 < active ? expf(v - mxv) : 0.f;
  float den = p;
#pragma unroll
  for (int d = 16; d >= 1; d /= 2)
    den = den + __shfl_xor(den, d, 32);
  const float weight = p / den;
  float x0 = 0.f, x1 = 0.f;
  for (int sp = 0; sp < active; ++sp) {
    const float w = __shfl(weight, sp, 64);
    const float *src = a.partial + (((size_t)seq * a.splits + sp) * a.hq + head) * kD;
    x0 = __builtin_fmaf(w, src[lane], x0);
    x1 = __builtin_fmaf(w, src[64 + lane], x1);
  }
  // back from the V rotation: two 64-point transforms (features lane and lane + 64)
#pragma unroll
  for (int bit = 1; bit < 64; bit *= 2) {
    const float o0 = __shfl_xor(x0, bit, 64), o1 = __shfl_xor(x1, bit, 64);
    x0 = (lane & bit) ? o0 - x0 : x0 + o0;
    x1 = (lane & bit) ? o1 - x1 : x1 + o1;
  }
  x0 *= .125f;
  x1 *= .125f;
  const uint32_t word = pack2(x0, x1); // lo: feature lane, hi: feature lane + 64
  if (__ballot(!isfinite(x0) || !isfinite(x1)) != 0 && lane == 0)
    raise_bad(a.bad);
  const size_t o = ((size_t)seq * a.hq + head) * kD;
  if constexpr (std::is_same<T, uint16_t>::value) {
    static_cast<uint16_t *>(a.out)[o + lane] = (uint16_t)(word & 0xffffu);
    static_cast<uint16_t *>(a.out)[o + 64 + lane] = (uint16_t)(word >> 16);
  } else {
    static_cast<float *>(a.out)[o + lane] = lo16(word);
    static_cast<float *>(a.out)[o + 64 + lane] = hi16(word);
  }
}

} // namespace

extern "C" long long padra_DecodeAttentionScratch(int format, int seqs, int q_heads,
                                                  int splits) {
  if (seqs < 1 || q_heads < 1 || splits < 1 || splits > 32 ||
      (format != PADRA_KV_BF16 && format != PADRA_KV_Q8 && format != PADRA_KV_Q8_0))
    return -1;
  const long long base = (long long)seqs * splits * q_heads * (kD + 1);
  // q8_0: the coded query (128 bytes) and its 4 block scales per head
  return format == PADRA_KV_Q8_0 ? base + (long long)seqs * q_heads * (kD / 4 + 4) : base;
}

extern "C" int padra_DecodeAttention(void *stream, const void *q, const padra_KVCache *kv,
                                     void *out, const padra_Positions *pos, int seqs,
                                     int q_heads, int kv_heads, int local, int splits,
                                     float *scratch, long long scratch_floats, int *bad,
                                     int act) {
  if (!q || !kv || !out || !pos || !bad || !scratch || seqs < 1 || q_heads < 1 ||
      kv_heads < 1 || q_heads % kv_heads || !kv->k || !kv->v || kv->cap < 1 ||
      kv->cap > 131072 || pos->mode != PADRA_POS_DECODE || !pos->decode || pos->maximum < 1 ||
      pos->maximum > 131072 || pos->vocab < 1 || (seqs > 1 && kv->seq_stride < kv->cap) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32) || !aligned16(kv->k) ||
      !aligned16(kv->v) || !aligned16(scratch) || splits < 0 || splits > 32)
    return PADRA_INVALID_ARGUMENT;
  if (kv->format != PADRA_KV_BF16 && kv->format != PADRA_KV_Q8 && kv->format != PADRA_KV_Q8_0)
    return PADRA_UNSUPPORTED;
  if (kv->format == PADRA_KV_Q8 && !kv->scales)
    return PADRA_INVALID_ARGUMENT;
  const bool q8 = kv->format == PADRA_KV_Q8_0, q8s = kv->format == PADRA_KV_Q8;
  if (q8 && kv_heads * kD != 512)
    return PADRA_UNSUPPORTED; // the 544-byte q8_0 row of 4 KV heads
  if (splits == 0) // the reference's counts
    splits = q8 ? (local ? 16 : 32) : std::min((kv->cap + kKeys - 1) / kKeys, local ? 16 : 32);
  const long long need = padra_DecodeAttentionScratch(kv->format, seqs, q_heads, splits);
  if (scratch_floats < need)
    return PADRA_INVALID_ARGUMENT;
  AttnArgs a{};
  a.q = q;
  a.kc = static_cast<const uint16_t *>(kv->k);
  a.vc = static_cast<const uint16_t *>(kv->v);
  a.out = out;
  a.partial = scratch;
  a.lse = scratch + (long long)seqs * splits * q_heads * kD;
  a.qscale = a.lse + (long long)seqs * splits * q_heads;
  a.qcodes = reinterpret_cast<int8_t *>(a.qscale + (long long)seqs * q_heads * 4);
  a.decode = pos->decode;
  a.seqs = seqs;
  a.hq = q_heads;
  a.hkv = kv_heads;
  a.cap = kv->cap;
  a.local = local ? 1 : 0;
  a.splits = splits;
  a.maximum = pos->maximum;
  a.vocab = pos->vocab;
  a.seq_stride = seqs > 1 ? kv->seq_stride : 0;
  a.bad = bad;
  a.kvscales = static_cast<const float *>(kv->scales);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 split_grid(splits, kv_heads, seqs), merge_grid(q_heads, seqs);
  const int group = q_heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return PADRA_UNSUPPORTED;
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    if (q8) {
      hipLaunchKernelGGL((k_q8_0_query<T>), merge_grid, dim3(64), 0, s, a);
      switch (group) {
      case 1:
        hipLaunchKernelGGL((k_q8_0_split<1>), split_grid, dim3(64), 0, s, a);
        break;
      case 2:
        hipLaunchKernelGGL((k_q8_0_split<2>), split_grid, dim3(64), 0, s, a);
        break;
      case 4:
        hipLaunchKernelGGL((k_q8_0_split<4>), split_grid, dim3(128), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((k_q8_0_split<8>), split_grid, dim3(256), 0, s, a);
        break;
      }
      hipLaunchKernelGGL((k_q8_0_merge<T>), merge_grid, dim3(64), 0, s, a);
      return launched("DecodeAttention");
    }
    auto split = [&](auto q8tag) {
      constexpr bool Q8 = decltype(q8tag)::value;
      switch (group) {
      case 1:
        hipLaunchKernelGGL((k_attn_mx<1, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      case 2:
        hipLaunchKernelGGL((k_attn_mx<2, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      case 4:
        hipLaunchKernelGGL((k_attn_mx<4, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((k_attn_mx<8, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      }
    };
    if (q8s)
      split(std::true_type{});
    else
      split(std::false_type{});
    hipLaunchKernelGGL((k_attn_merge<T>), merge_grid, dim3(64), 0, s, a);
    return launched("DecodeAttention");
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}
