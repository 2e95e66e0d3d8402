// Decode attention over a BF16 KV cache: split-K partial softmax, then a per-head merge.
//
// Reference: gqa8_fragment_validation::SplitBF16 (attention_gqa8_fragment_validation.cuh:
// 79-214) with attention_perhead_exact::Merge (attention_perhead_exact.cuh:7-38), for any
// number of query heads per KV head (the reference fixes 8).  One token per sequence, at
// its DecodeState position; keys are the last n positions (n = position + 1, or at most
// 1024 for a local ring), read from cache row (first + offset) % cap.
//
// Split kernel: one wave per (sequence, KV head, split), over that split's 32-key tiles.
//  - Scores: lane l takes key l % 32 and half l / 32 of the 128 dimensions, against the
//    G query rows held in LDS; the halves meet in one lane exchange.  scale 1/sqrt(128)
//    after the dot product, as the reference applies it.
//  - Online softmax per row with the reference's arithmetic: the tile maximum and the sum
//    of probabilities are xor-butterflies over the 32 key lanes (the reference's warp
//    order), probabilities in fp32 for the denominator (fmaf(den, alpha, total)) and
//    rounded to BF16 for the PV product.
//  - PV: lane l owns dimensions 2l, 2l+1 of every row; the V tile is staged in LDS.
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

// a.lo * b.lo + a.hi * b.hi + c for BF16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <class T> __device__ __forceinline__ float act_value(const void *p, size_t i) {
  if constexpr (std::is_same<T, uint16_t>::value)
    return __uint_as_float((uint32_t) static_cast<const uint16_t *>(p)[i] << 16);
  else
    return static_cast<const float *>(p)[i];
}

// q8 cache rows decoded into the BF16 tile: bf16(code * scale) (kv_q8::Decode,
// kv_q8.cuh:15-27); a -128 code, an invalid scale or a non-finite result raises the flag.
__device__ __forceinline__ void q8_decode16(uint4 codes, float scale, uint4 &lo, uint4 &hi,
                                            bool &fine) {
  const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
  uint32_t out[8];
  bool ok = isfinite(scale) && scale > 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = w[i] ^ 0x80808080u; // a byte 0x80 (code -128) becomes zero
    ok = ok && (((x - 0x01010101u) & ~x & 0x80808080u) == 0);
    out[2 * i] = pack2((float)(int8_t)(w[i] & 0xffu) * scale, (float)(int8_t)((w[i] >> 8) & 0xffu) * scale);
    out[2 * i + 1] = pack2((float)(int8_t)((w[i] >> 16) & 0xffu) * scale, (float)(int8_t)(w[i] >> 24) * scale);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    ok = ok && ((out[i] & 0x7f80u) != 0x7f80u) && ((out[i] & 0x7f800000u) != 0x7f800000u);
  lo = make_uint4(out[0], out[1], out[2], out[3]);
  hi = make_uint4(out[4], out[5], out[6], out[7]);
  fine = fine && ok;
}

template <int G, class T, bool Q8>
__global__ __launch_bounds__(64) void k_attn_split(AttnArgs a) {
  __shared__ uint32_t qs[G][kD / 2];         // query rows, BF16 pairs
  // K and V tiles, BF16 pairs; K rows padded to 68 words so that the 32 key lanes' 16-byte
  // reads spread over the banks.
  __shared__ uint32_t ks[kKeys][kD / 2 + 4];
  __shared__ uint32_t vs[kKeys][kD / 2];
  __shared__ uint16_t ps[kKeys / 2][G][2];   // BF16 probabilities, key pairs per row
  const int split = blockIdx.x, kv = blockIdx.y, seq = blockIdx.z, lane = threadIdx.x;
  int n, first;
  const bool ok = attn_window(a, seq, n, first);
  if (!ok) {
    if (split == 0 && kv == 0 && lane == 0)
      raise_bad(a.bad);
    return;
  }
  const int tiles = (n + kKeys - 1) / kKeys, active = min(a.splits, tiles);
  if (split >= active)
    return; // block-uniform
  const int begin = tiles * split / active, end = tiles * (split + 1) / active;
  const int features = a.hkv * kD;
  // element offset of this sequence's rows and this KV head (BF16 values or q8 codes)
  const size_t head_off = (size_t)seq * a.seq_stride * features + kv * kD;
  const uint16_t *kc = a.kc + head_off, *vc = a.vc + head_off;
  const int8_t *k8 = reinterpret_cast<const int8_t *>(a.kc) + head_off;
  const int8_t *v8 = reinterpret_cast<const int8_t *>(a.vc) + head_off;
  const float2 *sc = reinterpret_cast<const float2 *>(a.kvscales) +
                     (size_t)seq * a.seq_stride * a.hkv + kv;

  // Query rows: finite and BF16-exact, as the reference requires of its fp32 input.
  bool qfine = true;
  for (int i = lane; i < G * kD / 2; i += 64) {
    const size_t o = ((size_t)seq * a.hq + kv * G) * kD + 2 * i;
    const float x0 = act_value<T>(a.q, o), x1 = act_value<T>(a.q, o + 1);
    qfine = qfine && isfinite(x0) && isfinite(x1) && (__float_as_uint(x0) & 0xffffu) == 0 &&
            (__float_as_uint(x1) & 0xffffu) == 0;
    qs[i / (kD / 2)][i % (kD / 2)] = (__float_as_uint(x0) >> 16) | (__float_as_uint(x1) & 0xffff0000u);
  }
  if (__ballot(!qfine) != 0 && lane == 0)
    raise_bad(a.bad);

  const int key = lane & 31, half = lane >> 5;
  float maximum[G], den[G], acc[G][2];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    maximum[r] = -INFINITY;
    den[r] = 0.f;
    acc[r][0] = acc[r][1] = 0.f;
  }
  bool fine = true;
  __syncthreads();
  // Tile loads: 16-byte chunk c = lane + 64 m of the tile's 32 key rows (key c / 16,
  // dimensions 8 (c % 16) ..), contiguous 1 KB per instruction.  Rows past the window load
  // a valid row and are zeroed (the reference zero-fills them).
  // q8: chunk c = lane + 64 m (m < 4) holds 16 codes (key c / 8, dimensions 16 (c % 8) ..),
  // with that key's scale pair.
  constexpr int CH = Q8 ? 4 : 8;
  float2 kvs[CH];
  auto load_tile = [&](int tile, uint4 (&kw)[8], uint4 (&vw)[8]) {
#pragma unroll
    for (int m = 0; m < CH; ++m) {
      const int c = lane + 64 * m, o = tile * kKeys + (c >> (Q8 ? 3 : 4));
      const size_t row = (size_t)((first + (o < n ? o : 0)) % a.cap);
      if constexpr (Q8) {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(k8 + row * features) + (c & 7));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(v8 + row * features) + (c & 7));
        kvs[m] = sc[row * a.hkv];
      } else {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(kc + row * features) + (c & 15));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(vc + row * features) + (c & 15));
      }
    }
  };
  uint4 kw[8], vw[8];
  load_tile(begin, kw, vw);
  for (int tile = begin; tile < end; ++tile) {
#pragma unroll
    for (int m = 0; m < CH; ++m) {
      const int c = lane + 64 * m;
      if constexpr (Q8) {
        const int key8 = c >> 3, part = c & 7;
        uint4 klo, khi, vlo, vhi;
        if (tile * kKeys + key8 >= n) { // the reference stages zeros with unit scales
          klo = khi = vlo = vhi = make_uint4(0, 0, 0, 0);
        } else {
          q8_decode16(kw[m], kvs[m].x, klo, khi, fine);
          q8_decode16(vw[m], kvs[m].y, vlo, vhi, fine);
        }
        *reinterpret_cast<uint4 *>(&ks[key8][part * 8]) = klo;
        *reinterpret_cast<uint4 *>(&ks[key8][part * 8 + 4]) = khi;
        *reinterpret_cast<uint4 *>(&vs[key8][part * 8]) = vlo;
        *reinterpret_cast<uint4 *>(&vs[key8][part * 8 + 4]) = vhi;
      } else {
        if (tile * kKeys + (c >> 4) >= n)
          kw[m] = vw[m] = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4 *>(&ks[c >> 4][(c & 15) * 4]) = kw[m];
        *reinterpret_cast<uint4 *>(&vs[c >> 4][(c & 15) * 4]) = vw[m];
      }
    }
    __syncthreads();
    // The next tile's loads are in flight during this tile's arithmetic (the last tile
    // reloads itself, keeping the loads unconditional).
    load_tile(min(tile + 1, end - 1), kw, vw);
    const bool valid = tile * kKeys + key < n;
    // Scores of this lane's key for every row: dot products of BF16 pairs (each product of
    // two BF16 values is exact in fp32).
    float s[G];
#pragma unroll
    for (int r = 0; r < G; ++r) {
      float dot = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const uint4 qw = *reinterpret_cast<const uint4 *>(&qs[r][half * 32 + 4 * m]);
        const uint4 kq = *reinterpret_cast<const uint4 *>(&ks[key][half * 32 + 4 * m]);
        dot = dot2(qw.x, kq.x, dot);
        dot = dot2(qw.y, kq.y, dot);
        dot = dot2(qw.z, kq.z, dot);
        dot = dot2(qw.w, kq.w, dot);
      }
      s[r] = (dot + __shfl_xor(dot, 32, 64)) * kScoreScale;
      if (valid)
        fine = fine && isfinite(s[r]);
      else
        s[r] = -INFINITY;
    }
    // Online softmax per row (every lane holds every row's running state).
    float alpha[G];
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const float next = fmaxf(maximum[r], xor_max32(s[r]));
      alpha[r] = isfinite(maximum[r]) ? expf(maximum[r] - next) : 0.f;
      const float prob = isfinite(s[r]) ? expf(s[r] - next) : 0.f;
      const float total = xor_sum32(prob);
      if (half == 0)
        ps[key / 2][r][key & 1] = (uint16_t)(pack2(prob, 0.f) & 0xffffu);
      den[r] = __builtin_fmaf(den[r], alpha[r], total);
      maximum[r] = next;
    }
    __syncthreads();
    // PV: dimensions 2*lane, 2*lane + 1.
#pragma unroll
    for (int r = 0; r < G; ++r) {
      acc[r][0] *= alpha[r];
      acc[r][1] *= alpha[r];
    }
    // Key pairs: (V[2jp][d], V[2jp+1][d]) against the row's probability pair.  A
    // non-finite V value reaches the outputs (inf or NaN) and is flagged there.
#pragma unroll 4
    for (int jp = 0; jp < kKeys / 2; ++jp) {
      const uint32_t va = vs[2 * jp][lane], vb = vs[2 * jp + 1][lane];
      const uint32_t x0 = __builtin_amdgcn_perm(vb, va, 0x05040100u); // (va.lo, vb.lo)
      const uint32_t x1 = __builtin_amdgcn_perm(vb, va, 0x07060302u); // (va.hi, vb.hi)
#pragma unroll
      for (int r = 0; r < G; ++r) {
        const uint32_t pw = *reinterpret_cast<const uint32_t *>(ps[jp][r]);
        acc[r][0] = dot2(pw, x0, acc[r][0]);
        acc[r][1] = dot2(pw, x1, acc[r][1]);
      }
    }
    __syncthreads();
  }
  const int head0 = kv * G;
#pragma unroll
  for (int r = 0; r < G; ++r) {
    float *dst = a.partial + (((size_t)seq * a.splits + split) * a.hq + head0 + r) * kD;
    const float v0 = acc[r][0] / den[r], v1 = acc[r][1] / den[r];
    fine = fine && isfinite(v0) && isfinite(v1);
    *reinterpret_cast<float2 *>(dst + 2 * lane) = make_float2(v0, v1);
    if (lane == 0) {
      const float l = maximum[r] + logf(den[r]);
      fine = fine && isfinite(l);
      a.lse[((size_t)seq * a.splits + split) * a.hq + head0 + r] = l;
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
        hipLaunchKernelGGL((k_attn_split<1, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      case 2:
        hipLaunchKernelGGL((k_attn_split<2, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      case 4:
        hipLaunchKernelGGL((k_attn_split<4, T, Q8>), split_grid, dim3(64), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((k_attn_split<8, T, Q8>), split_grid, dim3(64), 0, s, a);
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
