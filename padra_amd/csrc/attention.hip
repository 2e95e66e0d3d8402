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
// The split kernels take their probabilities from the hardware exponential
// (v_exp_f32(x * log2 e), __expf): for x = score - maximum <= 0 its relative error grows
// with |x| (about 2^-24 |x| from rounding x * log2 e), so it is a few fp32 ulps where the
// probability matters and larger only for probabilities below e^-16.
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "norm_fp8.h"

using namespace padra;

namespace {

constexpr int kD = 128, kKeys = 32;
// Launches of up to this many sequences on a global cache order their split waves by
// window length (the ranking reads seqs^2 control records).
constexpr int kOrderMaxSeqs = 512;
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
  // The split kernels' sequence for grid slot z (longest window first), or null for
  // slot z = sequence z.
  int *order;
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

// Sequence `seq`'s place in the split kernels' dispatch order, written by a 64-lane block:
// windows by decreasing length (a sequence that is not admitted counts as 0 keys), ties
// by sequence index.  The split kernels give grid slot z to order[z], so the longest
// windows start first and the shortest fill the end of the launch; every output is the
// same as in sequence order.
__device__ __forceinline__ void attn_rank(const AttnArgs &a, int seq) {
  int n, first;
  const int mine = attn_window(a, seq, n, first) ? n : 0;
  int before = 0;
  for (int j = threadIdx.x; j < a.seqs; j += 64) {
    const int other = attn_window(a, j, n, first) ? n : 0;
    before += other > mine || (other == mine && j < seq);
  }
  before = xor_reduce<32>(before, [](int x, int y) { return x + y; });
  if (threadIdx.x == 0)
    a.order[before] = seq;
}
__device__ __forceinline__ int attn_seq(const AttnArgs &a) {
  return a.order ? a.order[blockIdx.z] : (int)blockIdx.z;
}

__global__ __launch_bounds__(64) void k_attn_order(AttnArgs a) { attn_rank(a, blockIdx.x); }

// Hadamard stages on lane bits 0..5, bit 0 first, of two values per lane.
__device__ __forceinline__ void hadamard64_pair(float &x0, float &x1, int lane) {
  x0 = hadamard_lane<1>(x0, lane);
  x1 = hadamard_lane<1>(x1, lane);
  x0 = hadamard_lane<2>(x0, lane);
  x1 = hadamard_lane<2>(x1, lane);
  x0 = hadamard_lane<4>(x0, lane);
  x1 = hadamard_lane<4>(x1, lane);
  x0 = hadamard_lane<8>(x0, lane);
  x1 = hadamard_lane<8>(x1, lane);
  x0 = hadamard_lane<16>(x0, lane);
  x1 = hadamard_lane<16>(x1, lane);
  x0 = hadamard_lane<32>(x0, lane);
  x1 = hadamard_lane<32>(x1, lane);
}
__device__ __forceinline__ float xor_max32(float v) {
  return xor_reduce<16>(v, [](float x, float y) { return fmaxf(x, y); });
}
__device__ __forceinline__ float xor_sum32(float v) {
  return xor_reduce<16>(v, [](float x, float y) { return x + y; });
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

// Whether every code * scale of a q8 row is finite in BF16 and the scale is valid:
// 0 < scale and 127 * scale below 0x1.ffp127, the least fp32 value that BF16 rounds to
// infinity (|code| <= 127, and rounding is monotonic).  Tiles with a row that fails it
// check each decoded value (q8_check16).
__device__ __forceinline__ bool q8_scale_fast(float scale) {
  return scale > 0.f && 127.f * scale < 0x1.ffp127f;
}

// The 16 values code * scale of a code chunk (kv_q8::Decode), with the least code seen
// (as a float; -128 is the code the reference rejects) and whether the scale passes
// q8_scale_fast.  The caller gives keys past the window zero codes and a unit scale, as
// the reference stages them.  Each code is one v_cvt_f32_i32 with a sign-extended byte
// select.
__device__ __forceinline__ void q8_values16(uint4 c, float scale, float (&f)[16], float &least,
                                            bool &slow) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  float code[16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      code[4 * i + b] = (float)(int8_t)((w[i] >> (8 * b)) & 0xffu);
#pragma unroll
  for (int i = 0; i < 16; ++i) // min(min(least, a), b): one v_min3_f32 per pair
    least = fminf(least, code[i]);
#pragma unroll
  for (int i = 0; i < 16; ++i)
    f[i] = code[i] * scale;
  slow = slow || !q8_scale_fast(scale);
}

// kv_q8::Decode's checks on a chunk whose scale failed q8_scale_fast: a valid scale and
// every code * scale finite in BF16.
__device__ __forceinline__ bool q8_check16(uint4 c, float scale) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  bool ok = isfinite(scale) && scale > 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float v = (float)(int8_t)((w[i] >> (8 * b)) & 0xffu) * scale;
      ok = ok & ((pack2(v, 0.f) & 0x7f80u) != 0x7f80u);
    }
  return ok;
}

// Slot of dimension d in a staged V row.  Each staging lane writes its dimension pairs at
// slots rotated by its chunk index (q8: 16-dimension chunks, rotation by the chunk; BF16:
// 8-dimension chunks, rotation by chunk / 4), which spreads a quarter-wave's 16-byte writes
// over all 64 banks.
template <bool Q8> __device__ __forceinline__ int vq_slot(int d) {
  if constexpr (Q8) {
    const int t = d >> 4;
    return 16 * t + 2 * (((d >> 1) + t) & 7) + (d & 1);
  } else {
    const int c = d >> 3;
    return 8 * c + 2 * (((d >> 1) + (c >> 2)) & 3) + (d & 1);
  }
}

template <int G, class T, bool Q8>
__global__ __launch_bounds__(64) void k_attn_mx(AttnArgs a) {
  constexpr int KW = kD / 2 + 4; // K row stride in words (padding spreads the banks)
  constexpr int VW = kD + 16;    // V group stride in uint2
  __shared__ __align__(16) uint32_t ks[kKeys][KW];
  // (V[4j][d], V[4j+1][d]), (V[4j+2][d], V[4j+3][d]) at slot vq_slot(d)
  __shared__ __align__(16) uint2 vq[kKeys / 4][VW];
  const int split = blockIdx.x, kv = blockIdx.y, seq = attn_seq(a), lane = threadIdx.x;
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

  // Tile loads, each instruction covering whole rows of the head (BF16: 256 B on 16 lanes;
  // q8: 128 codes on 8 lanes).
  //  BF16 K: chunk c = lane + 64 m is key c / 16, dimensions 8 (c % 16) ..; V: m = 4 h + p
  //  is key 16 h + 4 grp + p, dimensions 8 col ...
  //  q8 K: chunk c = lane + 64 m is key c / 8, dimensions 16 (c % 8) ..; V: m = p is key
  //  4 (lane / 8) + p, dimensions 16 (lane % 8) ..; each with its key's scale.
  // Rows past the window load a valid row and are zeroed (the reference zero-fills them).
  constexpr int CH = Q8 ? 4 : 8;
  float ksc[CH], vsc[CH];
  // Cache row of window offset tile * 32 + key: the tile's first row (one modulo per tile)
  // plus the key, wrapped once (the window holds at most cap keys); keys past the window
  // read the window's first row.
  const int first_row = first % a.cap;
  auto row_of = [&](int tile, int key) {
    const int base = (first + tile * kKeys) % a.cap, r = base + key;
    return (size_t)(tile * kKeys + key < n ? (r >= a.cap ? r - a.cap : r) : first_row);
  };
  auto vkey = [&](int m) {
    return Q8 ? 4 * (lane >> 3) + m : 16 * (m >> 2) + 4 * grp + (m & 3);
  };
  // A tile whose 32 keys are inside the window and do not wrap is 32 consecutive cache
  // rows from `base`: load m of a lane is then the tile's first row, plus this lane's
  // offset for m = 0 (bytes), plus a per-m step that is the same for every lane.
  //  q8 K: key lane / 8 + 8 m; V: key 4 (lane / 8) + m.  BF16 K: key lane / 16 + 4 m;
  //  V: key 4 grp + 16 (m / 4) + m % 4.
  constexpr int ES = Q8 ? 1 : 2; // bytes per cache element
  const size_t row_bytes = (size_t)features * ES;
  const uint32_t koff = (uint32_t)(Q8 ? (lane >> 3) * row_bytes + 16 * (lane & 7)
                                      : (lane >> 4) * row_bytes + 16 * (lane & 15));
  const uint32_t voff = (uint32_t)(Q8 ? 4 * (lane >> 3) * row_bytes + 16 * (lane & 7)
                                      : 4 * grp * row_bytes + 16 * col);
  const uint32_t kso = (uint32_t)((lane >> 3) * a.hkv * 8), vso = 4 * kso + 4;
  auto kstep = [&](int m) { return (size_t)(Q8 ? 8 * m : 4 * m) * row_bytes; };
  auto vstep = [&](int m) { return (size_t)(Q8 ? m : 16 * (m >> 2) + (m & 3)) * row_bytes; };
  const char *kbytes = Q8 ? reinterpret_cast<const char *>(k8) : reinterpret_cast<const char *>(kc);
  const char *vbytes = Q8 ? reinterpret_cast<const char *>(v8) : reinterpret_cast<const char *>(vc);
  const char *sbytes = reinterpret_cast<const char *>(sc);
  auto load_tile = [&](int tile, uint4 (&kw)[8], uint4 (&vw)[8]) {
    const int base = (first + tile * kKeys) % a.cap;
    if (tile * kKeys + kKeys <= n && base + kKeys <= a.cap) { // block-uniform
      const char *kt = kbytes + (size_t)base * row_bytes, *vt = vbytes + (size_t)base * row_bytes;
      const char *st = sbytes + (size_t)base * a.hkv * 8;
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(kt + kstep(m) + koff));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(vt + vstep(m) + voff));
        if constexpr (Q8) {
          ksc[m] = *reinterpret_cast<const float *>(st + (size_t)8 * m * a.hkv * 8 + kso);
          vsc[m] = *reinterpret_cast<const float *>(st + (size_t)m * a.hkv * 8 + vso);
        }
      }
      return;
    }
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
      if (left < kKeys) { // block-uniform: the window's last tile
#pragma unroll
        for (int m = 0; m < CH; ++m) {
          if (((lane + 64 * m) >> 3) >= left) {
            kw[m] = make_uint4(0, 0, 0, 0);
            ksc[m] = 1.f;
          }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (vkey(m) >= left) {
            vw[m] = make_uint4(0, 0, 0, 0);
            vsc[m] = 1.f;
          }
        }
      }
      float least = 0.f;
      bool slow = false;
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        const int c = lane + 64 * m, key = c >> 3, part = c & 7;
        float f[16];
        q8_values16(kw[m], ksc[m], f, least, slow);
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
        q8_values16(vw[m], vsc[m], fv[m], least, slow);
      fine = fine && least > -128.f;
      if (__ballot(slow) != 0) { // rare: huge or invalid scales
#pragma unroll
        for (int m = 0; m < CH; ++m) {
          if (((lane + 64 * m) >> 3) < left && !q8_scale_fast(ksc[m]))
            fine = fine && q8_check16(kw[m], ksc[m]);
          if (vkey(m) < left && !q8_scale_fast(vsc[m]))
            fine = fine && q8_check16(vw[m], vsc[m]);
        }
      }
      const int t7 = lane & 7;
      uint2 *dst = &vq[lane >> 3][16 * t7];
#pragma unroll
      for (int e = 0; e < 16; e += 2)
        *reinterpret_cast<uint4 *>(dst + 2 * ((e / 2 + t7) & 7)) =
            make_uint4(pack2(fv[0][e], fv[1][e]), pack2(fv[2][e], fv[3][e]),
                       pack2(fv[0][e + 1], fv[1][e + 1]), pack2(fv[2][e + 1], fv[3][e + 1]));
    } else {
      if (left < kKeys) { // block-uniform: the window's last tile
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          if (((lane + 64 * m) >> 4) >= left)
            kw[m] = make_uint4(0, 0, 0, 0);
          if (vkey(m) >= left)
            vw[m] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int c = lane + 64 * m;
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
          *reinterpret_cast<uint4 *>(dst + 2 * ((e + (col >> 2)) & 3)) = make_uint4(
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
    tmax = fmaxf(tmax, lane_xor<16>(tmax));
    tmax = fmaxf(tmax, lane_xor<32>(tmax));
    const float next = fmaxf(maximum, tmax);
    const float alpha = isfinite(maximum) ? __expf(maximum - next) : 0.f;
    float p[8], total = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      p[k] = isfinite(sv[k]) ? __expf(sv[k] - next) : 0.f;
      total += p[k];
    }
    total += lane_xor<16>(total);
    total += lane_xor<32>(total);
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
      const int d = vq_slot<Q8>(16 * b + col);
      const uint2 v0 = vq[grp][d], v1 = vq[4 + grp][d];
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


// MergeQuantize (attention_merge_quantize_wide_exact.cuh:9-66), the merge the reference
// runs after its q8 split (attention_gqa8_q8.cuh:278-300) and, with the FP8 output, after
// the BF16 one: the per-head merge of k_attn_merge for every head of a sequence in one
// workgroup, then the E4M3 encoding of the whole output row (q_heads x 128 values) with
// scale = max|out| / 448 (1 for a zero row), as padra_QuantizeFP8 writes it.  Waves take
// heads wave, wave + 4, ...; lane l holds dimensions 2l, 2l + 1 of each.
template <class T>
__global__ __launch_bounds__(256) void k_attn_merge_fp8(AttnArgs a, uint8_t *packed,
                                                        float *scales) {
  constexpr int kWaves = 4, kHeads = 32;
  __shared__ float weights[kHeads][32];
  __shared__ float maxima[kWaves];
  const int seq = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int n, first;
  if (!attn_window(a, seq, n, first))
    return; // block-uniform; the split kernel raised the flag
  const int active = min(a.splits, (n + kKeys - 1) / kKeys);
  bool fine = true;
  for (int head = wave; head < a.hq; head += kWaves) {
    const float v =
        lane < active ? a.lse[((size_t)seq * a.splits + lane) * a.hq + head] : -INFINITY;
    const float mx = xor_max32(v);
    const float w = lane < active ? expf(v - mx) : 0.f;
    const float total = xor_sum32(w);
    if (lane < active) {
      weights[head][lane] = w / total;
      fine = fine && isfinite(weights[head][lane]);
    }
  }
  __syncthreads();
  uint32_t words[kHeads / kWaves];
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < kHeads / kWaves; ++k) {
    const int head = wave + kWaves * k;
    words[k] = 0u;
    if (head >= a.hq)
      continue;
    float s0 = 0.f, s1 = 0.f;
    for (int sp = 0; sp < active; ++sp) {
      const float2 p = *reinterpret_cast<const float2 *>(
          a.partial + (((size_t)seq * a.splits + sp) * a.hq + head) * kD + 2 * lane);
      s0 = __builtin_fmaf(weights[head][sp], p.x, s0);
      s1 = __builtin_fmaf(weights[head][sp], p.y, s1);
    }
    const uint32_t word = pack2(s0, s1);
    words[k] = word;
    fine = fine && ((word & 0x7f80u) != 0x7f80u) && ((word & 0x7f800000u) != 0x7f800000u);
    amax = fmaxf(amax, fmaxf(fabsf(lo16(word)), fabsf(hi16(word))));
    const size_t o = ((size_t)seq * a.hq + head) * kD + 2 * lane;
    if constexpr (std::is_same<T, uint16_t>::value)
      static_cast<uint32_t *>(a.out)[o / 2] = word;
    else
      *reinterpret_cast<float2 *>(static_cast<float *>(a.out) + o) =
          make_float2(lo16(word), hi16(word));
  }
  amax = xor_reduce<32>(amax, [](float x, float y) { return fmaxf(x, y); });
  if (lane == 0)
    maxima[wave] = amax;
  const bool row_fine = !__syncthreads_or(!fine);
  amax = fmaxf(fmaxf(maxima[0], maxima[1]), fmaxf(maxima[2], maxima[3]));
  if (!row_fine && threadIdx.x == 0)
    raise_bad(a.bad);
  const float scale = amax == 0.f ? 1.f : amax / 448.f;
  const float inverse = 1.f / scale;
  if (threadIdx.x == 0)
    scales[seq] = scale;
  const bool fast = row_fine && fp8_fast_ok(amax, inverse); // block-uniform
#pragma unroll
  for (int k = 0; k < kHeads / kWaves; ++k) {
    const int head = wave + kWaves * k;
    if (head >= a.hq)
      continue;
    const uint32_t word = words[k];
    const uint32_t code =
        fast ? e4m3_pair_fast(fp8_quotient(lo16(word), scale, inverse),
                              fp8_quotient(hi16(word), scale, inverse))
             : e4m3_code(lo16(word) / scale) | (e4m3_code(hi16(word) / scale) << 8);
    *reinterpret_cast<uint16_t *>(packed + ((size_t)seq * a.hq + head) * kD + 2 * lane) =
        (uint16_t)code;
  }
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
// Here (k_q8_0_mx) each stream is its own partial entry and the merge joins the 4 * splits
// entries; scores and PV run on the matrix cores.

constexpr int kQ8Tile = 128, kRowBytes = 544;

template <class T> __global__ __launch_bounds__(64) void k_q8_0_query(AttnArgs a) {
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  if (a.order && head == 0) // the split kernel's dispatch order, one sequence per block
    attn_rank(a, seq);
  const size_t base = ((size_t)seq * a.hq + head) * kD;
  float x0 = act_value<T>(a.q, base + lane), x1 = act_value<T>(a.q, base + 64 + lane);
  if (__ballot(!isfinite(x0) || !isfinite(x1)) != 0) {
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  // features lane and lane + 64: stages on bits 0..5 across lanes, bit 6 in the lane
  hadamard64_pair(x0, x1, lane);
  const float y0 = (x0 + x1) * .08838834764831845f, y1 = (x0 - x1) * .08838834764831845f;
  // blocks lane / 32 (feature lane) and 2 + lane / 32 (feature lane + 64)
  float m0 = fabsf(y0), m1 = fabsf(y1);
  m0 = xor_max32(m0);
  m1 = xor_max32(m1);
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

// ---- q8_0 split on the matrix cores -----------------------------------------------------
// One workgroup per (sequence, split): four waves, one per KV head, each serving its G query
// heads; the slice's 544-byte rows are staged whole, once for the four heads.  The reference
// keeps four online-softmax streams per split (stream s: keys 32 s .. 32 s + 31 of every
// 128-key tile) and weighs them by exp(lse_s - max) at the end; here each stream runs on its
// own over the split's tiles and is folded into the split's combination when it ends.
// Per 32-key slice:
//  - QK on v_mfma_i32_16x16x64_i8: rows are (head 4 j + r, block b) pairs of a head group j,
//    whose A operand is the head's query codes masked to block b, so that each result is the
//    exact integer dot product of one block; the score is then
//    fma(float(dot_b), RN(k_scale_b * q_scale_b), ..) in block order, times 1/sqrt(128) (the
//    reference sums the same products with its own grouping of the fp32 additions).  Lane l
//    holds head 4 j + l / 16 of key 16 k + l % 16.
//  - Softmax per head with the reference's recurrences (den = fmaf(den, alpha, p) per key
//    position), maxima over the 16 key lanes by DPP row rotations.
//  - PV on v_mfma_f32_16x16x32_bf16: O[head][dim] += (p * v_scale)[head][key] code[key][dim].
//    Codes are exact in BF16; the fp32 factor enters as two BF16 terms (hi + lo, 2^-17
//    relative).  The factor depends on the dimension's block, so rows are (head, block of a
//    block pair): lane l holds rows 4 (l / 16) + i of dimension 16 t + l % 16, of which the
//    rows of the tile's own block are kept.
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kStreams = 4;

__device__ __forceinline__ i32x4_t mfma_i8(uint4 a, uint4 b, i32x4_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a),
                                               __builtin_bit_cast(i32x4_t, b), c, 0, 0, 0);
}

// v from lane (l + N) % 16 of the lane's 16-lane row.
template <int N> __device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}
// The maximum (fmaxf: NaN operands dropped) and the sum over a 16-lane row; every lane of
// the row gets the same value (each step adds the lane's value to its half-row partner's).
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  return fmaxf(v, row_ror<1>(v));
}
__device__ __forceinline__ float row_sum16(float v) {
  v = v + row_ror<8>(v);
  v = v + row_ror<4>(v);
  v = v + row_ror<2>(v);
  return v + row_ror<1>(v);
}

// x as a BF16 pair hi + lo (hi = RN(x), lo = RN(x - hi)): the packed hi and lo words of
// two values.
__device__ __forceinline__ void bf16_split2(float x0, float x1, uint32_t &hi, uint32_t &lo) {
  hi = pack2(x0, x1);
  lo = pack2(x0 - lo16(hi), x1 - hi16(hi));
}

template <int G> __global__ __launch_bounds__(256) void k_q8_0_mx(AttnArgs a) {
  // The 4 KV heads of a row, one wave each: the slice's rows are staged together, whole.
  // K codes of the slice (rows padded to 36 words) and V codes as BF16 (4 keys per dimension
  // and group, at slot vq_slot<true>(d)); head strides padded to 32 words modulo the banks.
  __shared__ __align__(16) struct { uint32_t r[32][36]; uint32_t pad[32]; } kq_all[4];
  __shared__ __align__(16) struct { uint2 r[8][kD + 8]; uint2 pad[16]; } vq_all[4];
  __shared__ float ksc_all[4][32][4];    // K block scales by key
  __shared__ float vsc_all[4][4][32];    // V block scales by block
  __shared__ float ps_all[4][8][36];     // probabilities by head (rows padded)
  const int split = blockIdx.x, seq = attn_seq(a), tid = threadIdx.x, kv = tid >> 6;
  const int lane = tid & 63, col = lane & 15, grp = lane >> 4;
  auto &kq = kq_all[kv].r;
  auto &vq = vq_all[kv].r;
  auto &ksc = ksc_all[kv];
  auto &vsc = vsc_all[kv];
  auto &ps = ps_all[kv];
  int n, first;
  if (!attn_window(a, seq, n, first) || (a.local && a.cap != 1024)) {
    if (split == 0 && tid == 0)
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
  const int head0 = kv * G;

  // Query A operands: row col = (head 4 j + col / 4, block col % 4); K-slot group grp of
  // step h covers dimensions 64 h + 16 grp .. + 15, of block 2 h + grp / 2.
  uint4 aq[2][2];
  float qd[2][4]; // block scales of head 4 j + grp
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int hh = 4 * j + (col >> 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      aq[j][h] = make_uint4(0, 0, 0, 0);
      if (hh < G && (col & 3) == 2 * h + (grp >> 1))
        aq[j][h] = *reinterpret_cast<const uint4 *>(
            a.qcodes + ((size_t)seq * a.hq + head0 + hh) * kD + 64 * h + 16 * grp);
    }
    const int hq = 4 * j + grp;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      qd[j][b] = hq < G ? a.qscale[((size_t)seq * a.hq + head0 + hq) * 4 + b] : 0.f;
  }

  // Slice loads over whole rows (512 codes = 32 chunks of 16 bytes): K chunk c = tid + 256 m
  // is key c / 32, part c % 32 (head part / 8, codes 16 (part % 8) ..); V chunk m is key
  // 4 (tid / 32) + m, part tid % 32.  Threads 0..127 load the 32-byte scale headers: half
  // tid % 2 (heads 2 (tid % 2), + 1) of K row tid / 2 (tid < 64) or V row tid / 2 - 32.
  // Keys past the window load the window's first row and are zeroed (the reference
  // zero-fills them).
  auto row_at = [&](int o) {
    const int r = o < n ? o : 0;
    return (size_t)(a.local ? (first + r) & 1023 : first + r) * kRowBytes;
  };
  uint4 kw[4], vw[4], hw = make_uint4(0, 0, 0, 0);
  const int hrow = (tid >> 1) & 31;
  // A slice whose 32 rows are inside the window and consecutive in the cache: load m is
  // the slice's first row plus a per-thread offset plus a step common to all threads
  // (K: 8 m rows, V: m rows).
  const uint32_t koff = (uint32_t)((tid >> 5) * kRowBytes + dbytes + 16 * (tid & 31));
  const uint32_t voff = (uint32_t)(4 * (tid >> 5) * kRowBytes + dbytes + 16 * (tid & 31));
  const uint32_t hoff = (uint32_t)(hrow * kRowBytes + 16 * (tid & 1));
  auto load_slice = [&](int tile, int s) {
    const int o0 = tile * kQ8Tile + 32 * s;
    const int r0 = a.local ? (first + o0) & 1023 : first + o0;
    if (o0 + 32 <= n && (!a.local || r0 + 32 <= 1024)) { // block-uniform
      const uint8_t *kt = krows + (size_t)r0 * kRowBytes, *vt = vrows + (size_t)r0 * kRowBytes;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        kw[m] = ld_nt(reinterpret_cast<const uint4 *>(kt + (size_t)(8 * m) * kRowBytes + koff));
        vw[m] = ld_nt(reinterpret_cast<const uint4 *>(vt + (size_t)m * kRowBytes + voff));
      }
      if (tid < 128)
        hw = *reinterpret_cast<const uint4 *>((tid < 64 ? kt : vt) + hoff);
      return;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = tid + 256 * m;
      kw[m] = ld_nt(reinterpret_cast<const uint4 *>(krows + row_at(o0 + (c >> 5)) + dbytes) +
                    (c & 31));
      vw[m] = ld_nt(reinterpret_cast<const uint4 *>(vrows + row_at(o0 + 4 * (tid >> 5) + m) +
                                                    dbytes) + (tid & 31));
    }
    if (tid < 128)
      hw = *reinterpret_cast<const uint4 *>((tid < 64 ? krows : vrows) + row_at(o0 + hrow) +
                                            16 * (tid & 1));
  };

  bool fine = true;
  // The split's combination of its streams, for rows 4 grp + i of the PV layout (head
  // (4 grp + i) % 8): the largest stream log-sum-exp, the total weight, and the weighted
  // outputs of this lane's four dimension tiles t = 4 u + 2 (grp / 2) + v.
  float cm[4], ct[4], cs[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    cm[i] = -INFINITY;
    ct[i] = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      cs[u][i] = 0.f;
  }
  bool has[2] = {false, false}; // a stream of head 4 j + grp with a finite log-sum-exp
  const int slices = end - begin;
  load_slice(begin, 0);
  for (int s = 0; s < kStreams; ++s) {
    float mx[2] = {-INFINITY, -INFINITY}, den[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    f32x4_t o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t)
      o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < slices; ++it) {
      const int tile = begin + it, o0 = tile * kQ8Tile + 32 * s;
      // Stage the slice.  Keys past the window stage zero codes: only a slice that crosses
      // the window's end (block-uniform test) zeroes them, with a mask per key.
      if (o0 + 32 > n) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t kkeep = o0 + ((tid + 256 * m) >> 5) < n ? ~0u : 0u;
          const uint32_t vkeep = o0 + 4 * (tid >> 5) + m < n ? ~0u : 0u;
          kw[m] = make_uint4(kw[m].x & kkeep, kw[m].y & kkeep, kw[m].z & kkeep, kw[m].w & kkeep);
          vw[m] = make_uint4(vw[m].x & vkeep, vw[m].y & vkeep, vw[m].z & vkeep, vw[m].w & vkeep);
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int c = tid + 256 * m;
        *reinterpret_cast<uint4 *>(&kq_all[(c >> 3) & 3].r[c >> 5][4 * (c & 7)]) = kw[m];
      }
      {
        float f[4][16];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t w[4] = {vw[m].x, vw[m].y, vw[m].z, vw[m].w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b)
              f[m][4 * i + b] = (float)(int8_t)((w[i] >> (8 * b)) & 0xffu);
        }
        const int t7 = tid & 7;
        uint2 *dst = &vq_all[(tid >> 3) & 3].r[tid >> 5][16 * t7];
#pragma unroll
        for (int e = 0; e < 16; e += 2)
          *reinterpret_cast<uint4 *>(dst + 2 * ((e / 2 + t7) & 7)) =
              make_uint4(pack2(f[0][e], f[1][e]), pack2(f[2][e], f[3][e]),
                         pack2(f[0][e + 1], f[1][e + 1]), pack2(f[2][e + 1], f[3][e + 1]));
      }
      if (tid < 128) {
        const bool inside = o0 + hrow < n;
        const uint32_t hv[4] = {hw.x, hw.y, hw.z, hw.w};
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) { // heads 2 (tid % 2) + h2
          const int hd = 2 * (tid & 1) + h2;
          float d[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t word = hv[2 * h2 + (b >> 1)];
            d[b] = inside ? f16_bits((b & 1) ? word >> 16 : word & 0xffffu) : 0.f;
          }
          if (tid < 64) {
            *reinterpret_cast<float4 *>(&ksc_all[hd][hrow][0]) =
                make_float4(d[0], d[1], d[2], d[3]);
          } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
              vsc_all[hd][b][hrow] = d[b];
          }
        }
      }
      __syncthreads();
      // The next slice's loads are in flight during this slice's arithmetic: the next tile
      // of this stream, or the next stream's first slice.  After the last slice the loads
      // stay unconditional and repeat the slice just read, which L2 still holds.
      {
        const bool last_tile = it + 1 == slices, last = last_tile && s == kStreams - 1;
        load_slice(last ? tile : (last_tile ? begin : tile + 1), last_tile && !last ? s + 1 : s);
      }

      // Scores: head 4 j + grp, key 16 k + col.
      float sc[2][2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint4 b0 = *reinterpret_cast<const uint4 *>(&kq[16 * k + col][4 * grp]);
        const uint4 b1 = *reinterpret_cast<const uint4 *>(&kq[16 * k + col][16 + 4 * grp]);
        const float4 kd = *reinterpret_cast<const float4 *>(&ksc[16 * k + col][0]);
        const bool valid = o0 + 16 * k + col < n;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          i32x4_t d = mfma_i8(aq[j][0], b0, i32x4_t{0, 0, 0, 0});
          d = mfma_i8(aq[j][1], b1, d);
          float dot = 0.f;
          dot = __builtin_fmaf((float)d[0], kd.x * qd[j][0], dot);
          dot = __builtin_fmaf((float)d[1], kd.y * qd[j][1], dot);
          dot = __builtin_fmaf((float)d[2], kd.z * qd[j][2], dot);
          dot = __builtin_fmaf((float)d[3], kd.w * qd[j][3], dot);
          sc[k][j] = valid ? dot * kScoreScale : -INFINITY;
        }
      }
      float alpha[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float next = fmaxf(mx[j], row_max16(fmaxf(sc[0][j], sc[1][j])));
        alpha[j] = isfinite(mx[j]) ? __expf(mx[j] - next) : 0.f;
        mx[j] = next;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const float p = isfinite(sc[k][j]) ? __expf(sc[k][j] - next) : 0.f;
          den[k][j] = __builtin_fmaf(den[k][j], alpha[j], p);
          ps[4 * j + grp][16 * k + col] = p;
        }
      }
      // Rows 4 grp + i of the PV accumulators are head (4 grp + i) % 8, whose alpha lane 16 i
      // holds (alpha[0] for heads 0..3, alpha[1] for 4..7).
      if (__ballot(alpha[0] != 1.f || alpha[1] != 1.f) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha[0]), 16 * i));
          const float a1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha[1]), 16 * i));
          const float ar = (grp & 1) ? a1 : a0;
#pragma unroll
          for (int t = 0; t < 8; ++t)
            o[t][i] *= ar;
        }
      }
      __syncthreads();
      // PV A operands: row col = (head col % 8, block 2 c + col / 8); K-slots of group grp are
      // keys 8 grp .. 8 grp + 7.
      uint4 ahi[2], alo[2];
      {
        const int hh = col & 7;
        const float4 p0 = *reinterpret_cast<const float4 *>(&ps[hh][8 * grp]);
        const float4 p1 = *reinterpret_cast<const float4 *>(&ps[hh][8 * grp + 4]);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int b = 2 * c + (col >> 3);
          const float4 v0 = *reinterpret_cast<const float4 *>(&vsc[b][8 * grp]);
          const float4 v1 = *reinterpret_cast<const float4 *>(&vsc[b][8 * grp + 4]);
          const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
          uint32_t hi[4], lo[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float f0 = hh < G ? pv[2 * e] * vv[2 * e] : 0.f;
            const float f1 = hh < G ? pv[2 * e + 1] * vv[2 * e + 1] : 0.f;
            bf16_split2(f0, f1, hi[e], lo[e]);
          }
          ahi[c] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
          alo[c] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int d = vq_slot<true>(16 * t + col);
        const uint2 v0 = vq[2 * grp][d], v1 = vq[2 * grp + 1][d];
        const uint4 bv = make_uint4(v0.x, v0.y, v1.x, v1.y);
        o[t] = mfma_bf16(ahi[t >> 2], bv, o[t]);
        o[t] = mfma_bf16(alo[t >> 2], bv, o[t]);
      }
      __syncthreads(); // the next slice restages the tiles
    }
    // The stream's log-sum-exp (den over the 32 key positions), folded into the split's
    // combination with weight exp(lse - max): the reference weighs its four streams the
    // same way once all are done; online here, in stream order.  Streams without a finite
    // log-sum-exp carry no weight, as there.
    float dsum[2], lse[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dsum[j] = row_sum16(den[0][j] + den[1][j]);
      lse[j] = dsum[j] > 0.f ? mx[j] + logf(dsum[j]) : -INFINITY;
      has[j] = has[j] || isfinite(lse[j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // head (4 grp + i) % 8 is head 4 (grp % 2) + i, whose values lane 16 i holds (in
      // dsum[grp % 2] and lse[grp % 2]: read both, then select per lane)
      const float d0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsum[0]), 16 * i));
      const float d1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsum[1]), 16 * i));
      const float l0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lse[0]), 16 * i));
      const float l1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lse[1]), 16 * i));
      const float d = (grp & 1) ? d1 : d0, l = (grp & 1) ? l1 : l0;
      if (isfinite(l)) {
        const float m2 = fmaxf(cm[i], l);
        const float wa = isfinite(cm[i]) ? expf(cm[i] - m2) : 0.f, wb = expf(l - m2);
        ct[i] = __builtin_fmaf(ct[i], wa, wb);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            // both values first: a conditional over the two array elements would select
            // an address and index the accumulators at run time
            const float xa = o[4 * u + v][i], xb = o[4 * u + 2 + v][i];
            const float x = (grp >> 1) ? xb : xa;
            cs[2 * u + v][i] = __builtin_fmaf(cs[2 * u + v][i], wa, wb * (x / d));
          }
        cm[i] = m2;
      }
    }
  }
  // The split's entry: the combined output and log-sum-exp of each head.
  const size_t entry = (size_t)seq * a.splits + split;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hh = (4 * grp + i) & 7;
    if (hh < G) {
      float *dst = a.partial + (entry * a.hq + head0 + hh) * kD + col;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v)
          dst[16 * (4 * u + 2 * (grp >> 1) + v)] = ct[i] > 0.f ? cs[2 * u + v][i] / ct[i] : 0.f;
      if (col == 0 && grp < 2)
        a.lse[entry * a.hq + head0 + hh] = ct[i] > 0.f ? cm[i] + logf(ct[i]) : -INFINITY;
    }
  }
  // The reference's check of the split's combined weight: it fails when no stream of a
  // head has a finite log-sum-exp (a stream's is finite or -inf).
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (4 * j + grp < G)
      fine = fine && has[j];
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
}

template <class T> __global__ __launch_bounds__(64) void k_q8_0_mx_merge(AttnArgs a) {
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  int n, first;
  if (!attn_window(a, seq, n, first) || (a.local && a.cap != 1024))
    return; // the split kernel raised the flag
  // One entry per active split (at most 32: lanes 0..31).
  const int active = min(a.splits, (n + kQ8Tile - 1) / kQ8Tile), l32 = lane & 31;
  const size_t base = (size_t)seq * a.splits;
  const float v = l32 < active ? a.lse[(base + l32) * a.hq + head] : -INFINITY;
  float mxv = v;
  mxv = xor_max32(mxv);
  const float p = isfinite(v) ? expf(v - mxv) : 0.f;
  float den = p;
  den = xor_sum32(den);
  const float weight = p / den;
  float x0 = 0.f, x1 = 0.f;
  for (int sp = 0; sp < active; ++sp) {
    const float w = __shfl(weight, sp, 64);
    const float *src = a.partial + ((base + sp) * a.hq + head) * kD;
    x0 = __builtin_fmaf(w, src[lane], x0);
    x1 = __builtin_fmaf(w, src[64 + lane], x1);
  }
  // back from the V rotation: two 64-point transforms (features lane and lane + 64)
  hadamard64_pair(x0, x1, lane);
  x0 *= .125f;
  x1 *= .125f;
  const uint32_t word = pack2(x0, x1); // lo: feature lane, hi: feature lane + 64
  if (__ballot(!isfinite(x0) || !isfinite(x1) || !(den > 0.f)) != 0 && lane == 0)
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
  // partial outputs and log-sum-exps per split, rounded up to 16 bytes
  const long long base = ((long long)seqs * splits * q_heads * (kD + 1) + 3) & ~3ll;
  // q8_0: the coded query (128 bytes) and its 4 block scales per head, after the lse
  const long long query = format == PADRA_KV_Q8_0 ? (long long)seqs * q_heads * (kD / 4 + 4) : 0;
  // then the split kernels' dispatch order, one int per sequence, rounded up to 16 bytes
  return base + query + ((seqs + 3) & ~3ll);
}

namespace {
// The reference's split counts: q8_0 16 (local) or 32; otherwise one per 32 keys of the
// ring, at most 16 (local) or 32.
int reference_splits(const padra_KVCache *kv, int local) {
  if (kv->format == PADRA_KV_Q8_0)
    return local ? 16 : 32;
  return std::min((kv->cap + kKeys - 1) / kKeys, local ? 16 : 32);
}

// The split count for splits = -1, from a sweep on MI355X (64-sequence decode step):
// global windows keep the reference's count (within 1.5% of the best of 8-32); a local
// ring's 1024-key windows want about 1,024 resident waves for BF16 and q8_0 and 2,048 for
// q8 (1 / 8 / 64 sequences, BF16: 16 / 16 / 4 splits best; q8: 32 / 32 / 8; q8_0:
// 16 / 16 / 4; at 64 sequences 29.4 / 23.7 / 30.2 us against 40.8 / 31.8 / 49.9 us with the
// reference's 16).
int tuned_splits(const padra_KVCache *kv, int local, int seqs, int kv_heads) {
  if (!local)
    return reference_splits(kv, local);
  const int per_seq = std::max(1, seqs);
  if (kv->format == PADRA_KV_Q8_0)
    return std::clamp(256 / per_seq, 4, 16); // one 4-wave workgroup per (split, sequence)
  const int waves = kv->format == PADRA_KV_Q8 ? 2048 : 1024;
  const int cap_splits = std::min((kv->cap + kKeys - 1) / kKeys, kv->format == PADRA_KV_Q8 ? 32 : 16);
  return std::clamp(waves / (per_seq * std::max(1, kv_heads)), std::min(2, cap_splits), cap_splits);
}

// splits as passed (1..32), 0: the reference's count, -1: the tuned count; 0 if invalid.
int resolve_splits(const padra_KVCache *kv, int local, int seqs, int kv_heads, int splits) {
  if (splits == 0)
    return reference_splits(kv, local);
  if (splits == -1)
    return tuned_splits(kv, local, seqs, kv_heads);
  return splits >= 1 && splits <= 32 ? splits : 0;
}

// Both entry points: packed/scales non-null selects the merge with the FP8 encoding.
int decode_attention(void *stream, const void *q, const padra_KVCache *kv, void *out,
                     uint8_t *packed, float *scales, const padra_Positions *pos, int seqs,
                     int q_heads, int kv_heads, int local, int splits, float *scratch,
                     long long scratch_floats, int *bad, int act) {
  if (!q || !kv || !out || !pos || !bad || !scratch || seqs < 1 || q_heads < 1 ||
      kv_heads < 1 || q_heads % kv_heads || !kv->k || !kv->v || kv->cap < 1 ||
      kv->cap > 131072 || pos->mode != PADRA_POS_DECODE || !pos->decode || pos->maximum < 1 ||
      pos->maximum > 131072 || pos->vocab < 1 || (seqs > 1 && kv->seq_stride < kv->cap) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32) || !aligned16(kv->k) ||
      !aligned16(kv->v) || !aligned16(scratch) || splits < -1 || splits > 32)
    return PADRA_INVALID_ARGUMENT;
  if (kv->format != PADRA_KV_BF16 && kv->format != PADRA_KV_Q8 && kv->format != PADRA_KV_Q8_0)
    return PADRA_UNSUPPORTED;
  if (kv->format == PADRA_KV_Q8 && !kv->scales)
    return PADRA_INVALID_ARGUMENT;
  const bool fp8 = packed != nullptr;
  if (fp8 && (!scales || q_heads > 32 || (reinterpret_cast<uintptr_t>(packed) & 1) ||
              (reinterpret_cast<uintptr_t>(scales) & 3)))
    return PADRA_INVALID_ARGUMENT;
  if (fp8 && kv->format == PADRA_KV_Q8_0)
    return PADRA_UNSUPPORTED; // the reference's q8_0 merge has no FP8 form
  const bool q8 = kv->format == PADRA_KV_Q8_0, q8s = kv->format == PADRA_KV_Q8;
  if (q8 && kv_heads * kD != 512)
    return PADRA_UNSUPPORTED; // the 544-byte q8_0 row of 4 KV heads
  splits = resolve_splits(kv, local, seqs, kv_heads, splits);
  const long long need = padra_DecodeAttentionScratch(kv->format, seqs, q_heads, splits);
  if (scratch_floats < need)
    return PADRA_INVALID_ARGUMENT;
  AttnArgs a{};
  a.q = q;
  a.kc = static_cast<const uint16_t *>(kv->k);
  a.vc = static_cast<const uint16_t *>(kv->v);
  a.out = out;
  // scratch: partial [seqs][splits][hq][128], lse [seqs][splits][hq], then (q8_0 only,
  // from the next 16-byte boundary) coded query [seqs][hq][128] bytes and query block
  // scales [seqs][hq][4]; the end is exactly padra_DecodeAttentionScratch's count
  const long long entries = (long long)seqs * splits * q_heads;
  const long long qbase = (entries * (kD + 1) + 3) & ~3ll;
  a.partial = scratch;
  a.lse = scratch + entries * kD;
  a.qcodes = reinterpret_cast<int8_t *>(scratch + qbase);
  a.qscale = scratch + qbase + (long long)seqs * q_heads * (kD / 4);
  // Longest windows first when the lengths can differ much: several sequences on a
  // global cache (a local ring's windows are at most 1024 keys).
  const long long obase = qbase + (q8 ? (long long)seqs * q_heads * (kD / 4 + 4) : 0);
  a.order = seqs >= 2 && seqs <= kOrderMaxSeqs && !local ? reinterpret_cast<int *>(scratch + obase)
                                                         : nullptr;
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
    if (a.order && !q8) // (the q8_0 query kernel ranks the sequences itself)
      hipLaunchKernelGGL(k_attn_order, dim3(seqs), dim3(64), 0, s, a);
    if (q8) {
      hipLaunchKernelGGL((k_q8_0_query<T>), merge_grid, dim3(64), 0, s, a);
      switch (group) {
      case 1:
        hipLaunchKernelGGL((k_q8_0_mx<1>), dim3(splits, 1, seqs), dim3(256), 0, s, a);
        break;
      case 2:
        hipLaunchKernelGGL((k_q8_0_mx<2>), dim3(splits, 1, seqs), dim3(256), 0, s, a);
        break;
      case 4:
        hipLaunchKernelGGL((k_q8_0_mx<4>), dim3(splits, 1, seqs), dim3(256), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((k_q8_0_mx<8>), dim3(splits, 1, seqs), dim3(256), 0, s, a);
        break;
      }
      hipLaunchKernelGGL((k_q8_0_mx_merge<T>), merge_grid, dim3(64), 0, s, a);
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
    if (fp8)
      hipLaunchKernelGGL((k_attn_merge_fp8<T>), dim3(seqs), dim3(256), 0, s, a, packed, scales);
    else
      hipLaunchKernelGGL((k_attn_merge<T>), merge_grid, dim3(64), 0, s, a);
    return launched("DecodeAttention");
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}
} // namespace

extern "C" int padra_DecodeAttentionSplits(const padra_KVCache *kv, int seqs, int kv_heads,
                                           int local, int splits) {
  if (!kv || seqs < 1 || kv_heads < 1 || kv->cap < 1 || splits < -1 || splits > 32 ||
      (kv->format != PADRA_KV_BF16 && kv->format != PADRA_KV_Q8 && kv->format != PADRA_KV_Q8_0))
    return -1;
  return resolve_splits(kv, local, seqs, kv_heads, splits);
}


extern "C" int padra_DecodeAttention(void *stream, const void *q, const padra_KVCache *kv,
                                     void *out, const padra_Positions *pos, int seqs,
                                     int q_heads, int kv_heads, int local, int splits,
                                     float *scratch, long long scratch_floats, int *bad,
                                     int act) {
  return decode_attention(stream, q, kv, out, nullptr, nullptr, pos, seqs, q_heads, kv_heads,
                          local, splits, scratch, scratch_floats, bad, act);
}

extern "C" int padra_DecodeAttentionFP8(void *stream, const void *q, const padra_KVCache *kv,
                                        void *out, uint8_t *packed, float *scales,
                                        const padra_Positions *pos, int seqs, int q_heads,
                                        int kv_heads, int local, int splits, float *scratch,
                                        long long scratch_floats, int *bad, int act) {
  if (!packed)
    return PADRA_INVALID_ARGUMENT;
  return decode_attention(stream, q, kv, out, packed, scales, pos, seqs, q_heads, kv_heads,
                          local, splits, scratch, scratch_floats, bad, act);
}

// ---- the entry point that allocates nothing ---------------------------------------------
//
// padra_DecodeAttentionNoAlloc's workspace: a fixed array in device memory, one copy per
// GPU the library runs on, held until the process ends.  Its name is a host-side
// stand-in, not a device address: host code uses only the address hipGetSymbolAddress
// returns for the current device (scratch_address below).
static __device__ __align__(256) float scratch[PADRA_DECODE_ATTENTION_STATIC_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<float *> g_scratch_address[kMaxDevices];
std::mutex g_scratch_mutex;

// The array's device address on the current device, looked up on the first call there;
// null when the lookup fails.
float *scratch_address() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return nullptr;
  float *p = g_scratch_address[dev].load(std::memory_order_acquire);
  if (p)
    return p;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch_address[dev].load(std::memory_order_relaxed);
  if (!p) {
    void *address = nullptr;
    const hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !address) {
      fprintf(stderr, "padra: DecodeAttentionNoAlloc: workspace lookup failed: %s\n",
              hipGetErrorString(e));
      return nullptr;
    }
    p = static_cast<float *>(address);
    g_scratch_address[dev].store(p, std::memory_order_release);
  }
  return p;
}
} // namespace

extern "C" int padra_DecodeAttentionNoAlloc(void *stream, const void *q, const padra_KVCache *kv,
                                            void *out, const padra_Positions *pos, int seqs,
                                            int q_heads, int kv_heads, int local, int splits,
                                            int *bad, int act) {
  if (!kv || splits < -1 || splits > 32)
    return PADRA_INVALID_ARGUMENT;
  splits = resolve_splits(kv, local, seqs, kv_heads, splits);
  const long long need = padra_DecodeAttentionScratch(kv->format, seqs, q_heads, splits);
  if (need < 0)
    return PADRA_INVALID_ARGUMENT;
  if (need > PADRA_DECODE_ATTENTION_STATIC_FLOATS) {
    fprintf(stderr,
            "padra: DecodeAttentionNoAlloc: %lld workspace floats needed (%d sequences, %d "
            "query heads), the fixed workspace holds %d; use padra_DecodeAttention\n",
            need, seqs, q_heads, PADRA_DECODE_ATTENTION_STATIC_FLOATS);
    return PADRA_INVALID_ARGUMENT;
  }
  float *ws = scratch_address();
  if (!ws)
    return PADRA_INTERNAL;
  return decode_attention(stream, q, kv, out, nullptr, nullptr, pos, seqs, q_heads, kv_heads,
                          local, splits, ws, PADRA_DECODE_ATTENTION_STATIC_FLOATS, bad, act);
}
