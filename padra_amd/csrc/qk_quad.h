// Q/K RMSNorm + NeoX RoPE (+ KV store) with four lanes per head: lane 4j + g owns
// features 32g .. 32g+31 of head j, i.e. exactly reference warp g of the head's 128-thread
// block (qk_rope_store_exact.cuh:28-44, inference.cu:110-135).  A wave covers 16 heads.
//
//  - Warp g's shuffle-down tree runs inside lane g.
//  - The tree over the four warp partials, (w0 + w2) + (w1 + w3), is two DPP quad
//    exchanges (lanes g^2, then g^1), then a broadcast from lane g = 0.
//  - RoPE pairs feature f < 64 with f + 64, i.e. lane g with lane g^2: the partner's
//    normalized values arrive by DPP, one move per feature.
// The block's head vectors (4 KB of BF16 or 8 KB of fp32 activations) are loaded and
// stored as coalesced 1 KB instructions and transposed through an LDS image.
#pragma once
#include <type_traits>

#include "qk_heads.h"

namespace padra {

// DPP quad permutations: the value of lane (lane ^ 2), of lane (lane ^ 1), and of lane
// (lane & ~3) (the first lane of the quad).
// Every lane of a quad permutation has a source, so no old value is needed (bound_ctrl).
__device__ __forceinline__ uint32_t quad_xor2(uint32_t v) {
  return __builtin_amdgcn_mov_dpp((int)v, 0x4e /* quad_perm [2,3,0,1] */, 0xf, 0xf, true);
}
__device__ __forceinline__ uint32_t quad_xor1(uint32_t v) {
  return __builtin_amdgcn_mov_dpp((int)v, 0xb1 /* quad_perm [1,0,3,2] */, 0xf, 0xf, true);
}
__device__ __forceinline__ uint32_t quad_first(uint32_t v) {
  return __builtin_amdgcn_mov_dpp((int)v, 0x00 /* quad_perm [0,0,0,0] */, 0xf, 0xf, true);
}
__device__ __forceinline__ float fquad_xor2(float v) { return __uint_as_float(quad_xor2(__float_as_uint(v))); }
__device__ __forceinline__ float fquad_xor1(float v) { return __uint_as_float(quad_xor1(__float_as_uint(v))); }
__device__ __forceinline__ float fquad_first(float v) { return __uint_as_float(quad_first(__float_as_uint(v))); }

// LDS image slot of piece p (0..3) owned by lane `owner`; pieces of one lane are 64 slots
// apart and rotated so both the transposing writes and the row reads are conflict-free.
__device__ __forceinline__ int quad_slot(int owner, int p) { return p * 64 + ((owner + 4 * p) & 63); }

// An all-V block (16 heads) with a BF16 cache: a coalesced copy into each token's slot.
template <class A>
__device__ __forceinline__ void v_rows_copy16(const A &a, unsigned block0, unsigned nq,
                                              unsigned nk) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, features = a.hkv * D;
  // Piece m of this lane is chunk (lane & 15) of head 4m + (lane >> 4) of the block; its
  // (token, KV head) pair advances by 4 heads per piece, without a division.
  const unsigned idx0 = block0 - nq - nk + (unsigned)(lane >> 4);
  const unsigned hk = (unsigned)a.hkv;
  unsigned tm[4], hm[4];
  tm[0] = idx0 / hk;
  hm[0] = idx0 - tm[0] * hk;
#pragma unroll
  for (int m = 1; m < 4; ++m) {
    tm[m] = tm[m - 1];
    hm[m] = hm[m - 1] + 4u;
    while (hm[m] >= hk) {
      hm[m] -= hk;
      ++tm[m];
    }
  }
  uint4 d[4];
  PosState ps[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned idx = min(idx0 + 4u * m, nk - 1u);
    ps[m] = fetch_state(a.pos, (int)min(tm[m], (unsigned)a.tokens - 1u));
    d[m] = ld_nt(reinterpret_cast<const uint4 *>(a.v + (size_t)idx * D) + (lane & 15));
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned idx = idx0 + 4u * m;
    if (idx >= nk)
      continue;
    const int t = (int)tm[m], h = (int)hm[m], ci = lane & 15;
    bool ok;
    const int pos = resolve_position(a.pos, ps[m], t, a.cap, a.first, false, ok);
    if (!ok || pos < 0 || pos >= a.table_rows) {
      if (ci == 0)
        raise_bad(a.bad);
      continue;
    }
    if (t < a.first)
      continue;
    const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
    const long long slot = seq * a.seq_stride + ring_slot(pos, a.cap);
    st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.vc) + slot * features + h * D) + ci, d[m]);
  }
}

// Hadamard stage across lanes of the quad: this lane's features pair with lane (lane ^ D)'s
// (D = 1: feature bit 5, D = 2: bit 6); the lower lane keeps lower + upper, the upper lane
// lower - upper.  Both are one fused multiply-add other + s * x with s = +-1: s * x is
// exact, so it rounds once, as the sum or difference does.
// Signed form, for values that only feed q8_0 codes: x + s * partner with s = -1 on the
// upper lane, one fused multiply-add whose partner operand is read across lanes inside the
// instruction (no separate lane move).  The upper lane then holds upper - lower, the exact
// negation of the rounded lower - upper (round-to-nearest-even is symmetric), so the true
// value is sign_quad * x with sign_quad = -1 on upper lanes; the caller folds the product
// of the stages' signs into its scale multiply.  Only the sign of a zero result can differ
// from hadamard_quad's, and codes (|x| maximum, rounded magnitudes) do not see it.
// The compiler does not fold a lane move into v_fmac_f32, so each half of the values is
// one asm block of sixteen v_fmac_f32_dpp.  The s_nop 1 at its head gives the two wait
// states a DPP read needs after a VALU write of its source; inside the block every
// instruction reads a register no earlier instruction of the block wrote; the s_nop 1 at
// its tail covers a DPP read of the block's last results that follows it (the hazard
// recognizer does not see the block's writes as VALU writes).
#define PADRA_FMAC_DPP(i, perm) \
  "v_fmac_f32_dpp %" #i ", %" #i ", %16 quad_perm:" perm " row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
#define PADRA_FMAC_DPP16(perm)                                                            \
  "s_nop 1\n" PADRA_FMAC_DPP(0, perm) PADRA_FMAC_DPP(1, perm) PADRA_FMAC_DPP(2, perm)     \
      PADRA_FMAC_DPP(3, perm) PADRA_FMAC_DPP(4, perm) PADRA_FMAC_DPP(5, perm)             \
          PADRA_FMAC_DPP(6, perm) PADRA_FMAC_DPP(7, perm) PADRA_FMAC_DPP(8, perm)         \
              PADRA_FMAC_DPP(9, perm) PADRA_FMAC_DPP(10, perm) PADRA_FMAC_DPP(11, perm)   \
                  PADRA_FMAC_DPP(12, perm) PADRA_FMAC_DPP(13, perm)                       \
                      PADRA_FMAC_DPP(14, perm) PADRA_FMAC_DPP(15, perm) "s_nop 1\n"
template <int D> __device__ __forceinline__ void hadamard_quad_signed(float (&x)[32], int g) {
  const float sgn = (g & D) ? -1.f : 1.f;
#pragma unroll
  for (int h = 0; h < 32; h += 16) {
    float *y = x + h;
    if constexpr (D == 1)
      asm volatile(PADRA_FMAC_DPP16("[1,0,3,2]")
                   : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
                     "+v"(y[6]), "+v"(y[7]), "+v"(y[8]), "+v"(y[9]), "+v"(y[10]), "+v"(y[11]),
                     "+v"(y[12]), "+v"(y[13]), "+v"(y[14]), "+v"(y[15])
                   : "v"(sgn));
    else
      asm volatile(PADRA_FMAC_DPP16("[2,3,0,1]")
                   : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
                     "+v"(y[6]), "+v"(y[7]), "+v"(y[8]), "+v"(y[9]), "+v"(y[10]), "+v"(y[11]),
                     "+v"(y[12]), "+v"(y[13]), "+v"(y[14]), "+v"(y[15])
                   : "v"(sgn));
  }
}
#undef PADRA_FMAC_DPP16
#undef PADRA_FMAC_DPP
template <int D> __device__ __forceinline__ void hadamard_quad(float (&x)[32], int g) {
  const float sgn = (g & D) ? -1.f : 1.f;
#pragma unroll
  for (int f = 0; f < 32; ++f) {
    const uint32_t o = D == 1 ? quad_xor1(__float_as_uint(x[f])) : quad_xor2(__float_as_uint(x[f]));
    x[f] = __builtin_fmaf(sgn, x[f], __uint_as_float(o));
  }
}

// The codes of one quantized head vector held by a quad (lane g: features 32g..32g+31 in
// x), computed but not stored.
//  - q8 (kv_q8::Encode, kv_q8.cuh:56-73): scale = amax/127 over the head (1 for a zero
//    head), codes RNE(x / scale) clamped to +-127.
//  - q8_0 (q8_native::EncodeKV, kv_q8_native.cuh:76-100): the rotation when FMT is the
//    rotated format (K: 128-point, stages on feature bits 0-4 in the lane, bits 5 and 6
//    across the quad, scale 1/sqrt(128); V: two 64-point transforms, no bit-6 stage,
//    scale 1/8), then block g = this lane's 32 values: d = half(amax/127), codes
//    roundf(x * (1/d_fp32)) clamped; `fail` when amax or d is not finite.
struct QuadCodes {
  uint32_t cw[8];
  float scale;   // q8: the head's scale
  uint16_t d;    // q8_0: this lane's block scale (fp16 bits)
  bool fail;     // q8_0: this lane's block cannot be encoded
};
template <int FMT, bool ISV>
__device__ __forceinline__ QuadCodes quad_codes(float (&x)[32], int g) {
  QuadCodes r;
  r.fail = false;
  r.d = 0;
  r.scale = 1.f;
  if constexpr (FMT == PADRA_KV_Q8) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      m = fmaxf(m, fabsf(x[i]));
    m = fmaxf(m, __uint_as_float(quad_xor1(__float_as_uint(m))));
    m = fmaxf(m, __uint_as_float(quad_xor2(__float_as_uint(m))));
    const float scale = m == 0.f ? 1.f : m / 127.f, inverse = 1.f / scale;
    r.scale = scale;
    if (q8_fast_ok(scale)) { // quad-uniform
#pragma unroll
      for (int i = 0; i < 8; ++i)
        r.cw[i] = pack_codes4(q8_code_fast(x[4 * i], scale, inverse),
                              q8_code_fast(x[4 * i + 1], scale, inverse),
                              q8_code_fast(x[4 * i + 2], scale, inverse),
                              q8_code_fast(x[4 * i + 3], scale, inverse));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        r.cw[i] = pack_codes4(q8_code(x[4 * i], scale), q8_code(x[4 * i + 1], scale),
                              q8_code(x[4 * i + 2], scale), q8_code(x[4 * i + 3], scale));
    }
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      // the stages' signs (lane bit 0 for bit 5, lane bit 1 for bit 6) ride in the scale
      hadamard32(x);
      hadamard_quad_signed<1>(x, g);
      if constexpr (!ISV)
        hadamard_quad_signed<2>(x, g);
      const float sc = ((g ^ (ISV ? 0 : g >> 1)) & 1) ? -(ISV ? .125f : .08838834764831845f)
                                                      : (ISV ? .125f : .08838834764831845f);
#pragma unroll
      for (int f = 0; f < 32; ++f)
        x[f] = x[f] * sc;
    }
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      am = fmaxf(am, fabsf(x[i]));
    const float ad = am / 127.f;
    const __half dh = __float2half(ad);
    r.fail = !isfinite(am) || !isfinite(__half2float(dh));
    r.d = __half_as_ushort(dh);
    const float inverse = ad == 0.f ? 0.f : 1.f / ad;
    q8_0_codes32(x, inverse, r.cw);
  }
  return r;
}

// Encodes one (token, KV head) pair held by a quad: the rotated K head (xk) and the V
// head (xv), as the reference's one warp per pair does (kv_q8.cuh:41-73,
// kv_q8_native.cuh:52-101).
//  - A non-finite value in K or V (q8: or a value that is not BF16-exact) raises the flag
//    and neither row is written (kv_q8.cuh:49-54, kv_q8_native.cuh:70-79).
//  - q8: codes of both, then the (k, v) scale pair as one 8-byte store.
//  - q8_0: block r of K and of V are written for every r before the first block whose
//    K or V scale fails (kv_q8_native.cuh:82-99); the flag is raised at a failing block.
// `active` is quad-uniform; DPP quad exchanges need only the quad's own lanes.
template <int FMT, class T, class A>
__device__ __forceinline__ void encode_pair_quad(const A &a, float (&xk)[32], const Act32<T> &xv,
                                                 long long slot, int h, int g, bool active) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    x[i] = xv.get(i);
  {
    bool valid = true;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      valid = valid && isfinite(xk[i]) && isfinite(x[i]);
      if constexpr (FMT == PADRA_KV_Q8)
        valid = valid && (__float_as_uint(xk[i]) & 0xffffu) == 0u &&
                (__float_as_uint(x[i]) & 0xffffu) == 0u;
    }
    uint32_t v = valid ? 1u : 0u;
    v &= quad_xor1(v);
    v &= quad_xor2(v);
    if (!active)
      return;
    if (!v) {
      if (g == 0)
        raise_bad(a.bad);
      return;
    }
  }
  const QuadCodes cv = quad_codes<FMT, true>(x, g);
  const QuadCodes ck = quad_codes<FMT, false>(xk, g);
  if constexpr (FMT == PADRA_KV_Q8) {
    int8_t *kq = static_cast<int8_t *>(a.kc) + slot * features + h * D + 32 * g;
    int8_t *vq = static_cast<int8_t *>(a.vc) + slot * features + h * D + 32 * g;
    st_nt(reinterpret_cast<uint4 *>(kq), make_uint4(ck.cw[0], ck.cw[1], ck.cw[2], ck.cw[3]));
    st_nt(reinterpret_cast<uint4 *>(kq) + 1, make_uint4(ck.cw[4], ck.cw[5], ck.cw[6], ck.cw[7]));
    st_nt(reinterpret_cast<uint4 *>(vq), make_uint4(cv.cw[0], cv.cw[1], cv.cw[2], cv.cw[3]));
    st_nt(reinterpret_cast<uint4 *>(vq) + 1, make_uint4(cv.cw[4], cv.cw[5], cv.cw[6], cv.cw[7]));
    if (g == 0)
      reinterpret_cast<float2 *>(a.scales)[slot * a.hkv + h] = make_float2(ck.scale, cv.scale);
  } else {
    uint32_t stop = (ck.fail || cv.fail) ? (uint32_t)g : 4u; // first failing block, 4 = none
    stop = min(stop, quad_xor1(stop));
    stop = min(stop, quad_xor2(stop));
    if (stop < 4u && g == 0)
      raise_bad(a.bad);
    if ((uint32_t)g >= stop)
      return;
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    const long long qoff = slot * row_bytes + 2 * (features / 32) + h * D + 32 * g;
    const long long doff = slot * row_bytes + 2 * (h * 4 + g);
    uint8_t *kc = static_cast<uint8_t *>(a.kc), *vc = static_cast<uint8_t *>(a.vc);
    st_nt(reinterpret_cast<uint4 *>(kc + qoff), make_uint4(ck.cw[0], ck.cw[1], ck.cw[2], ck.cw[3]));
    st_nt(reinterpret_cast<uint4 *>(kc + qoff) + 1, make_uint4(ck.cw[4], ck.cw[5], ck.cw[6], ck.cw[7]));
    st_nt(reinterpret_cast<uint4 *>(vc + qoff), make_uint4(cv.cw[0], cv.cw[1], cv.cw[2], cv.cw[3]));
    st_nt(reinterpret_cast<uint4 *>(vc + qoff) + 1, make_uint4(cv.cw[4], cv.cw[5], cv.cw[6], cv.cw[7]));
    *reinterpret_cast<uint16_t *>(kc + doff) = ck.d;
    *reinterpret_cast<uint16_t *>(vc + doff) = cv.d;
  }
}

// LDS image of a quad block: the activation pieces (BF16: 4 per lane, slots 0..255;
// fp32: 8 per lane, slots 0..511) and, for fp32 activations, the BF16 cache rows of the
// block's heads behind them (slots 512..767).  The fp32 pieces of one lane are 64 slots
// apart, rotated by 2 per piece: the eight lanes writing one owner's pieces and the eight
// writing the next owner's fall into sixteen different slots mod 16, and so do sixteen
// lanes reading their own piece p.
template <class T> constexpr int quad_image_slots() {
  return std::is_same<T, uint16_t>::value ? 256 : 768;
}
// With a quantized cache the K waves also stage their V heads, behind the K pieces.
template <class T, int FMT> constexpr int quad_image_slots_fmt() {
  return FMT > PADRA_KV_BF16 ? (std::is_same<T, uint16_t>::value ? 512 : 1024)
                             : quad_image_slots<T>();
}
template <class T> __device__ __forceinline__ int quad_piece_slot(int owner, int p) {
  if constexpr (std::is_same<T, uint16_t>::value)
    return quad_slot(owner, p);
  else
    return p * 64 + ((owner + 2 * p) & 63);
}

// FMT: -1 (no cache), PADRA_KV_BF16, or a quantized cache format.
// `stage`: quad_image_slots<T>() uint4 of LDS (the block's transposition image), owned by
// the caller.
// FAST: the order-free sum of squares (sumsq_margin, common.h) with the tree as fallback;
// measured slower with a quantized cache and on fp32 activations, which keep the tree.
template <class T, int FMT, bool FAST = (FMT <= PADRA_KV_BF16 && std::is_same<T, uint16_t>::value)>
__device__ __forceinline__ void qk_heads_wave_quad(const QKArgs<T> &a, long long wave,
                                                   uint4 *stage) {
  constexpr int D = 128;
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int PL = F32 ? 8 : 4; // 16-byte pieces per lane
  constexpr int CH = 4 * PL;      // 16-byte chunks per head
  // Per head of the block: 1 = write the activation, 0 = write nothing; and the element
  // offset of its BF16 cache row (-1 = no cache write).
  __shared__ int head_live[16];
  __shared__ long long head_row[16];
  const int lane = threadIdx.x & 63, g = lane & 3;
  const unsigned block0 = (unsigned)wave * 16u;
  const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned total = nq + nk + (FMT >= 0 ? nk : 0u);
  // Flat head index (q heads, k heads, v heads) of block slot j, or `total` for none.
  // Quantized caches: the Q heads fill the first qk_q_waves waves, 16 per wave; every
  // later wave takes 16 K heads and stages their 16 V heads too, so that one quad holds
  // both vectors of a (token, KV head) pair, as the encoder needs.  Otherwise slots
  // follow the flat order.
  const unsigned nqw = (nq + 15u) / 16u;
  const bool kv_wave = FMT > PADRA_KV_BF16 && (unsigned)wave >= nqw; // wave-uniform
  auto slot_head = [&](unsigned j) -> unsigned {
    if constexpr (FMT > PADRA_KV_BF16) {
      if ((unsigned)wave < nqw) {
        const unsigned h = (unsigned)wave * 16u + j;
        return h < nq ? h : total;
      }
      const unsigned kvi = ((unsigned)wave - nqw) * 16u + j;
      return kvi < nk ? nq + kvi : total;
    } else {
      const unsigned h = block0 + j;
      return h < total ? h : total;
    }
  };
  if constexpr (FMT == PADRA_KV_BF16 && !F32) {
    if (block0 >= nq + nk) { // wave-uniform
      v_rows_copy16(a, block0, nq, nk);
      return;
    }
  }

  // This lane's head and warp group; its control record is requested first.
  const unsigned hv = slot_head((unsigned)(lane >> 2));
  const bool live = hv < total;
  const int role = hv < nq ? 0 : (hv < nq + nk ? 1 : 2); // 0 q, 1 k, 2 v
  const unsigned idx = role == 0 ? hv : (role == 1 ? hv - nq : hv - nq - nk);
  const unsigned heads = role == 0 ? (unsigned)a.hq : (unsigned)a.hkv;
  const int t = live ? (int)(idx / heads) : 0;
  const int hh = live ? (int)(idx - (unsigned)t * heads) : 0;
  const PosState ps = fetch_state(a.pos, t);

  // A block of 16 live heads of one role (every block when the head counts divide into
  // blocks) is 16 consecutive head vectors: its pieces are 64 m + lane 16-byte units from
  // the block's first vector, with no per-piece head lookup.
  const unsigned h0 = slot_head(0u);
  const bool whole = slot_head(15u) == h0 + 15u &&
                     (h0 + 15u < nq || (h0 >= nq && h0 + 15u < nq + nk)); // wave-uniform
  const uint4 *block = reinterpret_cast<const uint4 *>(head_src(a, whole ? h0 : 0u, nq, nk));
  const uint4 *vblock = reinterpret_cast<const uint4 *>(a.v + (size_t)(whole && h0 >= nq ? h0 - nq : 0u) * D);

  // 1. PL coalesced loads per lane (clamped, unconditional), for the LDS image.
  uint4 in[PL];
  if (whole) {
#pragma unroll
    for (int m = 0; m < PL; ++m)
      in[m] = ld_nt(block + 64 * m + lane);
  } else {
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      const int c = 64 * m + lane;
      const unsigned hc = min(slot_head((unsigned)(c / CH)), total - 1u);
      in[m] = ld_nt(reinterpret_cast<const uint4 *>(head_src(a, hc, nq, nk)) + (c % CH));
    }
  }
  // The V heads of a K wave (quantized cache), the same pieces of a.v.
  uint4 inv_[FMT > PADRA_KV_BF16 ? PL : 1];
  if constexpr (FMT > PADRA_KV_BF16) {
    if (kv_wave) {
      if (whole) {
#pragma unroll
        for (int m = 0; m < PL; ++m)
          inv_[m] = ld_nt(vblock + 64 * m + lane);
      } else {
#pragma unroll
        for (int m = 0; m < PL; ++m) {
          const int c = 64 * m + lane;
          const unsigned hc = min(slot_head((unsigned)(c / CH)), nq + nk - 1u) - nq;
          inv_[m] = ld_nt(reinterpret_cast<const uint4 *>(a.v + (size_t)hc * D) + (c % CH));
        }
      }
    }
  }
  // 2. The norm weights of the group (independent of the position), the head's position
  // (its control record was requested first), then the table loads, so that they are in
  // flight with the data loads.
  const uint16_t *wsrc = (role == 1 ? a.kn : a.qn) + 32 * g;
  Bf8 w8[4], c8[4], s8[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    w8[m].load(wsrc + 8 * m);
  bool ok = false;
  int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first, FMT > PADRA_KV_BF16,
                             ok);
  ok = ok && live && pos >= 0 && pos < a.table_rows;
  if (live && !ok && g == 0)
    raise_bad(a.bad);
  // The table entries of the group's pair index (f mod 64).
  const uint16_t *row = a.table + (size_t)(ok ? pos : 0) * D + 32 * (g & 1);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    c8[m].load(row + 8 * m);
    s8[m].load(row + 64 + 8 * m);
  }
  // 3. The data into the image.
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    const int c = 64 * m + lane;
    stage[quad_piece_slot<T>(4 * (c / CH) + (c % CH) / PL, c % PL)] = in[m];
  }
  constexpr int VIMG = 64 * PL; // V pieces behind the K pieces
  if constexpr (FMT > PADRA_KV_BF16) {
    if (kv_wave) {
#pragma unroll
      for (int m = 0; m < PL; ++m) {
        const int c = 64 * m + lane;
        stage[VIMG + quad_piece_slot<T>(4 * (c / CH) + (c % CH) / PL, c % PL)] = inv_[m];
      }
    }
  }
  __syncthreads();
  Act32<T> x;
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const uint4 v = stage[quad_piece_slot<T>(lane, p)];
    if constexpr (F32)
      x.f[p] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                           __uint_as_float(v.w));
    else
      x.w[p] = v;
  }

  uint32_t out[16];
  const bool qk = live && ok && role < 2;
  if (qk) {
    // FAST: the order-free sum over the quad (sumsq_margin), with the reference's tree as
    // its rarely taken (quad-uniform) fallback; otherwise the tree alone.  The tree: warp
    // g's in lane g, then (w0 + w2) at g = 0 and (w1 + w3) at g = 1, then their sum at
    // g = 0.
    float sum;
    auto tree = [&](auto depth_first) {
      float S, E;
      if constexpr (decltype(depth_first)::value)
        group_sumsq_df(x, S, E);
      else
        group_sumsq(x, S, E);
      const float s2 = fquad_xor2(S), e2 = fquad_xor2(E);
      fold(s2, e2, S, E);
      const float s1 = fquad_xor1(S), e1 = fquad_xor1(E);
      fold(s1, e1, S, E);
      return fquad_first(S + E);
    };
    if constexpr (FAST) {
      double a4[4] = {0.0, 0.0, 0.0, 0.0}; // independent fp64 chains
#pragma unroll
      for (int f = 0; f < 32; ++f)
        a4[f & 3] = F32 ? sq64_rn(x.get(f), a4[f & 3]) : sq64(x.get(f), a4[f & 3]);
      double acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
      acc = acc + lane_xor<2>(acc);
      acc = acc + lane_xor<1>(acc);
      if (!certified_sum(acc, sumsq_margin(1, 12), sum))
        sum = tree(std::true_type{});
    } else {
      sum = tree(std::false_type{});
    }
    const float inv = 1.f / sqrtf(sum / (float)D + a.eps);
    // Normalized group: A = B(B(x * inv) * w) (qk_rope_store_exact.cuh:39), as floats.
    float an[32];
#pragma unroll
    for (int f = 0; f < 32; ++f)
      an[f] = B(B(x.get(f) * inv) * w8[f / 8].get(f & 7));
    // Partner group (features f +- 64, lane g ^ 2): lower lanes rotate lo = A c - P s,
    // upper lanes hi = A c + P s (c, s of the pair index).  B(-P s) = B(P (-s)): the lower
    // lanes flip the sign bits of their s words.
    const uint32_t sgn = g < 2 ? 0x80008000u : 0u;
    bool fine = isfinite(sum);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int k0 = 2 * i, k1 = 2 * i + 1;
      const float c0 = c8[k0 / 8].get(k0 & 7), c1 = c8[k1 / 8].get(k1 & 7);
      const uint32_t sword = s8[k0 / 8].word((k0 & 7) / 2) ^ sgn;
      const float s0 = lo16(sword), s1 = hi16(sword);
      const float r0 = B(an[k0] * c0) + B(fquad_xor2(an[k0]) * s0);
      const float r1 = B(an[k1] * c1) + B(fquad_xor2(an[k1]) * s1);
      fine = fine && bf16_finite_after_round(r0) && bf16_finite_after_round(r1);
      out[i] = pack2(r0, r1);
    }
    if (!fine)
      raise_bad(a.bad);
  }
  if constexpr (FMT > PADRA_KV_BF16) {
    if (kv_wave) {
      // Each quad encodes its K head (the rotated values) with the V head of the same
      // (token, KV head) from the V image.
      Act32<T> xv;
#pragma unroll
      for (int p = 0; p < PL; ++p) {
        const uint4 v = stage[VIMG + quad_piece_slot<T>(lane, p)];
        if constexpr (F32)
          xv.f[p] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                                __uint_as_float(v.z), __uint_as_float(v.w));
        else
          xv.w[p] = v;
      }
      const bool enc = live && ok && t >= a.first;
      const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
      const long long slot = seq * a.seq_stride + (ok ? ring_slot(pos, max(a.cap, 1)) : 0);
      float xe[32];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xe[2 * i] = lo16(out[i]);
        xe[2 * i + 1] = hi16(out[i]);
      }
      encode_pair_quad<FMT>(a, xe, xv, slot, hh, g, enc);
    }
  }
  __syncthreads(); // every lane has read its input pieces: the image can be overwritten

  // 4. Outputs back into the image, then coalesced stores.
  const bool vcopy = FMT == PADRA_KV_BF16 && live && ok && role == 2 && t >= a.first;
  if (qk) {
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      if constexpr (F32) {
        const uint32_t l = out[2 * p], u = out[2 * p + 1];
        stage[quad_piece_slot<T>(lane, p)] =
            make_uint4(l << 16, l & 0xffff0000u, u << 16, u & 0xffff0000u);
      } else {
        stage[quad_piece_slot<T>(lane, p)] =
            make_uint4(out[4 * p], out[4 * p + 1], out[4 * p + 2], out[4 * p + 3]);
      }
    }
  }
  if constexpr (F32 && FMT == PADRA_KV_BF16) {
    // The BF16 cache rows: rotated K, or V rounded to BF16 (the reference stores
    // bf16(v), prefill_control.cuh:36-37).
    if (role == 1 ? qk : vcopy) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = role == 1 ? out[4 * p + i] : pack2(x.get(8 * p + 2 * i), x.get(8 * p + 2 * i + 1));
        stage[512 + quad_slot(lane, p)] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
  const int features = a.hkv * D;
  if (g == 0) {
    head_live[lane >> 2] = (qk || vcopy) ? 1 : 0;
    long long r = -1;
    if (FMT == PADRA_KV_BF16 && live && ok && role >= 1 && t >= a.first) {
      const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
      r = (seq * a.seq_stride + ring_slot(pos, a.cap)) * features + hh * D;
    }
    head_row[lane >> 2] = r;
  }
  __syncthreads();
  if constexpr (F32) {
    // fp32 activations of the Q and K heads: eight 1 KB stores per lane.
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      const int c = 64 * m + lane, j = c / CH, ci = c % CH;
      if (whole) {
        if (head_live[j])
          st_nt(const_cast<uint4 *>(block) + c, stage[quad_piece_slot<T>(4 * j + ci / PL, ci % PL)]);
        continue;
      }
      const unsigned hc = slot_head((unsigned)j);
      if (!head_live[j] || hc >= nq + nk)
        continue;
      const uint4 d = stage[quad_piece_slot<T>(4 * j + ci / PL, ci % PL)];
      st_nt(reinterpret_cast<uint4 *>(const_cast<T *>(head_src(a, hc, nq, nk))) + ci, d);
    }
    if constexpr (FMT == PADRA_KV_BF16) {
      // BF16 cache rows of the K and V heads: four 1 KB stores per lane.
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int c = 64 * m + lane, j = c >> 4, ci = c & 15;
        const long long r = head_row[j];
        if (!head_live[j] || r < 0)
          continue;
        const unsigned hc = slot_head((unsigned)j);
        const uint4 d = stage[512 + quad_slot(4 * j + (ci >> 2), ci & 3)];
        uint16_t *cache = static_cast<uint16_t *>(hc >= nq + nk ? a.vc : a.kc);
        st_nt(reinterpret_cast<uint4 *>(cache + r) + ci, d);
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = 64 * m + lane, j = c >> 4, ci = c & 15;
      if (!head_live[j])
        continue; // past the end, or a head that writes nothing
      const uint4 d = stage[quad_slot(4 * j + (ci >> 2), ci & 3)];
      if (whole) { // Q or K heads of one block
        st_nt(const_cast<uint4 *>(block) + c, d);
        if constexpr (FMT == PADRA_KV_BF16) {
          const long long r = head_row[j];
          if (r >= 0)
            st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.kc) + r) + ci, d);
        }
        continue;
      }
      const unsigned hc = slot_head((unsigned)j);
      if constexpr (FMT == PADRA_KV_BF16) {
        const long long r = head_row[j];
        if (hc >= nq + nk) { // V head: cache only
          st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.vc) + r) + ci, d);
          continue;
        }
        st_nt(reinterpret_cast<uint4 *>(const_cast<uint16_t *>(head_src(a, hc, nq, nk))) + ci, d);
        if (r >= 0)
          st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.kc) + r) + ci, d);
      } else {
        st_nt(reinterpret_cast<uint4 *>(const_cast<uint16_t *>(head_src(a, hc, nq, nk))) + ci, d);
      }
    }
  }
}

// Waves of a Q/K launch: 16 head vectors per wave in the flat order (no cache, BF16
// cache), or the Q waves and then the K waves (16 K heads with their V heads) of a
// quantized cache.
template <int FMT>
__host__ __device__ inline long long qk_wave_count(int tokens, int q_heads, int kv_heads) {
  const long long nq = (long long)tokens * q_heads, nk = (long long)tokens * kv_heads;
  if (FMT > PADRA_KV_BF16)
    return (nq + 15) / 16 + (nk + 15) / 16;
  return (nq + nk * (FMT >= 0 ? 2 : 1) + 15) / 16;
}
// The waves holding Q heads only, before the K-with-V waves of a quantized cache.
__host__ __device__ inline long long qk_q_waves(int tokens, int q_heads) {
  return ((long long)tokens * q_heads + 15) / 16;
}

// Four lanes per head for both activation types.
template <class T, int FMT>
__device__ __forceinline__ void qk_heads_wave(const QKArgs<T> &a, long long wave, uint4 *lds) {
  qk_heads_wave_quad<T, FMT>(a, wave, lds);
}

} // namespace padra
