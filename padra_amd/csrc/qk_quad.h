// Q/K RMSNorm + NeoX RoPE (+ BF16 KV store) with four lanes per head: lane 4j + g owns
// features 32g .. 32g+31 of head j, i.e. exactly reference warp g of the head's 128-thread
// block (qk_rope_store_exact.cuh:28-44, inference.cu:110-135).  A wave covers 16 heads.
//
//  - Warp g's shuffle-down tree runs inside lane g.
//  - The tree over the four warp partials, (w0 + w2) + (w1 + w3), is two DPP quad
//    exchanges (lanes g^2, then g^1), then a broadcast from lane g = 0.
//  - RoPE pairs feature f < 64 with f + 64, i.e. lane g with lane g^2: the partner's
//    normalized values arrive packed, sixteen DPP moves per lane.
// Loads and stores of the 4 KB block are four coalesced 1 KB instructions, transposed
// through LDS as in the lane-pair path.
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
  uint4 d[4];
  PosState ps[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const unsigned idx = min(block0 + (unsigned)((64 * m + lane) >> 4) - nq - nk, nk - 1u);
    ps[m] = fetch_state(a.pos, (int)(idx / (unsigned)a.hkv));
    d[m] = ld_nt(reinterpret_cast<const uint4 *>(a.v + (size_t)idx * D) + ((64 * m + lane) & 15));
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 64 * m + lane;
    const unsigned idx = block0 + (unsigned)(c >> 4) - nq - nk;
    if (idx >= nk)
      continue;
    const int t = (int)(idx / (unsigned)a.hkv), h = (int)(idx % (unsigned)a.hkv), ci = c & 15;
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
    const long long slot = seq * a.seq_stride + pos % a.cap;
    st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.vc) + slot * features + h * D) + ci, d[m]);
  }
}

// FMT: -1 (no cache) or PADRA_KV_BF16.
template <int FMT>
__device__ __forceinline__ void qk_heads_wave_quad(const QKArgs<uint16_t> &a, long long wave) {
  constexpr int D = 128;
  __shared__ uint4 stage[256];
  __shared__ int head_pos[16]; // per head of the block: cache position, -1 = write nothing
  const int lane = threadIdx.x & 63, g = lane & 3;
  const unsigned block0 = (unsigned)wave * 16u;
  const unsigned nq = (unsigned)a.tokens * (unsigned)a.hq;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned total = nq + nk + (FMT >= 0 ? nk : 0u);
  if constexpr (FMT == PADRA_KV_BF16) {
    if (block0 >= nq + nk) { // wave-uniform
      v_rows_copy16(a, block0, nq, nk);
      return;
    }
  }

  // This lane's head and warp group; its control record is requested first.
  const unsigned hv = block0 + (unsigned)(lane >> 2);
  const bool live = hv < total;
  const int role = hv < nq ? 0 : (hv < nq + nk ? 1 : 2); // 0 q, 1 k, 2 v
  const unsigned idx = role == 0 ? hv : (role == 1 ? hv - nq : hv - nq - nk);
  const unsigned heads = role == 0 ? (unsigned)a.hq : (unsigned)a.hkv;
  const int t = live ? (int)(idx / heads) : 0;
  const PosState ps = fetch_state(a.pos, t);

  // 1. Four coalesced loads per lane (clamped, unconditional), into the LDS image.
  uint4 in[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 64 * m + lane;
    const unsigned hc = min(block0 + (unsigned)(c >> 4), total - 1u);
    in[m] = ld_nt(reinterpret_cast<const uint4 *>(head_src(a, hc, nq, nk)) + (c & 15));
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 64 * m + lane;
    stage[quad_slot(4 * (c >> 4) + ((c & 15) >> 2), c & 3)] = in[m];
  }

  // 2. The head's position.
  bool ok = false;
  int pos = resolve_position(a.pos, ps, t, FMT >= 0 ? a.cap : 0, a.first, false, ok);
  ok = ok && live && pos >= 0 && pos < a.table_rows;
  if (live && !ok && g == 0)
    raise_bad(a.bad);
  // Norm weights of the group and the table entries of its pair index (f mod 64).
  const uint16_t *wsrc = (role == 1 ? a.kn : a.qn) + 32 * g;
  const uint16_t *row = a.table + (size_t)(ok ? pos : 0) * D + 32 * (g & 1);
  Bf8 w8[4], c8[4], s8[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    w8[m].load(wsrc + 8 * m);
    c8[m].load(row + 8 * m);
    s8[m].load(row + 64 + 8 * m);
  }
  __syncthreads();
  Act32<uint16_t> x;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    x.w[p] = stage[quad_slot(lane, p)];

  uint32_t out[16];
  const bool qk = live && ok && role < 2;
  if (qk) {
    float S, E;
    group_sumsq(x, S, E);
    // (w0 + w2) at g = 0 and (w1 + w3) at g = 1, then their sum at g = 0.
    {
      const float s2 = fquad_xor2(S), e2 = fquad_xor2(E);
      fold(s2, e2, S, E);
      const float s1 = fquad_xor1(S), e1 = fquad_xor1(E);
      fold(s1, e1, S, E);
    }
    const float sum = fquad_first(S + E);
    const float inv = 1.f / sqrtf(sum / (float)D + a.eps);
    // Normalized group, packed: A = B(B(x * inv) * w) (qk_rope_store_exact.cuh:39).
    uint32_t an[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t p1 = pack2(x.get(2 * i) * inv, x.get(2 * i + 1) * inv);
      an[i] = pack2(lo16(p1) * w8[i / 4].get((2 * i) & 7), hi16(p1) * w8[i / 4].get((2 * i + 1) & 7));
    }
    // Partner group (features f +- 64): lower lanes rotate lo = A c - P s, upper lanes
    // hi = A c + P s (c, s of the pair index).
    // B(-P s) = -B(P s): the lower lanes flip the partner's sign bits.
    const uint32_t sgn = g < 2 ? 0x80008000u : 0u;
    bool fine = isfinite(sum);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pw = quad_xor2(an[i]) ^ sgn;
      const int k0 = 2 * i, k1 = 2 * i + 1;
      const float c0 = c8[k0 / 8].get(k0 & 7), c1 = c8[k1 / 8].get(k1 & 7);
      const float s0 = s8[k0 / 8].get(k0 & 7), s1 = s8[k1 / 8].get(k1 & 7);
      const uint32_t p3 = pack2(lo16(an[i]) * c0, hi16(an[i]) * c1);
      const uint32_t p4 = pack2(lo16(pw) * s0, hi16(pw) * s1);
      const float r0 = lo16(p3) + lo16(p4), r1 = hi16(p3) + hi16(p4);
      fine = fine && bf16_finite_after_round(r0) && bf16_finite_after_round(r1);
      out[i] = pack2(r0, r1);
    }
    if (!fine)
      raise_bad(a.bad);
  }
  __syncthreads(); // every lane has read its input pieces: the image can be overwritten

  // 3. Outputs back into the image, then four coalesced stores per lane.
  if (qk) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      stage[quad_slot(lane, p)] = make_uint4(out[4 * p], out[4 * p + 1], out[4 * p + 2], out[4 * p + 3]);
  }
  const bool vcopy = FMT == PADRA_KV_BF16 && live && ok && role == 2 && t >= a.first;
  if (g == 0)
    head_pos[lane >> 2] = (qk || vcopy) ? pos : -1;
  __syncthreads();
  const int features = a.hkv * D;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 64 * m + lane, j = c >> 4, ci = c & 15;
    const unsigned hc = block0 + (unsigned)j;
    const int hp = head_pos[j];
    if (hp < 0)
      continue; // past the end, or a head that writes nothing
    const uint4 d = stage[quad_slot(4 * j + (ci >> 2), ci & 3)];
    if constexpr (FMT == PADRA_KV_BF16) {
      if (hc >= nq + nk) { // V head: cache only
        const unsigned vi = hc - nq - nk;
        const int tc = (int)(vi / (unsigned)a.hkv), hh = (int)(vi % (unsigned)a.hkv);
        const long long sq = a.pos.mode == PADRA_POS_DECODE ? tc : 0;
        const long long sl = sq * a.seq_stride + hp % a.cap;
        st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.vc) + sl * features + hh * D) + ci, d);
        continue;
      }
    }
    st_nt(reinterpret_cast<uint4 *>(const_cast<uint16_t *>(head_src(a, hc, nq, nk))) + ci, d);
    if constexpr (FMT == PADRA_KV_BF16) {
      if (hc >= nq) {
        const unsigned kvi = hc - nq;
        const int tc = (int)(kvi / (unsigned)a.hkv), hh = (int)(kvi % (unsigned)a.hkv);
        if (tc >= a.first) {
          const long long sq = a.pos.mode == PADRA_POS_DECODE ? tc : 0;
          const long long sl = sq * a.seq_stride + hp % a.cap;
          st_nt(reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.kc) + sl * features + hh * D) + ci, d);
        }
      }
    }
  }
}

// Head vectors per wave of each Q/K kernel variant.
template <class T, int FMT> constexpr int qk_heads_per_wave() {
  return std::is_same<T, uint16_t>::value && FMT <= PADRA_KV_BF16 ? 16 : 32;
}

// BF16 without a cache or with a BF16 cache: four lanes per head; quantized caches and
// fp32 activations: two lanes per head.
template <class T, int FMT>
__device__ __forceinline__ void qk_heads_wave(const QKArgs<T> &a, long long wave) {
  if constexpr (std::is_same<T, uint16_t>::value) {
    if constexpr (FMT <= PADRA_KV_BF16)
      qk_heads_wave_quad<FMT>(a, wave);
    else
      qk_heads_wave_staged<FMT>(a, wave);
  } else {
    qk_heads_wave_direct<T, FMT>(a, wave);
  }
}

} // namespace padra
