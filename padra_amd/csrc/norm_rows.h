// Residual-add + RMSNorm over hidden rows: one 64-lane wavefront per row.
//
// The sum of squares: where a kernel takes the order-free fp64 sum (sumsq_margin,
// common.h), the tree below is its rarely taken fallback; elsewhere it is the sum.
//
// Reference: Add + Norm (inference.cu:475-481, 188-214) for VT = 128 and
// ResidualPostNormWideExact (residual_norm_wide_exact.cuh:6-80) for VT = 256.  The
// reference block has VT threads; thread t owns elements t, t+VT, t+2VT, ... and sums
// their squares in that order, then a 32-lane shuffle-down tree per warp and one more
// tree over the warp partials.  Here lane l owns the K = VT/64 consecutive threads
// K*l .. K*l+K-1, so one K-element load per j lands exactly the elements those threads
// own, and the same tree is replayed: tree levels d >= K cross lanes (lane l folds lane
// l + d/K, a DPP row shift), levels d < K stay inside the lane, and the warp partials
// sit in lanes 0, 32/K, 64/K, ... .  Levels of the final tree that only add zero lanes
// are exact no-ops and are skipped.  The result is bit-identical to the reference's
// fadd(sum, error).
//
// Memory schedule: every load of the row (x, residual, gamma) is issued before the first
// store, so the wave pays one HBM round trip, not one per 16-byte slice (an in-place
// store to x may alias the residual for all the compiler knows, which would otherwise
// pin each load behind the previous store).
#pragma once
#include <type_traits>

#include "common.h"

namespace padra {

template <class T> struct NormArgs {
  T *x;
  const T *residual;
  T *y;
  const uint16_t *gamma;
  float *stats;
  int *bad;
  int rows;
  float eps;
  // Embedding gather in front of the residual add (the fused decode step): row t's x is
  // gather[token_t] ([vocab][H] BF16); a row whose token is invalid raises the flag and
  // reads x as it is, as the separate gather launch would have left it.
  const uint16_t *gather = nullptr;
  const int32_t *ids = nullptr;
  int vocab = 0;
  PosSrc src{};
};

// Largest |y| whose BF16 rounding stays finite: 0x7f7f8000 is the midpoint between the
// largest finite BF16 (0x7f7f, odd) and infinity, and it rounds to infinity.
__device__ __forceinline__ bool bf16_finite_after_round(float y) {
  return fabsf(y) < __uint_as_float(0x7f7f8000u);
}

// K consecutive activations: K BF16 (K*2 bytes) or K fp32.
template <class T, int K> struct Lanes;
template <int K> struct Lanes<uint16_t, K> {
  uint32_t w[K / 2];
  template <bool NT = true> __device__ __forceinline__ void load(const uint16_t *p) {
    if constexpr (K == 2) {
      w[0] = NT ? ld_nt(reinterpret_cast<const uint32_t *>(p)) : *reinterpret_cast<const uint32_t *>(p);
    } else {
      const uint2 v = NT ? ld_nt(reinterpret_cast<const uint2 *>(p)) : *reinterpret_cast<const uint2 *>(p);
      w[0] = v.x;
      w[1] = v.y;
    }
  }
  __device__ __forceinline__ float get(int i) const { return i & 1 ? hi16(w[i / 2]) : lo16(w[i / 2]); }
  template <bool WT = false>
  static __device__ __forceinline__ void store(uint16_t *p, const uint32_t *w) {
    if constexpr (K == 2)
      st_stream<WT>(reinterpret_cast<uint32_t *>(p), w[0]);
    else
      st_stream<WT>(reinterpret_cast<uint2 *>(p), make_uint2(w[0], w[1]));
  }
};
template <int K> struct Lanes<float, K> {
  float f[K];
  template <bool NT = true> __device__ __forceinline__ void load(const float *p) {
    if constexpr (K == 2) {
      const uint2 v = ld_nt(reinterpret_cast<const uint2 *>(p));
      f[0] = __uint_as_float(v.x);
      f[1] = __uint_as_float(v.y);
    } else {
      const uint4 v = ld_nt(reinterpret_cast<const uint4 *>(p));
      f[0] = __uint_as_float(v.x);
      f[1] = __uint_as_float(v.y);
      f[2] = __uint_as_float(v.z);
      f[3] = __uint_as_float(v.w);
    }
  }
  __device__ __forceinline__ float get(int i) const { return f[i]; }
  template <bool WT = false>
  static __device__ __forceinline__ void store(float *p, const uint32_t *w) {
    if constexpr (K == 2)
      st_stream<WT>(reinterpret_cast<uint2 *>(p), make_uint2(w[0] << 16, w[0] & 0xffff0000u));
    else
      st_stream<WT>(reinterpret_cast<uint4 *>(p), make_uint4(w[0] << 16, w[0] & 0xffff0000u, w[1] << 16,
                                                     w[1] & 0xffff0000u));
  }
};

// Value of lane (lane + L) for L < 16 inside the same 16-lane DPP row (row_shl:L), and
// through the LDS crossbar (ds_bpermute) for longer strides.  Lanes whose source falls
// outside the row read garbage; the trees below never consume those lanes.
template <int L> __device__ __forceinline__ float lane_down(float v) {
  if constexpr (L < 16)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + L, 0xf, 0xf, false));
  else
    return __shfl_down(v, L, 64);
}

// Folds lane + L's partial into this lane's for every slot (one tree level).
template <int L, int K>
__device__ __forceinline__ void fold_lanes(float (&s)[K], float (&e)[K]) {
  float s2[K], e2[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s2[k] = lane_down<L>(s[k]);
    e2[k] = lane_down<L>(e[k]);
  }
#pragma unroll
  for (int k = 0; k < K; ++k)
    fold(s2[k], e2[k], s[k], e[k]);
}

// One level of the 32-thread warp tree (inference.cu:111-119) for lanes owning K
// consecutive threads: d >= K folds lane + d/K, d < K folds slot k + d into slot k.
template <int D, int K>
__device__ __forceinline__ void warp_level(float (&s)[K], float (&e)[K]) {
  if constexpr (D >= K) {
    fold_lanes<D / K, K>(s, e);
  } else {
#pragma unroll
    for (int k = 0; k < D; ++k)
      fold(s[k + D], e[k + D], s[k], e[k]);
  }
}
template <int K> __device__ __forceinline__ void warp_tree(float (&s)[K], float (&e)[K]) {
  warp_level<16, K>(s, e);
  warp_level<8, K>(s, e);
  warp_level<4, K>(s, e);
  warp_level<2, K>(s, e);
  warp_level<1, K>(s, e);
}
// Tree over WARPS warp partials held by lanes 0, LPW, 2*LPW, ... (inference.cu:120-135).
template <int WARPS, int LPW>
__device__ __forceinline__ void partials_tree(float &S, float &E) {
  if constexpr (WARPS >= 2) {
    constexpr int D = WARPS / 2;
    const float s2 = lane_down<D * LPW>(S), e2 = lane_down<D * LPW>(E);
    fold(s2, e2, S, E);
    partials_tree<D, LPW>(S, E);
  }
}

// One row's raw inputs in registers (x, residual), as loaded by norm_load.
template <int VT, int J, class T> struct RowIn {
  Lanes<T, VT / 64> x[J], r[J];
};

template <int VT, int J, class T, bool RES>
__device__ __forceinline__ void norm_load(const NormArgs<T> &a, int row, RowIn<VT, J, T> &in) {
  constexpr int K = VT / 64, H = VT * J;
  const size_t off = (size_t)row * H + K * (threadIdx.x & 63);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    in.x[j].load(a.x + off + VT * j);
    if constexpr (RES)
      in.r[j].load(a.residual + off + VT * j);
  }
}

// norm_load with the embedding gather: the residual loads first, then the token (its
// control record) and the embedding row.
template <int VT, int J>
__device__ __forceinline__ void norm_load_gather(const NormArgs<uint16_t> &a, int row,
                                                 RowIn<VT, J, uint16_t> &in) {
  constexpr int K = VT / 64, H = VT * J;
  const int lane = threadIdx.x & 63;
  const size_t off = (size_t)row * H + K * lane;
#pragma unroll
  for (int j = 0; j < J; ++j)
    in.r[j].load(a.residual + off + VT * j);
  bool ok;
  const int token = embed_token(a.src, a.ids, row, a.vocab, ok);
  if (!ok && lane == 0)
    raise_bad(a.bad);
  const uint16_t *src = ok ? a.gather + (size_t)token * H + K * lane : a.x + off;
#pragma unroll
  for (int j = 0; j < J; ++j)
    in.x[j].load(src + VT * j);
}

template <int VT, int J>
__device__ __forceinline__ void norm_load_gamma(const uint16_t *gamma,
                                                Lanes<uint16_t, VT / 64> (&gr)[J]) {
  constexpr int K = VT / 64;
#pragma unroll
  for (int j = 0; j < J; ++j)
    gr[j].template load<false>(gamma + K * (threadIdx.x & 63) + VT * j);
}

// The reference's per-thread compensated sums over packed v words (lane l: threads
// K l .. K l + K - 1, words vp[j][w]) and its tree: the row's total in every lane.
template <int VT, int J>
__device__ __forceinline__ float ordered_total(const uint32_t (&vp)[J][VT / 128]) {
  constexpr int K = VT / 64, LPW = 32 / K, WARPS = VT / 32;
  float s[K], e[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s[k] = 0.f;
    e[k] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
#pragma unroll
    for (int w = 0; w < K / 2; ++w) {
      const float v0 = lo16(vp[j][w]), v1 = hi16(vp[j][w]);
      acc_pos(v0 * v0, s[2 * w], e[2 * w]);
      acc_pos(v1 * v1, s[2 * w + 1], e[2 * w + 1]);
    }
  }
  warp_tree<K>(s, e);
  float S = s[0], E = e[0];
  partials_tree<WARPS, LPW>(S, E);
  // lane 0's total through ds_bpermute: a v_readlane here measured 0.8% slower on the
  // quantized chunk chains (13.76 -> 13.89 us, q8_0)
  return __shfl(S + E, 0, 64);
}

// Everything after the loads: v = B(x + r), the sum of squares, the outputs.  FAST: the
// order-free fp64 sum (sumsq_margin, common.h) with the reference tree as its rarely
// taken fallback; otherwise the reference tree alone.  The fast form is slower in the
// quantized-cache chain and on fp32 rows (both lose a wave of occupancy or its memory
// schedule to it), so those keep the tree.
template <int VT, int J, class T, bool RES, bool FAST = true>
__device__ __forceinline__ void norm_compute(const NormArgs<T> &a, int row,
                                             const RowIn<VT, J, T> &in,
                                             const Lanes<uint16_t, VT / 64> (&gr)[J]) {
  constexpr int K = VT / 64, H = VT * J, LPW = 32 / K, WARPS = VT / 32;
  const int lane = threadIdx.x & 63;
  const size_t off = (size_t)row * H + K * lane;
  uint32_t vp[J][K / 2];
  float total;
  if constexpr (FAST) {
    double acc[4] = {0.0, 0.0, 0.0, 0.0}; // independent fp64 chains
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
      for (int w = 0; w < K / 2; ++w) {
        const float a0 = RES ? in.x[j].get(2 * w) + in.r[j].get(2 * w) : in.x[j].get(2 * w);
        const float a1 =
            RES ? in.x[j].get(2 * w + 1) + in.r[j].get(2 * w + 1) : in.x[j].get(2 * w + 1);
        vp[j][w] = pack2(a0, a1);
        const int c = (2 * (j * (K / 2) + w)) & 3;
        acc[c] = sq64(lo16(vp[j][w]), acc[c]);
        acc[c + 1] = sq64(hi16(vp[j][w]), acc[c + 1]);
      }
    }
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < J; ++j)
        Lanes<T, K>::store(a.x + off + VT * j, vp[j]);
    }
    // keep the gamma loads ahead of the rarely taken branch below (see norm_row_wave_wide)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int w = 0; w < K / 2; ++w)
        pin(gr[j].w[w]);
    const double lane_sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if (!certified_sum(wave_sum64(lane_sum), sumsq_margin(J, J * K + 6), total))
      total = ordered_total<VT, J>(vp); // rare, wave-uniform
  } else {
    // The tree alone, its per-thread sums interleaved with v (this order schedules best).
    float s[K], e[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s[k] = 0.f;
      e[k] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
      for (int w = 0; w < K / 2; ++w) {
        const float a0 = RES ? in.x[j].get(2 * w) + in.r[j].get(2 * w) : in.x[j].get(2 * w);
        const float a1 =
            RES ? in.x[j].get(2 * w + 1) + in.r[j].get(2 * w + 1) : in.x[j].get(2 * w + 1);
        vp[j][w] = pack2(a0, a1);
        const float v0 = lo16(vp[j][w]), v1 = hi16(vp[j][w]);
        acc_pos(v0 * v0, s[2 * w], e[2 * w]);
        acc_pos(v1 * v1, s[2 * w + 1], e[2 * w + 1]);
      }
    }
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < J; ++j)
        Lanes<T, K>::store(a.x + off + VT * j, vp[j]);
    }
    warp_tree<K>(s, e);
    float S = s[0], E = e[0];
    partials_tree<WARPS, LPW>(S, E);
    // lane 0's total through ds_bpermute: a v_readlane here measured 0.8% slower on the
    // quantized chunk chains (13.76 -> 13.89 us, q8_0)
    total = __shfl(S + E, 0, 64);
  }
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && lane == 0) {
    a.stats[2 * row] = variance;
    a.stats[2 * row + 1] = inv;
  }
  // Error flag, as the reference kernels set it: with a residual, a non-finite v (Add,
  // inference.cu:479) shows as a non-finite row sum, and the 256-thread decode kernel also
  // checks the sum and every output (residual_norm_wide_exact.cuh:30, 61, 77); without a
  // residual, NormFP8Exact / NormFP8WideExact check every output (norm_fp8_exact.cuh:42).
  constexpr bool CHECK_Y = VT == 256 || !RES;
  bool fine = !RES || isfinite(total);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    uint32_t out[K / 2];
#pragma unroll
    for (int w = 0; w < K / 2; ++w) {
      const float y0 = B(lo16(vp[j][w]) * inv) * gr[j].get(2 * w);
      const float y1 = B(hi16(vp[j][w]) * inv) * gr[j].get(2 * w + 1);
      if constexpr (CHECK_Y)
        fine = fine && bf16_finite_after_round(y0) && bf16_finite_after_round(y1);
      out[w] = pack2(y0, y1);
    }
    Lanes<T, K>::store(a.y + off + VT * j, out);
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
}

// BF16 rows with 16-byte accesses.  Piece c of lane L is elements 512c + 8L .. 512c + 8L + 7
// of x, the residual, gamma and the outputs: every load and store of the row is a 1 KB
// coalesced instruction (4 per tensor at H = 2048, instead of 16 of 4 or 8 bytes).  The
// sum of squares is the order-free fp64 sum (sumsq_margin, common.h), so it needs no
// thread ownership; only its rare fallback, the reference's per-thread sums (thread t:
// elements t + VT j, summed in j order) and tree, sends v = B(x + r) across LDS once so
// that each lane can read the words of its K threads.
template <int VT, int J, bool RES>
__device__ __forceinline__ void norm_wide_finish(const NormArgs<uint16_t> &a, int row,
                                                 const uint4 (&xin)[(VT * J + 511) / 512],
                                                 const uint4 (&rin)[(VT * J + 511) / 512],
                                                 const uint4 (&gin)[(VT * J + 511) / 512],
                                                 uint4 *vlds);

// R consecutive rows per wave (row0 .. row0 + R - 1; rows past a.rows are skipped): the
// gamma pieces once, then every row's loads, then each row's arithmetic and stores.
template <int VT, int J, bool RES, int R = 1>
__device__ __forceinline__ void norm_row_wave_wide(const NormArgs<uint16_t> &a, int row0,
                                                   uint4 *vlds) {
  constexpr int H = VT * J, C = (H + 511) / 512;
  const int lane = threadIdx.x & 63;
  uint4 xin[R][C], rin[R][C], gin[C];
  // gamma first (cache-resident: it returns first), then x and the residual
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = (512 * c + 8 * lane < H) ? 512 * c + 8 * lane : 0; // clamped, unconditional
    gin[c] = *reinterpret_cast<const uint4 *>(a.gamma + e);
  }
  issue_point();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const size_t base = (size_t)min(row0 + r, a.rows - 1) * H;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int e = (512 * c + 8 * lane < H) ? 512 * c + 8 * lane : 0;
      xin[r][c] = ld_nt(reinterpret_cast<const uint4 *>(a.x + base + e));
      if constexpr (RES)
        rin[r][c] = ld_nt(reinterpret_cast<const uint4 *>(a.residual + base + e));
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (row0 + r < a.rows) // wave-uniform
      norm_wide_finish<VT, J, RES>(a, row0 + r, xin[r], rin[r], gin, vlds);
}

template <int VT, int J, bool RES>
__device__ __forceinline__ void norm_wide_finish(const NormArgs<uint16_t> &a, int row,
                                                 const uint4 (&xin)[(VT * J + 511) / 512],
                                                 const uint4 (&rin)[(VT * J + 511) / 512],
                                                 const uint4 (&gin)[(VT * J + 511) / 512],
                                                 uint4 *vlds) {
  constexpr int K = VT / 64, H = VT * J, C = (H + 511) / 512, LPW = 32 / K, WARPS = VT / 32;
  constexpr bool CHECK_Y = VT == 256 || !RES;
  const int lane = threadIdx.x & 63;
  const size_t base = (size_t)row * H;
  // v = B(x + r), packed, into x and LDS.
  uint4 vw[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if constexpr (RES) {
      const uint32_t xw[4] = {xin[c].x, xin[c].y, xin[c].z, xin[c].w};
      const uint32_t rw[4] = {rin[c].x, rin[c].y, rin[c].z, rin[c].w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = pack2(lo16(xw[k]) + lo16(rw[k]), hi16(xw[k]) + hi16(rw[k]));
      vw[c] = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
      vw[c] = xin[c];
    }
    if constexpr (RES)
      if (512 * c + 8 * lane < H)
        st_nt(reinterpret_cast<uint4 *>(a.x + base + 512 * c + 8 * lane), vw[c]);
  }
  // gamma is used only after the sum, past the rarely taken branch below; without this
  // use the compiler sinks its loads behind that branch, a memory round trip per row
  // (0.4 us per config-1 chunk).
#pragma unroll
  for (int c = 0; c < C; ++c)
    pin(gin[c]);
  // The order-free sum over the lane's valid pieces (the clamped pieces past H repeat
  // elements 0..7 and are left out).
  // Eight independent fp64 chains (a single one is a 32-deep dependent chain that the
  // wave waits on).
  double acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    acc[k] = 0.0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if (512 * c + 8 * lane < H) {
      const uint32_t vv[4] = {vw[c].x, vw[c].y, vw[c].z, vw[c].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[2 * k] = sq64(lo16(vv[k]), acc[2 * k]);
        acc[2 * k + 1] = sq64(hi16(vv[k]), acc[2 * k + 1]);
      }
    }
  }
  const double lane_sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  float total;
  if (!certified_sum(wave_sum64(lane_sum), sumsq_margin(J, C + 3 + 6), total)) {
    // Rare (wave-uniform): the reference's per-thread sums and tree.  v crosses LDS so
    // that lane l can read the words of threads K l .. K l + K - 1, i.e. the K / 2 words
    // K l / 2 + (VT / 2) j of the packed row.
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (512 * c + 8 * lane < H)
        vlds[64 * c + lane] = vw[c];
    __syncthreads();
    const uint32_t *vwords = reinterpret_cast<const uint32_t *>(vlds);
    float s[K], e[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s[k] = 0.f;
      e[k] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
      for (int w = 0; w < K / 2; ++w) {
        const uint32_t word = vwords[(K / 2) * lane + w + (VT / 2) * j];
        const float v0 = lo16(word), v1 = hi16(word);
        acc_pos(v0 * v0, s[2 * w], e[2 * w]);
        acc_pos(v1 * v1, s[2 * w + 1], e[2 * w + 1]);
      }
    }
    warp_tree<K>(s, e);
    float S = s[0], E = e[0];
    partials_tree<WARPS, LPW>(S, E);
    total = __shfl(S + E, 0, 64);
    __syncthreads(); // the image is free again for the caller
  }
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && lane == 0) {
    a.stats[2 * row] = variance;
    a.stats[2 * row + 1] = inv;
  }
  // Error flag as in norm_compute.
  bool fine = !RES || isfinite(total);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint32_t vv[4] = {vw[c].x, vw[c].y, vw[c].z, vw[c].w};
    const uint32_t gg[4] = {gin[c].x, gin[c].y, gin[c].z, gin[c].w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float y0 = B(lo16(vv[k]) * inv) * lo16(gg[k]);
      const float y1 = B(hi16(vv[k]) * inv) * hi16(gg[k]);
      if constexpr (CHECK_Y)
        fine = fine && bf16_finite_after_round(y0) && bf16_finite_after_round(y1);
      o[k] = pack2(y0, y1);
    }
    if (512 * c + 8 * lane < H)
      st_nt(reinterpret_cast<uint4 *>(a.y + base + 512 * c + 8 * lane), make_uint4(o[0], o[1], o[2], o[3]));
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
}

// One row per wave: all loads of the row, then compute and stores.  WIDE (BF16 rows): the
// 16-byte layout of norm_row_wave_wide, with `lds` (VT * J / 8 uint4 of LDS owned by the
// caller, for the rare ordered replay); otherwise every access is in the reference's
// thread-ownership layout, and FAST selects the sum (norm_compute).
template <int VT, int J, class T, bool RES, bool WIDE = true, bool GATHER = false,
          bool FAST = true>
__device__ __forceinline__ void norm_row_wave(const NormArgs<T> &a, int row, uint4 *lds) {
  if (row >= a.rows)
    return; // wave-uniform
  if constexpr (WIDE && std::is_same<T, uint16_t>::value) {
    norm_row_wave_wide<VT, J, RES>(a, row, lds);
    return;
  }
  RowIn<VT, J, T> in;
  Lanes<uint16_t, VT / 64> gr[J];
  if constexpr (GATHER) {
    static_assert(RES && std::is_same<T, uint16_t>::value, "gather: BF16 residual rows");
    norm_load_gather<VT, J>(a, row, in);
  } else {
    norm_load<VT, J, T, RES>(a, row, in);
  }
  norm_load_gamma<VT, J>(a.gamma, gr);
  norm_compute<VT, J, T, RES, FAST>(a, row, in, gr);
}

} // namespace padra
