// Residual-add + RMSNorm over hidden rows, one 64-lane wavefront per VT/8-lane row group.
//
// Reference: Add + Norm (inference.cu:475-481, 188-214) for VT = 128 and
// ResidualPostNormWideExact (residual_norm_wide_exact.cuh:6-80) for VT = 256.  The
// reference block has VT threads; thread t owns elements t, t+VT, t+2VT, ... and sums
// their squares in that order, then a 32-lane shuffle-down tree per warp and one more
// tree over the warp partials.  Here each lane owns EIGHT consecutive "threads"
// (8*lr .. 8*lr+7), so every 16-byte load lands exactly the elements those threads own
// for one j, and the same tree is replayed: tree levels 16 and 8 cross lanes (shuffle
// down by 2 and 1 lanes), levels 4, 2, 1 stay inside the lane, and the warp partials
// sit in lanes 0, 4, 8, ... of the row group.  Levels of the final tree that only add
// zero lanes are exact no-ops and are skipped.  The result is bit-identical to the
// reference's fadd(sum, error).
#pragma once
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
};

// Largest |y| whose BF16 rounding stays finite: 0x7f7f8000 is the midpoint between the
// largest finite BF16 (0x7f7f, odd) and infinity, and it rounds to infinity.
__device__ __forceinline__ bool bf16_finite_after_round(float y) {
  return fabsf(y) < __uint_as_float(0x7f7f8000u);
}

template <int VT, int J, class T, bool RES>
__device__ __forceinline__ void norm_rows_wave(const NormArgs<T> &a, int wave) {
  constexpr int LPR = VT / 8, RPW = 64 / LPR, H = VT * J, WARPS = VT / 32;
  const int lane = threadIdx.x & 63, lr = lane % LPR, rsub = lane / LPR;
  const int row = wave * RPW + rsub;
  const bool live = row < a.rows;
  const size_t off = (size_t)(live ? row : 0) * H;

  uint32_t vp[J][4];
  float s[8], e[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    s[k] = 0.f;
    e[k] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int col = VT * j + 8 * lr;
    float xv[8];
    ActIO<T>::load8(a.x + off + col, xv);
    if constexpr (RES) {
      float rv[8];
      ActIO<T>::load8(a.residual + off + col, rv);
#pragma unroll
      for (int w = 0; w < 4; ++w)
        vp[j][w] = pack2(xv[2 * w] + rv[2 * w], xv[2 * w + 1] + rv[2 * w + 1]);
      if (live)
        ActIO<T>::store8(a.x + off + col, vp[j]);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        vp[j][w] = pack2(xv[2 * w], xv[2 * w + 1]);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float v0 = lo16(vp[j][w]), v1 = hi16(vp[j][w]);
      acc_pos(v0 * v0, s[2 * w], e[2 * w]);
      acc_pos(v1 * v1, s[2 * w + 1], e[2 * w + 1]);
    }
  }
  // Warp tree level 16: threads 8*lr+k with (lr%4) < 2 fold threads 16 further on,
  // i.e. the same slot two lanes down; level 8: one lane down.
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float s2 = shfl_down(s[k], 2), e2 = shfl_down(e[k], 2);
    fold(s2, e2, s[k], e[k]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float s2 = shfl_down(s[k], 1), e2 = shfl_down(e[k], 1);
    fold(s2, e2, s[k], e[k]);
  }
  // Levels 4, 2, 1 inside the lane.
#pragma unroll
  for (int k = 0; k < 4; ++k)
    fold(s[k + 4], e[k + 4], s[k], e[k]);
#pragma unroll
  for (int k = 0; k < 2; ++k)
    fold(s[k + 2], e[k + 2], s[k], e[k]);
  fold(s[1], e[1], s[0], e[0]);
  // Final tree over the WARPS partials held by lanes 0, 4, 8, ... of the row group.
#pragma unroll
  for (int d = WARPS / 2; d >= 1; d /= 2) {
    const float s2 = shfl_down(s[0], 4 * d), e2 = shfl_down(e[0], 4 * d);
    fold(s2, e2, s[0], e[0]);
  }
  const float total = __shfl(s[0] + e[0], rsub * LPR, 64);
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  bool fine = isfinite(total);
  if (a.stats && live && lr == 0) {
    a.stats[2 * row] = variance;
    a.stats[2 * row + 1] = inv;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int col = VT * j + 8 * lr;
    float g[8];
    load8_bf16(a.gamma + col, g);
    uint32_t out[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float y0 = B(lo16(vp[j][w]) * inv) * g[2 * w];
      const float y1 = B(hi16(vp[j][w]) * inv) * g[2 * w + 1];
      fine = fine && bf16_finite_after_round(y0) && bf16_finite_after_round(y1);
      out[w] = pack2(y0, y1);
    }
    if (live)
      ActIO<T>::store8(a.y + off + col, out);
  }
  if (__ballot(live && !fine) != 0 && lane == 0)
    raise_bad(a.bad);
}

} // namespace padra
