// Residual-add + RMSNorm of one row by a 256-lane workgroup, one lane per reference thread,
// for launches with few rows (a decode step).  The reference block has VT threads
// (residual_norm_wide_exact.cuh:6-80 for VT = 256, Norm inference.cu:188-214 for 128):
// thread t sums the squares of elements t, t + VT, ... in that order, its warp folds the
// partials with a shuffle-down tree, and the VT / 32 warp partials fold in the
// shuffle-down order of inference.cu:120-135.  Here lane l of wave w is thread 64w + l;
// the warp trees are the lane exchanges of qk_head.h, and the warp partials cross LDS.
// One wave per row (norm_rows.h) holds 32 elements per lane; with a few dozen rows each
// such wave runs alone on its SIMD and its ~700 dependent instructions set the launch's
// time.  Here a lane holds VT... H / VT elements (8 at H = 2048).
#pragma once
#include "qk_head.h"

namespace padra {

// Row `row` by the calling workgroup (blockDim.x == 256).  Lanes t >= VT take part in the
// barriers only.  The sum of squares is the order-free fp64 sum when its fp32 rounding is
// certain to equal the reference's (sumsq_margin, common.h); otherwise the reference's
// tree runs as described above.  GATHER: x is the embedding row of the row's token
// (norm_load_gather's rule: an invalid token raises the flag and reads x as it is).
template <int VT, int J, bool GATHER>
__device__ __forceinline__ void norm_row_wg(const NormArgs<uint16_t> &a, int row,
                                            float (*partials)[2]) {
  static_assert(VT == 128 || VT == 256, "reference trees of 128 or 256 threads");
  constexpr int H = VT * J, WARPS = VT / 32;
  constexpr bool CHECK_Y = VT == 256;
  const int t = threadIdx.x;
  const bool act = t < VT; // wave-uniform
  const size_t off = (size_t)row * H + (act ? t : 0);
  float v[J];
  double acc = 0.0;
  // The norm weights first: independent of the row, they are in flight during the sums.
  uint16_t gw[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    gw[j] = a.gamma[(act ? t : 0) + VT * j];
  if (act) {
    uint16_t rr[J], xx[J];
#pragma unroll
    for (int j = 0; j < J; ++j)
      rr[j] = a.residual[off + VT * j];
    const uint16_t *src = a.x + off;
    if constexpr (GATHER) {
      bool ok;
      const int token = embed_token(a.src, a.ids, row, a.vocab, ok);
      if (!ok && t == 0)
        raise_bad(a.bad);
      if (ok)
        src = a.gather + (size_t)token * H + t;
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
      xx[j] = src[VT * j];
    uint16_t vb[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      v[j] = B(__uint_as_float((uint32_t)xx[j] << 16) + __uint_as_float((uint32_t)rr[j] << 16));
      vb[j] = (uint16_t)(__float_as_uint(v[j]) >> 16);
      acc = sq64(v[j], acc);
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
      a.x[off + VT * j] = vb[j];
  }
#pragma unroll
  for (int j = 0; j < J; ++j)
    pin((uint32_t)gw[j]); // the weight loads stay ahead of the rarely taken branch below
  // The order-free sum (sumsq_margin): per wave, then the four wave totals through LDS.
  double *wave_totals = reinterpret_cast<double *>(partials);
  {
    const double w = wave_sum64(acc);
    if ((t & 63) == 0)
      wave_totals[t >> 6] = w;
  }
  __syncthreads();
  const double s64 = (wave_totals[0] + wave_totals[1]) + (wave_totals[2] + wave_totals[3]);
  float total;
  if (!certified_sum(s64, sumsq_margin(J, J + 8), total)) {
    // Rare (workgroup-uniform: every wave read the same totals): the reference's tree.
    __syncthreads(); // the totals are read before the partials overwrite them
    if (act) {
      float s = 0.f, e = 0.f;
#pragma unroll
      for (int j = 0; j < J; ++j)
        acc_pos(v[j] * v[j], s, e);
      warp_tree_lanes(s, e);
      if ((t & 31) == 0) {
        partials[t >> 5][0] = s;
        partials[t >> 5][1] = e;
      }
    }
    __syncthreads();
    // The warp partials' tree: partial w folds partial w + D for D = WARPS/2, ..., 1.
    float ps[WARPS], pe[WARPS];
#pragma unroll
    for (int w = 0; w < WARPS; ++w) {
      ps[w] = partials[w][0];
      pe[w] = partials[w][1];
    }
#pragma unroll
    for (int d = WARPS / 2; d >= 1; d /= 2)
#pragma unroll
      for (int w = 0; w < d; ++w)
        fold(ps[w + d], pe[w + d], ps[w], pe[w]);
    total = ps[0] + pe[0];
  }
  if (!act)
    return;
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && t == 0) {
    a.stats[2 * row] = variance;
    a.stats[2 * row + 1] = inv;
  }
  bool fine = isfinite(total);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float g = __uint_as_float((uint32_t)gw[j] << 16);
    const float y = B(v[j] * inv) * g;
    if constexpr (CHECK_Y)
      fine = fine && bf16_finite_after_round(y);
    a.y[off + VT * j] = (uint16_t)(pack2(0.f, y) >> 16);
  }
  if (__ballot(!fine) != 0 && (t & 63) == 0)
    raise_bad(a.bad);
}

} // namespace padra
