// RMSNorm with the FP8 E4M3 row encoding fused in: NormFP8Exact (norm_fp8_exact.cuh:6-62)
// and NormFP8WideExact (norm_fp8_wide_exact.cuh:7-67).  Both reference kernels sum the
// squares with the 128-thread ownership and tree (the wide one keeps the first 128 threads'
// products, rms_wide_exact.cuh:3-30), so one wave per row replays the 128-thread tree of
// norm_rows.h.  Then, per row:
//   y_i      = B(B(x_i * inv) * gamma_i)          (normalized, BF16-exact; flag if not finite)
//   scale    = max|y| == 0 ? 1 : max|y| / 448     (fmaxf drops NaN, as MaxReduce does)
//   packed_i = E4M3 code of y_i / scale, through the cached reciprocal with a correctly
//              rounded division near rounding midpoints (fp8_exact_reciprocal.cuh:5-21)
// The maximum is order-independent, so the wave reduces it with any exchange pattern.
#pragma once
#include "norm_rows.h"

namespace padra {

template <class T> struct NormFP8Args {
  const T *x;
  T *y;
  const uint16_t *gamma;
  uint8_t *packed;
  float *scales;
  float *stats; // {variance, inv} of row 0, as the reference writes them
  int *bad;
  int rows;
  float eps;
};

// OCP E4M3 code of x (bias 7, max 448, no infinities, NaN S.1111.111): round to nearest
// even; finite overflow and infinities saturate to +-448; every NaN gives 0x7f (NaN
// signs and payloads differ between platforms, the code does not).
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  const uint32_t bits = __float_as_uint(x), sign = (bits >> 24) & 0x80u, mag = bits & 0x7fffffffu;
  const float a = __uint_as_float(mag);
  const uint32_t sub = (uint32_t)rintf(a * 512.f); // k * 2^-9, k = 8 is the least normal
  const uint32_t normal = ((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - (120u << 3);
  uint32_t code = a < 0.015625f ? sub : min(normal, 0x7eu);
  code = a >= 448.f ? 0x7eu : code;
  return mag > 0x7f800000u ? 0x7fu : (sign | code);
}

// fp8_exact_reciprocal::NeedsDivision: q's magnitude within 4 ulp of an E4M3 midpoint.
__device__ __forceinline__ bool fp8_needs_division(uint32_t b) {
  if (b < 0x3a800000u)
    return b >= 0x3a800000u - 4u;
  const uint32_t e = b >> 23, shift = e < 121u ? 140u - e : 19u;
  const uint32_t residue = b & ((2u << shift) - 1u), midpoint = 1u << shift;
  return residue - (midpoint - 4u) <= 8u;
}

// fp8_exact_reciprocal::Encode.
__device__ __forceinline__ uint32_t fp8_encode(float value, float scale, float inverse) {
  const uint32_t ie = __float_as_uint(inverse) & 0x7f800000u;
  float q = value * inverse;
  if (ie == 0 || ie == 0x7f800000u || fp8_needs_division(__float_as_uint(q) & 0x7fffffffu))
    q = value / scale;
  return e4m3_code(q);
}

template <int J, class T>
__device__ __forceinline__ void norm_fp8_row_wave(const NormFP8Args<T> &a, int row) {
  constexpr int VT = 128, K = 2, H = VT * J;
  if (row >= a.rows)
    return; // wave-uniform
  const int lane = threadIdx.x & 63;
  const size_t off = (size_t)row * H + K * lane;
  Lanes<T, K> x[J];
  Lanes<uint16_t, K> gr[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    x[j].load(a.x + off + VT * j);
  norm_load_gamma<VT, J>(a.gamma, gr);

  // Sum of squares: thread 2l+k owns elements 2l + k + 128 j, summed in j order.
  uint32_t vp[J];
  float s[K] = {0.f, 0.f}, e[K] = {0.f, 0.f};
#pragma unroll
  for (int j = 0; j < J; ++j) {
    vp[j] = pack2(x[j].get(0), x[j].get(1));
    const float v0 = lo16(vp[j]), v1 = hi16(vp[j]);
    acc_pos(v0 * v0, s[0], e[0]);
    acc_pos(v1 * v1, s[1], e[1]);
  }
  warp_tree<K>(s, e);
  float S = s[0], E = e[0];
  partials_tree<VT / 32, 32 / K>(S, E);
  const float total = __shfl(S + E, 0, 64);
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && row == 0 && lane == 0) {
    a.stats[0] = variance;
    a.stats[1] = inv;
  }

  // y, its maximum magnitude, the normalized row.
  uint32_t yw[J];
  float amax = 0.f;
  bool fine = true;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t p = pack2(lo16(vp[j]) * inv, hi16(vp[j]) * inv);
    yw[j] = pack2(lo16(p) * gr[j].get(0), hi16(p) * gr[j].get(1));
    const float y0 = lo16(yw[j]), y1 = hi16(yw[j]);
    fine = fine && isfinite(y0) && isfinite(y1);
    amax = fmaxf(amax, fmaxf(fabsf(y0), fabsf(y1)));
    Lanes<T, K>::store(a.y + off + VT * j, &yw[j]);
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
#pragma unroll
  for (int d = 32; d >= 1; d /= 2)
    amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  const float scale = amax == 0.f ? 1.f : amax / 448.f;
  const float inverse = 1.f / scale;
  if (lane == 0)
    a.scales[row] = scale;

  // Codes: two per j, one 2-byte store each (128 contiguous bytes per instruction).
  uint8_t *const out = a.packed + off;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t c0 = fp8_encode(lo16(yw[j]), scale, inverse);
    const uint32_t c1 = fp8_encode(hi16(yw[j]), scale, inverse);
    *reinterpret_cast<uint16_t *>(out + VT * j) = (uint16_t)(c0 | (c1 << 8));
  }
}

} // namespace padra
