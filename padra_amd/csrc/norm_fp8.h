// RMSNorm with the FP8 E4M3 row encoding fused in: NormFP8Exact (norm_fp8_exact.cuh:6-62)
// and NormFP8WideExact (norm_fp8_wide_exact.cuh:7-67).  Both reference kernels sum the
// squares with the 128-thread ownership and tree (the wide one keeps the first 128 threads'
// products, rms_wide_exact.cuh:3-30), so one wave per row replays the 128-thread tree of
// norm_rows.h.  Then, per row:
//   y_i      = B(B(x_i * inv) * gamma_i)          (normalized, BF16-exact; flag if not finite)
//   scale    = max|y| == 0 ? 1 : max|y| / 448     (fmaxf drops NaN, as MaxReduce does)
//   packed_i = E4M3 code of the correctly rounded y_i / scale, which is what the
//              reference's reciprocal-with-midpoint-division computes
//              (fp8_exact_reciprocal.cuh:5-21); see fp8_encode_pairs for how
//              it is computed here
// The maximum is order-independent, so the wave reduces it with any exchange pattern.
#pragma once
#include <type_traits>

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
  const uint32_t normal = min(((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - (120u << 3), 0x7eu);
  // Branch-free selects (the compiler would otherwise branch per element).
  const uint32_t small = 0u - (uint32_t)(mag < 0x3c800000u); // a < 2^-6
  const uint32_t big = 0u - (uint32_t)(mag >= 0x43e00000u);  // a >= 448 (infinities too)
  const uint32_t nan = 0u - (uint32_t)(mag > 0x7f800000u);
  uint32_t code = (sub & small) | (normal & ~small);
  code = (0x7eu & big) | (code & ~big);
  return (0x7fu & nan) | ((sign | code) & ~nan);
}

// E4M3 code of a finite quotient q with |q| <= 480 through gfx950's v_cvt_pk_fp8_f32 (OCP
// E4M3, round to nearest even), after clamping to +-448; equal to e4m3_code there
// (padra_CheckFP8Paths compares the two on every such float).
__device__ __forceinline__ uint32_t e4m3_pair_hw(float q0, float q1) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(q0, -448.f, 448.f),
                                                   __builtin_amdgcn_fmed3f(q1, -448.f, 448.f), 0,
                                                   false) & 0xffffu;
}

// The same conversion without the clamp, for the row fast path: there |q| is within one
// ulp of |y| / scale <= amax / RN(amax / 448) < 448.001, which the conversion rounds to
// at most 448 (the overflow threshold is 464).  padra_CheckFP8Paths compares it with
// e4m3_code on every float up to 460 and, through fp8_quotient, on every BF16 (maximum,
// value) pair of the fast path.
__device__ __forceinline__ uint32_t e4m3_pair_fast(float q0, float q1) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false) & 0xffffu;
}

// The quotient v / scale from the cached reciprocal plus one exact-remainder correction:
// q = v * inverse, r = q * scale - v (one fused multiply-add), q - r * inverse.  Written
// with r of that sign, a zero v keeps its sign through both steps (-0: q = -0, r = +0,
// -0 * inverse + -0 = -0), and the negations are free operand modifiers.  For BF16 v and
// a scale derived from a BF16 maximum of at least 2^-100 (inverse normal), its E4M3 code
// equals the code of the correctly rounded quotient for every such pair, as
// padra_CheckFP8Paths verifies.
__device__ __forceinline__ float fp8_quotient(float v, float scale, float inverse) {
  const float q = v * inverse;
  const float r = __builtin_fmaf(q, scale, -v);
  return __builtin_fmaf(-r, inverse, q);
}

// Whether a row may take the fast path: finite values, maximum >= 2^-100, normal inverse.
__device__ __forceinline__ bool fp8_fast_ok(float amax, float inverse) {
  const uint32_t ie = __float_as_uint(inverse) & 0x7f800000u;
  return amax >= 0x1p-100f && ie != 0 && ie != 0x7f800000u;
}

// The codes of J pairs of values (BF16 pairs in words w) with one scale: the reference's
// fp8_exact_reciprocal::Encode, whose code is the code of the correctly rounded quotient
// (its midpoint test only chooses when to divide; the CPU tests check this on values aimed
// at every E4M3 midpoint).  FAST: fp8_quotient and the hardware conversion; otherwise a
// correctly rounded division and e4m3_code (rows with a NaN or an infinity, tiny maxima).
template <int J, bool FAST>
__device__ __forceinline__ void fp8_encode_pairs(const uint32_t (&w)[J], float scale,
                                                 float inverse, uint32_t (&codes)[J]) {
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if constexpr (FAST)
      codes[j] = e4m3_pair_fast(fp8_quotient(lo16(w[j]), scale, inverse),
                                fp8_quotient(hi16(w[j]), scale, inverse));
    else
      codes[j] = e4m3_code(lo16(w[j]) / scale) | (e4m3_code(hi16(w[j]) / scale) << 8);
  }
}

// Everything after the row's values are in registers: lane l holds v_{2l+k+128j} (k = 0, 1)
// in vp[j] (BF16 pair) and the matching gamma pairs.  The 128-thread tree, the normalized
// row, and with FP8 the scale and codes.
template <int J, class T, bool FP8, bool WT = false>
__device__ __forceinline__ void norm_fp8_finish(const NormFP8Args<T> &a, int row,
                                                const uint32_t (&vp)[J],
                                                const Lanes<uint16_t, 2> (&gr)[J]) {
  constexpr int VT = 128, K = 2, H = VT * J;
  const int lane = threadIdx.x & 63;
  const size_t off = (size_t)row * H + K * lane;
  // The order-free sum (sumsq_margin, common.h), or (rarely; wave-uniform) the tree.
  double acc[4] = {0.0, 0.0, 0.0, 0.0}; // independent fp64 chains
#pragma unroll
  for (int j = 0; j < J; ++j) {
    acc[2 * (j & 1)] = sq64(lo16(vp[j]), acc[2 * (j & 1)]);
    acc[2 * (j & 1) + 1] = sq64(hi16(vp[j]), acc[2 * (j & 1) + 1]);
  }
  const double lane_sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
  for (int j = 0; j < J; ++j)
    pin(gr[j].w[0]); // the gamma loads stay ahead of the rarely taken branch below
  float total;
  if (!certified_sum(wave_sum64(lane_sum), sumsq_margin(J, 2 * J + 6), total)) {
    float s[K] = {0.f, 0.f}, e[K] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float v0 = lo16(vp[j]), v1 = hi16(vp[j]);
      acc_pos(v0 * v0, s[0], e[0]);
      acc_pos(v1 * v1, s[1], e[1]);
    }
    warp_tree<K>(s, e);
    float S = s[0], E = e[0];
    partials_tree<VT / 32, 32 / K>(S, E);
    total = lane0(S + E);
  }
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && row == 0 && lane == 0) {
    a.stats[0] = variance;
    a.stats[1] = inv;
  }

  // y, the normalized row, and the largest |y| as BF16 magnitude bits: two 16-bit lanes of
  // an unsigned max per word (the integer order of magnitude bits is the order of |y|, with
  // infinities above every finite value and NaNs above infinities).
  typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
  uint32_t yw[J];
  u16x2_t mag2 = {0, 0};
#pragma unroll
  for (int j = 0; j < J; ++j) {
    yw[j] = pack2(B(lo16(vp[j]) * inv) * gr[j].get(0), B(hi16(vp[j]) * inv) * gr[j].get(1));
    mag2 = __builtin_elementwise_max(mag2, __builtin_bit_cast(u16x2_t, yw[j] & 0x7fff7fffu));
    Lanes<T, K>::template store<WT>(a.y + off + VT * j, &yw[j]);
  }
  uint32_t mag = max((uint32_t)mag2.x, (uint32_t)mag2.y);
  mag = xor_reduce<32>(mag, [](uint32_t x, uint32_t y) { return max(x, y); });
  // Every y finite <=> the largest magnitude is below the BF16 infinity (wave-uniform).
  const bool row_fine = mag < 0x7f80u;
  if (!row_fine && lane == 0)
    raise_bad(a.bad);
  if constexpr (FP8) {
    if (!row_fine) {
      // MaxReduce's fmaxf drops NaN operands: the maximum over the non-NaN magnitudes.
      mag = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t lo = yw[j] & 0x7fffu, hi = (yw[j] >> 16) & 0x7fffu;
        mag = max(mag, lo > 0x7f80u ? 0u : lo);
        mag = max(mag, hi > 0x7f80u ? 0u : hi);
      }
      mag = xor_reduce<32>(mag, [](uint32_t x, uint32_t y) { return max(x, y); });
    }
    const float amax = __uint_as_float(mag << 16);
    const float scale = amax == 0.f ? 1.f : amax / 448.f;
    const float inverse = 1.f / scale;
    if (lane == 0)
      a.scales[row] = scale;

    // Codes: two per j, one 2-byte store each (128 contiguous bytes per instruction).
    uint32_t codes[J];
    if (row_fine && fp8_fast_ok(amax, inverse)) // wave-uniform
      fp8_encode_pairs<J, true>(yw, scale, inverse, codes);
    else
      fp8_encode_pairs<J, false>(yw, scale, inverse, codes);
    uint8_t *const out = a.packed + off;
#pragma unroll
    for (int j = 0; j < J; ++j)
      *reinterpret_cast<uint16_t *>(out + VT * j) = (uint16_t)codes[j];
  }
}

// BF16 rows with 16-byte accesses, as norm_row_wave_wide: piece c of lane L is elements
// 512 c + 8 L .. + 7 of x, gamma, normalized (16 bytes) and packed (8 bytes), all stores
// non-temporal (2048 x 2048, inputs cold: 5.29 us, against 6.57 us for the 4-byte
// thread-ownership layout and 5.93 us with written-through stores).  The
// order-free sum needs no thread ownership; its rare fallback sends the row across `vlds`
// (VT * J / 8 uint4) into the reference's 128-thread ownership and tree.  The maximum is
// order-free; pieces past H (H not a multiple of 512) are clamped to elements 0..7, which
// the maximum may see twice and nothing stores.
template <int J>
__device__ __forceinline__ void norm_fp8_row_wide(const NormFP8Args<uint16_t> &a, int row,
                                                  uint4 *vlds) {
  constexpr int VT = 128, K = 2, H = VT * J, C = (H + 511) / 512;
  if (row >= a.rows)
    return; // wave-uniform
  const int lane = threadIdx.x & 63;
  const size_t base = (size_t)row * H;
  uint4 xin[C], gin[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = (512 * c + 8 * lane < H) ? 512 * c + 8 * lane : 0; // clamped, unconditional
    gin[c] = *reinterpret_cast<const uint4 *>(a.gamma + e);
  }
  issue_point();
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = (512 * c + 8 * lane < H) ? 512 * c + 8 * lane : 0;
    xin[c] = ld_nt(reinterpret_cast<const uint4 *>(a.x + base + e));
  }
#pragma unroll
  for (int c = 0; c < C; ++c)
    pin(gin[c]); // the gamma loads stay ahead of the rarely taken branch below
  double acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    acc[k] = 0.0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if (512 * c + 8 * lane < H) {
      const uint32_t vv[4] = {xin[c].x, xin[c].y, xin[c].z, xin[c].w};
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
    // Rare (wave-uniform): thread 2 l + k owns elements 2 l + k + 128 j, word l + 64 j of
    // the packed row.
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (512 * c + 8 * lane < H)
        vlds[64 * c + lane] = xin[c];
    __syncthreads();
    const uint32_t *vwords = reinterpret_cast<const uint32_t *>(vlds);
    float s[K] = {0.f, 0.f}, e[K] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t word = vwords[lane + (VT / 2) * j];
      const float v0 = lo16(word), v1 = hi16(word);
      acc_pos(v0 * v0, s[0], e[0]);
      acc_pos(v1 * v1, s[1], e[1]);
    }
    warp_tree<K>(s, e);
    float S = s[0], E = e[0];
    partials_tree<VT / 32, 32 / K>(S, E);
    total = __shfl(S + E, 0, 64);
    __syncthreads(); // the image is free again
  }
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && row == 0 && lane == 0) {
    a.stats[0] = variance;
    a.stats[1] = inv;
  }
  // y and the largest |y| as BF16 magnitude bits (see norm_fp8_finish)
  typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
  uint32_t yw[C][4];
  u16x2_t mag2 = {0, 0};
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint32_t vv[4] = {xin[c].x, xin[c].y, xin[c].z, xin[c].w};
    const uint32_t gg[4] = {gin[c].x, gin[c].y, gin[c].z, gin[c].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      yw[c][k] = pack2(B(lo16(vv[k]) * inv) * lo16(gg[k]), B(hi16(vv[k]) * inv) * hi16(gg[k]));
      mag2 = __builtin_elementwise_max(mag2, __builtin_bit_cast(u16x2_t, yw[c][k] & 0x7fff7fffu));
    }
    if (512 * c + 8 * lane < H)
      st_nt(reinterpret_cast<uint4 *>(a.y + base + 512 * c + 8 * lane),
                             make_uint4(yw[c][0], yw[c][1], yw[c][2], yw[c][3]));
  }
  uint32_t mag = max((uint32_t)mag2.x, (uint32_t)mag2.y);
  mag = xor_reduce<32>(mag, [](uint32_t x, uint32_t y) { return max(x, y); });
  const bool row_fine = mag < 0x7f80u; // wave-uniform
  if (!row_fine) {
    if (lane == 0)
      raise_bad(a.bad);
    mag = 0; // MaxReduce's fmaxf drops NaN operands
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = yw[c][k] & 0x7fffu, hi = (yw[c][k] >> 16) & 0x7fffu;
        mag = max(mag, lo > 0x7f80u ? 0u : lo);
        mag = max(mag, hi > 0x7f80u ? 0u : hi);
      }
    mag = xor_reduce<32>(mag, [](uint32_t x, uint32_t y) { return max(x, y); });
  }
  const float amax = __uint_as_float(mag << 16);
  const float scale = amax == 0.f ? 1.f : amax / 448.f;
  const float inverse = 1.f / scale;
  if (lane == 0)
    a.scales[row] = scale;
  const bool fast = row_fine && fp8_fast_ok(amax, inverse); // wave-uniform
#pragma unroll
  for (int c = 0; c < C; ++c) {
    uint32_t codes[4];
    if (fast)
      fp8_encode_pairs<4, true>(yw[c], scale, inverse, codes);
    else
      fp8_encode_pairs<4, false>(yw[c], scale, inverse, codes);
    if (512 * c + 8 * lane < H)
      st_nt(reinterpret_cast<uint2 *>(a.packed + base + 512 * c + 8 * lane),
                             make_uint2(codes[0] | (codes[1] << 16), codes[2] | (codes[3] << 16)));
  }
}

template <int J, class T>
__device__ __forceinline__ void norm_fp8_row_wave(const NormFP8Args<T> &a, int row) {
  constexpr int VT = 128, K = 2, H = VT * J;
  if (row >= a.rows)
    return; // wave-uniform
  const size_t off = (size_t)row * H + K * (threadIdx.x & 63);
  Lanes<T, K> x[J];
  Lanes<uint16_t, K> gr[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    x[j].load(a.x + off + VT * j);
  norm_load_gamma<VT, J>(a.gamma, gr);
  // Thread 2l+k owns elements 2l + k + 128 j, summed in j order.
  uint32_t vp[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if constexpr (std::is_same<T, uint16_t>::value)
      vp[j] = x[j].w[0]; // BF16 input: the pair is the loaded word
    else
      vp[j] = pack2(x[j].get(0), x[j].get(1));
  }
  norm_fp8_finish<J, T, true, true>(a, row, vp, gr); // written-through: 6.34 -> 6.25 us
}

} // namespace padra
