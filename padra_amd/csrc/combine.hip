// Expert combine (+ residual) and the fused combine + RMSNorm (+ FP8 E4M3) that follows the
// MoE down projection.
//
// Combine (inference.cu:580-590), exl3_packed_activations::Combine
// (expert_exl3_prefill_packed_activations.cuh:86-102): for row t and column i,
//   c = 0;  for e = 0..7: c = B(c + B(down[t][e][i] * w[t][e]));  x = residual ? B(x + c) : c
// with the experts in their routing order.  combine_norm_exact::CombineNorm
// (combine_norm_exact.cuh:7-72) continues with the 128-thread RMSNorm of the new row and,
// optionally, its E4M3 encoding.
#include <stdio.h>

#include <algorithm>

#include "norm_fp8.h"

using namespace padra;

namespace {

constexpr int kExperts = 8; // the reference's top-8 routing

int launched(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fprintf(stderr, "padra: %s launch failed: %s\n", what, hipGetErrorString(e));
    return PADRA_INTERNAL;
  }
  return PADRA_OK;
}
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The combine of 8 consecutive columns: every load (the row's 8 weights, the 8 expert rows,
// x) is issued before the arithmetic.  Returns the packed BF16 results; `fine` is false
// when one of them is not finite.
template <class T, bool RES>
__device__ __forceinline__ void combine8(const T *x, const T *down, size_t expert_stride,
                                         const float *w, uint32_t (&out)[4], bool &fine) {
  float d[kExperts][8], xv[8];
  float wt[kExperts];
#pragma unroll
  for (int e = 0; e < kExperts; ++e)
    wt[e] = w[e];
#pragma unroll
  for (int e = 0; e < kExperts; ++e)
    ActIO<T>::load8(down + e * expert_stride, d[e]);
  if constexpr (RES)
    ActIO<T>::load8(x, xv);
  float c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    c[k] = 0.f;
  // B() of one value is one conversion whose result is already the float; rounding a pair
  // with one conversion would need two unpacks to continue.
#pragma unroll
  for (int e = 0; e < kExperts; ++e)
#pragma unroll
    for (int k = 0; k < 8; ++k)
      c[k] = B(c[k] + B(d[e][k] * wt[e]));
  uint32_t bad_bits = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    out[k] = RES ? pack2(xv[2 * k] + c[2 * k], xv[2 * k + 1] + c[2 * k + 1])
                 : pack2(c[2 * k], c[2 * k + 1]);
    // a half is not finite iff its exponent bits are all ones
    bad_bits |= ((out[k] & 0x7f80u) == 0x7f80u) | ((out[k] & 0x7f800000u) == 0x7f800000u);
  }
  fine = bad_bits == 0;
}

// Plain combine: one thread per 8 consecutive columns, grid-stride over the rows.
template <class T, bool RES>
__global__ __launch_bounds__(256) void k_combine(T *x, const T *down, const float *weights,
                                                 int hidden, long long groups, int *bad) {
  const int per_row = hidden / 8;
  bool all_fine = true;
  for (long long g = blockIdx.x * 256ll + threadIdx.x; g < groups; g += (long long)gridDim.x * 256) {
    const long long t = g / per_row;
    const int col = (int)(g - t * per_row) * 8;
    T *xr = x + t * hidden + col;
    uint32_t out[4];
    bool fine;
    combine8<T, RES>(xr, down + (t * kExperts) * hidden + col, (size_t)hidden,
                     weights + t * kExperts, out, fine);
    ActIO<T>::store8(xr, out);
    all_fine = all_fine && fine;
  }
  if (!all_fine)
    raise_bad(bad);
}

// Waves per row of the combine + norm kernel.  The row's 36 sixteen-byte loads per lane
// (8 expert rows and x, four 512-column chunks at H = 2048) do not fit one wave's registers
// at once, so one wave per row loaded them in dependent rounds; four waves, one chunk
// each, put them all in flight: 2048 x 2048 with FP8, 21.1 -> 19.3 us.  With the ordered
// tree, finishing the norm in every wave (each storing a quarter of the row after the same
// reductions) measured slower (22.6 us), so for fp32 rows wave 0 finishes the row alone;
// BF16 rows take k_combine_norm_wide, whose order-free sum makes every wave's finish cheap.
constexpr int kCombineWaves = 4;

// Combine + RMSNorm (+ FP8): W waves per row.  The combine runs in the natural layout
// (lane l takes columns 8l..8l+7 of each 512-column chunk, 16-byte accesses; wave w takes
// chunks w, w + W, ...), its BF16 results go through LDS, and wave 0 reads them back in
// the 128-thread ownership layout (lane l: columns 2l, 2l+1 of each 128) for the norm.
template <int J, class T, bool FP8, int W>
__global__ __launch_bounds__(64 * W) void k_combine_norm(T *x, const T *down, const float *weights,
                                                         NormFP8Args<T> a) {
  constexpr int H = 128 * J, CHUNKS = (H + 511) / 512;
  __shared__ uint32_t v_lds[H / 2];
  const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (row >= a.rows)
    return; // block-uniform
  Lanes<uint16_t, 2> gr[J];
  if (wave == 0)
    norm_load_gamma<128, J>(a.gamma, gr);
  bool fine = true;
#pragma unroll
  for (int i = 0; i < (CHUNKS + W - 1) / W; ++i) {
    const int ch = wave + W * i, col = ch * 512 + 8 * lane;
    if (ch < CHUNKS && col < H) {
      T *xr = x + (size_t)row * H + col;
      uint32_t out[4];
      bool f;
      combine8<T, true>(xr, down + (size_t)row * kExperts * H + col, (size_t)H,
                        weights + (size_t)row * kExperts, out, f);
      ActIO<T>::template store8<true>(xr, out);
      fine = fine && f;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v_lds[col / 2 + k] = out[k];
    }
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
  __syncthreads();
  if (wave != 0)
    return;
  uint32_t vp[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    vp[j] = v_lds[64 * j + lane];
  norm_fp8_finish<J, T, FP8, true>(a, row, vp, gr);
}

// BF16 rows: the same combine, with the norm and the encoding spread over the W waves too.
// Each wave keeps its chunks' combined words in registers and adds their squares into an
// order-free fp64 partial (sumsq_margin, common.h); the W partials meet in LDS, summed in
// wave order by every wave, so the certification (and its rare fallback: the row crosses
// LDS and wave 0 runs the reference's 128-thread ownership and tree) is block-uniform.
// Every wave then normalizes and stores its own chunks (16-byte pieces of normalized, 8
// bytes of codes), with the row maximum met the same way.  2048 x 2048, inputs cold, this
// form and wave 0 finishing the row in the ownership layout (k_combine_norm) both measure
// 19.36 us with FP8 and 17.13 us without; the combine alone (padra_Combine) 14.8 us.
template <int J, bool FP8, int W>
__global__ __launch_bounds__(64 * W) void k_combine_norm_wide(uint16_t *x, const uint16_t *down,
                                                              const float *weights,
                                                              NormFP8Args<uint16_t> a) {
  constexpr int VT = 128, K = 2, H = VT * J, CHUNKS = (H + 511) / 512, CW = (CHUNKS + W - 1) / W;
  __shared__ uint4 v_lds[H / 8]; // the row, for the rare ordered replay
  __shared__ double part[W];
  __shared__ uint32_t mags[2][W];
  __shared__ float tree_total;
  const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (row >= a.rows)
    return; // block-uniform
  const size_t base = (size_t)row * H;
  auto valid = [&](int i) {
    const int ch = wave + W * i;
    return ch < CHUNKS && ch * 512 + 8 * lane < H;
  };
  auto column = [&](int i) { return (wave + W * i) * 512 + 8 * lane; };
  uint4 gin[CW];
#pragma unroll
  for (int i = 0; i < CW; ++i)
    gin[i] = *reinterpret_cast<const uint4 *>(a.gamma + (valid(i) ? column(i) : 0));
  uint32_t v[CW][4];
  bool fine = true;
#pragma unroll
  for (int i = 0; i < CW; ++i) {
    v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0;
    if (valid(i)) {
      uint16_t *xr = x + base + column(i);
      bool f;
      combine8<uint16_t, true>(xr, down + (size_t)row * kExperts * H + column(i), (size_t)H,
                               weights + (size_t)row * kExperts, v[i], f);
      ActIO<uint16_t>::store8(xr, v[i]);
      fine = fine && f;
    }
  }
  if (__ballot(!fine) != 0 && lane == 0)
    raise_bad(a.bad);
#pragma unroll
  for (int i = 0; i < CW; ++i)
    pin(gin[i]);
  double acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    acc[k] = 0.0;
#pragma unroll
  for (int i = 0; i < CW; ++i)
    if (valid(i)) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[2 * k] = sq64(lo16(v[i][k]), acc[2 * k]);
        acc[2 * k + 1] = sq64(hi16(v[i][k]), acc[2 * k + 1]);
      }
    }
  const double wsum =
      wave_sum64(((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])));
  if (lane == 0)
    part[wave] = wsum;
  __syncthreads();
  double s64 = part[0];
#pragma unroll
  for (int w = 1; w < W; ++w)
    s64 += part[w];
  float total;
  if (!certified_sum(s64, sumsq_margin(J, CW + 3 + 6 + W - 1), total)) { // block-uniform
#pragma unroll
    for (int i = 0; i < CW; ++i)
      if (valid(i))
        v_lds[column(i) / 8] = make_uint4(v[i][0], v[i][1], v[i][2], v[i][3]);
    __syncthreads();
    if (wave == 0) {
      // thread 2 l + k owns elements 2 l + k + 128 j: word l + 64 j of the packed row
      const uint32_t *vwords = reinterpret_cast<const uint32_t *>(v_lds);
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
      if (lane == 0)
        tree_total = S + E;
    }
    __syncthreads();
    total = tree_total;
  }
  const float variance = total / (float)H;
  const float inv = 1.f / sqrtf(variance + a.eps);
  if (a.stats && row == 0 && threadIdx.x == 0) {
    a.stats[0] = variance;
    a.stats[1] = inv;
  }
  typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
  uint32_t yw[CW][4];
  u16x2_t mag2 = {0, 0};
#pragma unroll
  for (int i = 0; i < CW; ++i) {
    const uint32_t gg[4] = {gin[i].x, gin[i].y, gin[i].z, gin[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      yw[i][k] = pack2(B(lo16(v[i][k]) * inv) * lo16(gg[k]), B(hi16(v[i][k]) * inv) * hi16(gg[k]));
      if (valid(i))
        mag2 = __builtin_elementwise_max(mag2, __builtin_bit_cast(u16x2_t, yw[i][k] & 0x7fff7fffu));
    }
    if (valid(i))
      st_nt(reinterpret_cast<uint4 *>(a.y + base + column(i)),
            make_uint4(yw[i][0], yw[i][1], yw[i][2], yw[i][3]));
  }
  // the row's largest |y| as BF16 magnitude bits (see norm_fp8_finish)
  uint32_t mag = max((uint32_t)mag2.x, (uint32_t)mag2.y);
  mag = xor_reduce<32>(mag, [](uint32_t p, uint32_t q) { return max(p, q); });
  if (lane == 0)
    mags[0][wave] = mag;
  __syncthreads();
  mag = mags[0][0];
#pragma unroll
  for (int w = 1; w < W; ++w)
    mag = max(mag, mags[0][w]);
  const bool row_fine = mag < 0x7f80u; // block-uniform
  if (!row_fine && threadIdx.x == 0)
    raise_bad(a.bad);
  if constexpr (FP8) {
    if (!row_fine) {
      // MaxReduce's fmaxf drops NaN operands: the maximum over the non-NaN magnitudes
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < CW; ++i)
        if (valid(i))
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t lo = yw[i][k] & 0x7fffu, hi = (yw[i][k] >> 16) & 0x7fffu;
            m = max(m, lo > 0x7f80u ? 0u : lo);
            m = max(m, hi > 0x7f80u ? 0u : hi);
          }
      m = xor_reduce<32>(m, [](uint32_t p, uint32_t q) { return max(p, q); });
      if (lane == 0)
        mags[1][wave] = m;
      __syncthreads();
      mag = mags[1][0];
#pragma unroll
      for (int w = 1; w < W; ++w)
        mag = max(mag, mags[1][w]);
    }
    const float amax = __uint_as_float(mag << 16);
    const float scale = amax == 0.f ? 1.f : amax / 448.f;
    const float inverse = 1.f / scale;
    if (threadIdx.x == 0)
      a.scales[row] = scale;
    const bool fast = row_fine && fp8_fast_ok(amax, inverse); // block-uniform
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      uint32_t codes[4];
      if (fast)
        fp8_encode_pairs<4, true>(yw[i], scale, inverse, codes);
      else
        fp8_encode_pairs<4, false>(yw[i], scale, inverse, codes);
      if (valid(i))
        st_nt(reinterpret_cast<uint2 *>(a.packed + base + column(i)),
              make_uint2(codes[0] | (codes[1] << 16), codes[2] | (codes[3] << 16)));
    }
  }
}

// QuantizeFP8 (prefill.cuh:46-66): per row of x [rows][cols], scale = max|x| / 448 (1 for a
// zero row; fmaxf drops NaN) and codes = E4M3 of the correctly rounded x / scale; a
// non-finite value raises the flag.  One wave per row, 8 consecutive values per lane and
// step.  BF16 rows whose values are finite and whose maximum is >= 2^-100 take the fast
// quotient and the hardware conversion (the identities padra_CheckFP8Paths verifies for
// BF16 values); other rows divide.
template <class T>
__global__ __launch_bounds__(64) void k_quantize_fp8(const T *x, uint8_t *packed, float *scales,
                                                     int rows, int cols, int *bad) {
  const int row = blockIdx.x, lane = threadIdx.x;
  if (row >= rows)
    return;
  const T *xr = x + (size_t)row * cols;
  float amax = 0.f;
  bool fine = true, exact = true;
  for (int c = 8 * lane; c < cols; c += 512) {
    float v[8];
    ActIO<T>::load8(xr + c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      fine = fine && isfinite(v[i]);
      exact = exact && (__float_as_uint(v[i]) & 0xffffu) == 0;
      amax = fmaxf(amax, fabsf(v[i]));
    }
  }
  amax = xor_reduce<32>(amax, [](float x, float y) { return fmaxf(x, y); });
  const bool row_fine = __ballot(!fine) == 0, row_bf16 = __ballot(!exact) == 0;
  if (!row_fine && lane == 0)
    raise_bad(bad);
  const float scale = amax == 0.f ? 1.f : amax / 448.f;
  const float inverse = 1.f / scale;
  if (lane == 0)
    scales[row] = scale;
  const bool fast = row_fine && row_bf16 && fp8_fast_ok(amax, inverse); // wave-uniform
  for (int c = 8 * lane; c < cols; c += 512) {
    float v[8];
    ActIO<T>::load8(xr + c, v);
    uint32_t w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t lo, hi;
      if (fast) {
        lo = e4m3_pair_hw(fp8_quotient(v[4 * h], scale, inverse),
                          fp8_quotient(v[4 * h + 1], scale, inverse));
        hi = e4m3_pair_hw(fp8_quotient(v[4 * h + 2], scale, inverse),
                          fp8_quotient(v[4 * h + 3], scale, inverse));
      } else {
        lo = e4m3_code(v[4 * h] / scale) | (e4m3_code(v[4 * h + 1] / scale) << 8);
        hi = e4m3_code(v[4 * h + 2] / scale) | (e4m3_code(v[4 * h + 3] / scale) << 8);
      }
      w[h] = lo | (hi << 16);
    }
    *reinterpret_cast<uint2 *>(packed + (size_t)row * cols + c) = make_uint2(w[0], w[1]);
  }
}

#define PADRA_COMBINE_J(JV)                                                                  \
  case JV:                                                                                   \
    return f(std::integral_constant<int, JV>{});
template <class F> int combine_shape(int hidden, F &&f) {
  if (hidden % 128)
    return PADRA_UNSUPPORTED;
  switch (hidden / 128) {
    PADRA_COMBINE_J(8)
    PADRA_COMBINE_J(9)
    PADRA_COMBINE_J(16)
    PADRA_COMBINE_J(18)
    PADRA_COMBINE_J(32)
    PADRA_COMBINE_J(36)
  }
  return PADRA_UNSUPPORTED;
}
#undef PADRA_COMBINE_J

} // namespace

extern "C" int padra_Combine(void *stream, void *x, const void *down, const float *weights,
                             int rows, int hidden, int experts, int residual, int *bad,
                             int act) {
  if (!x || !down || !weights || !bad || rows < 1 || hidden < 8 || hidden % 8 ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32) || !aligned16(x) || !aligned16(down))
    return PADRA_INVALID_ARGUMENT;
  if (experts != kExperts)
    return PADRA_UNSUPPORTED;
  const long long groups = (long long)rows * (hidden / 8);
  const unsigned grid = (unsigned)std::min<long long>((groups + 255) / 256, 8192);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    if (residual)
      hipLaunchKernelGGL((k_combine<T, true>), dim3(grid), dim3(256), 0, s, static_cast<T *>(x),
                         static_cast<const T *>(down), weights, hidden, groups, bad);
    else
      hipLaunchKernelGGL((k_combine<T, false>), dim3(grid), dim3(256), 0, s,
                         static_cast<T *>(x), static_cast<const T *>(down), weights, hidden,
                         groups, bad);
    return launched("Combine");
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

extern "C" int padra_CombineNorm(void *stream, void *x, const void *down, const float *weights,
                                 void *normalized, const uint16_t *gamma, uint8_t *packed,
                                 float *scales, int rows, int hidden, int experts, float eps,
                                 float *statistics, int *bad, int act) {
  if (!x || !down || !weights || !normalized || !gamma || !bad || x == normalized || rows < 1 ||
      !(eps >= 0.f) || (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32) || !aligned16(x) ||
      !aligned16(down) || !aligned16(normalized) || !aligned16(gamma) ||
      (packed && (!scales || !aligned16(packed))))
    return PADRA_INVALID_ARGUMENT;
  if (experts != kExperts)
    return PADRA_UNSUPPORTED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    NormFP8Args<T> a;
    a.x = static_cast<const T *>(x);
    a.y = static_cast<T *>(normalized);
    a.gamma = gamma;
    a.packed = packed;
    a.scales = scales;
    a.stats = statistics;
    a.bad = bad;
    a.rows = rows;
    a.eps = eps;
    return combine_shape(hidden, [&](auto j) -> int {
      if constexpr (std::is_same<T, uint16_t>::value) {
        if (packed)
          hipLaunchKernelGGL((k_combine_norm_wide<j.value, true, kCombineWaves>), dim3(rows),
                             dim3(64 * kCombineWaves), 0, s, static_cast<uint16_t *>(x),
                             static_cast<const uint16_t *>(down), weights, a);
        else
          hipLaunchKernelGGL((k_combine_norm_wide<j.value, false, kCombineWaves>), dim3(rows),
                             dim3(64 * kCombineWaves), 0, s, static_cast<uint16_t *>(x),
                             static_cast<const uint16_t *>(down), weights, a);
      } else {
        if (packed)
          hipLaunchKernelGGL((k_combine_norm<j.value, T, true, kCombineWaves>), dim3(rows),
                             dim3(64 * kCombineWaves), 0, s,
                             static_cast<T *>(x), static_cast<const T *>(down), weights, a);
        else
          hipLaunchKernelGGL((k_combine_norm<j.value, T, false, kCombineWaves>), dim3(rows),
                             dim3(64 * kCombineWaves), 0, s,
                             static_cast<T *>(x), static_cast<const T *>(down), weights, a);
      }
      return launched("CombineNorm");
    });
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

extern "C" int padra_QuantizeFP8(void *stream, const void *x, uint8_t *packed, float *scales,
                                 int rows, int cols, int *bad, int act) {
  if (!x || !packed || !scales || !bad || rows < 1 || cols < 8 || cols % 8 ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32) || !aligned16(x) ||
      (reinterpret_cast<uintptr_t>(packed) & 7))
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == PADRA_ACT_BF16)
    hipLaunchKernelGGL((k_quantize_fp8<uint16_t>), dim3(rows), dim3(64), 0, s,
                       static_cast<const uint16_t *>(x), packed, scales, rows, cols, bad);
  else
    hipLaunchKernelGGL((k_quantize_fp8<float>), dim3(rows), dim3(64), 0, s,
                       static_cast<const float *>(x), packed, scales, rows, cols, bad);
  return launched("QuantizeFP8");
}
