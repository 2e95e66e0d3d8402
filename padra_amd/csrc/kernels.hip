// gfx950 kernels and the extern "C" entry points of include/padra_hip.h for the
// residual-norm, Q/K-norm + RoPE + KV-store and fused chain paths.
//
// Launch geometry: one 64-lane wavefront per workgroup.  A residual-norm wave covers one
// row; a Q/K wave covers 16 head vectors, four lanes each.  Every wave issues its loads before any
// arithmetic, and there is no inter-wave communication, so the grid is a flat list of
// independent waves (thousands for a 2048-token chunk: >> 256 CUs).
#include <stdio.h>

#include <type_traits>

#include "norm_fp8.h"
#include "norm_rows.h"
#include "padra_hip_diag.h"
#include "norm_wg.h"
#include "qk_head.h"
#include "qk_quad.h"

using namespace padra;

namespace {

// BF16 rows: the 16-byte layout and the order-free sum of squares; fp32 rows: the
// ownership layout and the reference tree (the order-free sum measured slower there:
// 11.28 -> 11.95 us at 2048 x 2048).
template <int VT, int J, class T, bool RES>
__global__ __launch_bounds__(64) void k_norm(NormArgs<T> a) {
  __shared__ uint4 lds[VT * J / 8];
  constexpr bool BF = std::is_same<T, uint16_t>::value;
  norm_row_wave<VT, J, T, RES, BF, false, BF>(a, blockIdx.x, lds);
}

template <class T, int FMT> __global__ __launch_bounds__(64) void k_qk(QKArgs<T> a) {
  // the quad layout's image: 4 KB (BF16 activations) or 12 KB (fp32), twice the
  // activation pieces with a quantized cache (the K waves stage their V heads)
  __shared__ uint4 lds[quad_image_slots_fmt<T, FMT>()];
  // Quantized caches: the K waves (K heads with their V heads, the heaviest waves)
  // first, as in k_chain.
  long long w = blockIdx.x;
  if constexpr (FMT > PADRA_KV_BF16) {
    w += qk_q_waves(a.tokens, a.hq);
    if (w >= (long long)gridDim.x)
      w -= gridDim.x;
  }
  qk_heads_wave<T, FMT>(a, w, lds);
}

// Self-check of the two fast-path identities, over their whole domains:
//   A. e4m3_pair_hw(x) == e4m3_code(x) for every float with |x| <= 480 (2.28e9 inputs),
//      and the unclamped e4m3_pair_fast(x) == e4m3_code(x) for |x| <= 460;
//   B. for every BF16 maximum m >= 2^-100 (scale = m/448, inverse normal) and every BF16
//      v with |v| <= m, both signs: the code of fp8_quotient, through either conversion,
//      == the code of the correctly rounded division (2.1e9 pairs).
// Mismatches are added to counts[0] (A) and counts[1] (B).
__global__ __launch_bounds__(256) void k_check_fp8_hw(unsigned long long n,
                                                      unsigned long long *counts) {
  unsigned long long bad = 0;
  const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
  for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x; i < n;
       i += stride) {
    const float x = __uint_as_float((uint32_t)(i >> 1) | ((uint32_t)(i & 1) << 31));
    const uint32_t code = e4m3_code(x);
    bad += (e4m3_pair_hw(x, 0.f) & 0xffu) != code;
    if ((__float_as_uint(x) & 0x7fffffffu) <= 0x43e60000u) // |x| <= 460
      bad += (e4m3_pair_fast(x, 0.f) & 0xffu) != code;
  }
  if (bad)
    atomicAdd(&counts[0], bad);
}
__global__ __launch_bounds__(256) void k_check_fp8_quotient(unsigned long long *counts) {
  const uint32_t mb = blockIdx.x + 1; // BF16 bits of the maximum, 0x0001 .. 0x7f7f
  const float amax = __uint_as_float(mb << 16);
  const float scale = amax / 448.f, inverse = 1.f / scale;
  if (!fp8_fast_ok(amax, inverse))
    return; // block-uniform
  unsigned long long bad = 0;
  for (uint32_t vb = threadIdx.x; vb <= mb; vb += blockDim.x) {
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      const float v = __uint_as_float((vb << 16) | (sg ? 0x80000000u : 0u));
      const float q = fp8_quotient(v, scale, inverse);
      const uint32_t code = e4m3_code(v / scale);
      bad += ((e4m3_pair_hw(q, 0.f) & 0xffu) != code) + ((e4m3_pair_fast(q, 0.f) & 0xffu) != code);
    }
  }
  if (bad)
    atomicAdd(&counts[1], bad);
}

__global__ void k_zero_u64(unsigned long long *p, int n) {
  if ((int)threadIdx.x < n)
    p[threadIdx.x] = 0;
}

template <int J, class T> __global__ __launch_bounds__(64) void k_norm_fp8(NormFP8Args<T> a) {
  if constexpr (std::is_same<T, uint16_t>::value) {
    __shared__ uint4 lds[128 * J / 8]; // the row, for the rare ordered replay
    norm_fp8_row_wide<J>(a, blockIdx.x, lds);
  } else {
    norm_fp8_row_wave<J, T>(a, blockIdx.x);
  }
}

// Residual-norm rows per wave in the chain (BF16 or no cache).  Two rows per wave (1,024
// norm waves, so that with the Q/K waves the grid fits one round of 4 waves per SIMD)
// measured slower on the config-1 chunk: 13.21 -> 13.30 us, and with the inputs restored
// clean in HBM before each timed replay 12.55 -> 12.70 us.
constexpr int kChainRows = 1;

// Residual-norm waves first, then the Q/K waves.  Measured on MI355X for a 2048-token
// chunk, this order is 10% faster than spreading the norm rows evenly over the grid
// (Bresenham interleave) or over its first half: the early grid streams the four norm
// tensors alone, and the VALU-heavier Q/K waves follow as norm waves retire.  Putting the
// Q/K waves first measured 15% slower.
// GATHER: the norm rows read their x from the embedding table (the fused decode step).
// T: the activation type (BF16, or fp32 words holding BF16-exact values).
template <int VT, int J, int FMT, bool GATHER = false, class T = uint16_t>
__global__ __launch_bounds__(64) void k_chain(NormArgs<T> n, QKArgs<T> q, long long norm_waves,
                                              long long waves) {
  // The order-free sums of squares (sumsq_margin, common.h) with a BF16 or no cache; the
  // reference trees alone with a quantized cache or fp32 activations, where the order-free
  // form measured slower (config-1 chunk, inputs cold in HBM: rotated q8_0 14.12 -> 14.35
  // us; q8 and unrotated q8_0 within 1%; with inputs partly served by the Infinity Cache:
  // rotated q8_0 13.56 -> 14.59 us, q8 13.10 -> 13.86 us).
  constexpr bool FAST = FMT <= PADRA_KV_BF16 && std::is_same<T, uint16_t>::value;
  // the Q/K waves' image, or a BF16 row of the norm waves (the rare ordered-sum replay)
  constexpr int SLOTS = quad_image_slots_fmt<T, FMT>() > VT * J / 8 ? quad_image_slots_fmt<T, FMT>()
                                                                    : VT * J / 8;
  __shared__ uint4 lds[SLOTS];
  // Norm waves first, then the Q/K waves: measured against Q/K first (12.58 -> 13.53 us,
  // config-1 BF16 chunk) and a 2:3 interleave of the two kinds (12.85 us).
  const long long b = blockIdx.x;
  if (b < norm_waves) {
    if constexpr (FAST && !GATHER)
      norm_row_wave_wide<VT, J, true, kChainRows>(n, (int)b * kChainRows, lds);
    else
      norm_row_wave<VT, J, T, true, false, GATHER, FAST>(n, (int)b, lds);
  } else if (b < waves) {
    // Quantized caches: the K waves (K norm + RoPE, then the K and V encodings: the
    // heaviest waves) are dispatched before the Q waves instead of last, so they do not
    // form the grid's tail.
    long long w = b - norm_waves;
    if constexpr (FMT > PADRA_KV_BF16) {
      w += qk_q_waves(q.tokens, q.hq);
      if (w >= waves - norm_waves)
        w -= waves - norm_waves;
    }
    qk_heads_wave<T, FMT>(q, w, lds);
  }
}

// The fused chain for few tokens: a 256-lane workgroup per residual-norm row (norm_wg.h),
// then four Q/K head vectors per workgroup, one wave each (qk_head.h).
template <int VT, int J, int FMT, bool GATHER = false>
__global__ __launch_bounds__(256) void k_chain_small(NormArgs<uint16_t> n, QKArgs<uint16_t> q,
                                                     long long rows, long long head_waves) {
  __shared__ __attribute__((aligned(16))) float partials[8][2];
  const long long b = blockIdx.x;
  if (b < rows) { // workgroup-uniform
    norm_row_wg<VT, J, GATHER>(n, (int)b, partials);
    return;
  }
  const long long hv = (b - rows) * 4 + (threadIdx.x >> 6);
  if (hv < head_waves)
    qk_head_wave<uint16_t, FMT>(q, (unsigned)hv);
}

// The same with one wave per residual-norm row (norm_rows.h), for the 128-thread tree:
// its 16 elements per lane at H = 2048 measured faster in one wave (16 / 64 / 128 tokens:
// 3.4 / 3.7 / 4.0 us) than in a workgroup (4.1 / 4.1 / 4.5 us); the 256-thread decode tree
// is the other way round (64-sequence decode step: 4.5 -> 3.5 us).
// T: the activation type; fp32 activations take this kernel with either tree.
template <int VT, int J, int FMT, bool GATHER = false, class T = uint16_t>
__global__ __launch_bounds__(64) void k_chain_heads(NormArgs<T> n, QKArgs<T> q,
                                                    long long norm_waves, long long waves) {
  const long long b = blockIdx.x;
  if (b < norm_waves)
    norm_row_wave<VT, J, T, true, false, GATHER>(n, (int)b, nullptr);
  else if (b < waves)
    qk_head_wave<T, FMT>(q, (unsigned)(b - norm_waves));
}

// Residual + RMSNorm, BF16 rows, one 256-lane workgroup per row (norm_wg.h).
template <int VT, int J>
__global__ __launch_bounds__(256) void k_norm_small(NormArgs<uint16_t> n) {
  __shared__ __attribute__((aligned(16))) float partials[8][2];
  norm_row_wg<VT, J, false>(n, blockIdx.x, partials);
}

template <class T, int FMT> __global__ __launch_bounds__(64) void k_qk_heads(QKArgs<T> a) {
  qk_head_wave<T, FMT>(a, blockIdx.x);
}

#ifndef PADRA_HEAD_WAVE_TOKENS
#define PADRA_HEAD_WAVE_TOKENS 192
#endif
#ifndef PADRA_HEAD_WAVE_TOKENS_Q
#define PADRA_HEAD_WAVE_TOKENS_Q 320
#endif
// Launches of at most this many tokens use one wave per Q/K head vector (qk_head.h; with
// a quantized cache one wave per K head that also encodes the pair) and, in the fused
// chain, a workgroup (256-thread tree) or a wave (128) per norm row; larger ones the
// four-lanes-per-head waves (qk_quad.h) and a wave per row.  Measured on MI355X (prefill
// chain, 128-thread tree), per-head against quad:
//   BF16 cache: 3.0 / 3.2 / 3.8 / 4.5 / 5.2 / 6.7 us at 16 / 64 / 128 / 192 / 256 / 384
//   tokens against 4.3 / 4.4 / 4.9 / 5.0 / 5.2 / 5.3 us;
//   q8: 3.6 / 3.9 / 4.4 / 4.7 / 6.1 / 7.6 us against 6.6 / 6.9 / 7.2 / 7.3 / 7.4 / 7.5 us;
//   q8_0: 3.6 / 4.3 / 4.9 / 5.2 / 6.6 / 8.3 us against 7.1 / 7.3 / 7.6 / 7.7 / 7.9 / 8.1 us.
// fp32 activations (fused chain, 64 tokens): BF16 cache 4.0 against 5.8 us, q8 4.1 against
// 8.9, q8_0 4.2 against 8.1; with a BF16 cache per-head stays ahead up to 384 tokens (7.3
// against 7.6 us), quad from 512 (8.9 against 8.2).
#ifndef PADRA_HEAD_WAVE_TOKENS_F32
#define PADRA_HEAD_WAVE_TOKENS_F32 384
#endif
template <int FMT, class T = uint16_t> constexpr int head_wave_tokens() {
  if (FMT > PADRA_KV_BF16)
    return PADRA_HEAD_WAVE_TOKENS_Q;
  return std::is_same<T, float>::value ? PADRA_HEAD_WAVE_TOKENS_F32 : PADRA_HEAD_WAVE_TOKENS;
}
// The standalone residual-norm with the 256-thread tree takes a workgroup per row up to
// this many rows.
constexpr int kNormWgRows = 128;

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launched() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fprintf(stderr, "padra: kernel launch failed: %s\n", hipGetErrorString(e));
    return PADRA_INTERNAL;
  }
  return PADRA_OK;
}

// Residual-norm dispatch over the supported (tree, hidden/tree) pairs.
#define PADRA_NORM_J(VT, JV)                                                                 \
  case JV:                                                                                   \
    return f(std::integral_constant<int, VT>{}, std::integral_constant<int, JV>{});
template <class F> int norm_shape(int tree, int j, F &&f) {
  if (tree == 128) {
    switch (j) {
      PADRA_NORM_J(128, 8)
      PADRA_NORM_J(128, 9)
      PADRA_NORM_J(128, 16)
      PADRA_NORM_J(128, 18)
      PADRA_NORM_J(128, 32)
      PADRA_NORM_J(128, 36)
    }
  } else if (tree == 256) {
    switch (j) {
      PADRA_NORM_J(256, 4)
      PADRA_NORM_J(256, 8)
      PADRA_NORM_J(256, 9)
      PADRA_NORM_J(256, 16)
      PADRA_NORM_J(256, 18)
    }
  }
  return PADRA_UNSUPPORTED;
}
#undef PADRA_NORM_J

// The (tree, hidden/tree) pairs of the fused chain: H = 2048 and 2304 in either tree.
template <class F> int chain_shape(int tree, int j, F &&f) {
  using std::integral_constant;
  if (tree == 128 && j == 16)
    return f(integral_constant<int, 128>{}, integral_constant<int, 16>{});
  if (tree == 128 && j == 18)
    return f(integral_constant<int, 128>{}, integral_constant<int, 18>{});
  if (tree == 256 && j == 8)
    return f(integral_constant<int, 256>{}, integral_constant<int, 8>{});
  if (tree == 256 && j == 9)
    return f(integral_constant<int, 256>{}, integral_constant<int, 9>{});
  return PADRA_UNSUPPORTED;
}

// A runtime flag as a compile-time one.
template <class F> int with_flag(bool b, F &&f) {
  return b ? f(std::true_type{}) : f(std::false_type{});
}

int check_norm(const void *x, const void *normalized, const uint16_t *gamma, int rows,
               int hidden, float eps, int tree, int *bad, int act) {
  if (!x || !normalized || !gamma || !bad || x == normalized || rows < 1 || hidden < 1 ||
      !(eps >= 0.f) || (tree != 128 && tree != 256) || (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  if (!aligned16(x) || !aligned16(normalized) || !aligned16(gamma))
    return PADRA_INVALID_ARGUMENT;
  if (hidden % tree != 0)
    return PADRA_UNSUPPORTED;
  return PADRA_OK;
}

int rows_per_wave(int) { return 1; }

PosSrc make_pos(const padra_Positions &p, int tokens) {
  PosSrc s;
  s.mode = p.mode;
  s.base = p.base;
  s.maximum = p.maximum;
  s.vocab = p.vocab;
  s.tokens = tokens;
  s.epoch = p.binding_epoch;
  s.prefill = p.prefill;
  s.decode = p.decode;
  return s;
}

int check_qk(const void *q, const void *k, const void *v, const uint16_t *qn, const uint16_t *kn,
             const uint16_t *table, int table_rows, const padra_Positions *pos, int tokens,
             int q_heads, int kv_heads, int head_dim, float eps, const padra_KVCache *kv,
             int *bad, int act) {
  if (!q || !k || !qn || !kn || !table || !pos || !bad || table_rows < 1 || tokens < 1 ||
      q_heads < 1 || kv_heads < 1 || !(eps >= 0.f) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  if (head_dim != 128)
    return PADRA_UNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(qn) || !aligned16(kn) || !aligned16(table))
    return PADRA_INVALID_ARGUMENT;
  switch (pos->mode) {
  case PADRA_POS_BASE:
    if (pos->base < 0 || (long long)pos->base + tokens > 0x7fffffffLL)
      return PADRA_INVALID_ARGUMENT;
    break;
  case PADRA_POS_PREFILL:
    if (!pos->prefill || tokens > 2048 || pos->maximum < 1 || pos->maximum > 131072)
      return PADRA_INVALID_ARGUMENT;
    break;
  case PADRA_POS_DECODE:
    if (!pos->decode || pos->maximum < 1 || pos->maximum > 131072 || pos->vocab < 1)
      return PADRA_INVALID_ARGUMENT;
    break;
  default:
    return PADRA_INVALID_ARGUMENT;
  }
  if (kv) {
    if (!v || !kv->k || !kv->v || !aligned16(v) || !aligned16(kv->k) || !aligned16(kv->v) ||
        kv->cap < 1 || kv->first < 0 || kv->first >= tokens || kv->seq_stride < 0)
      return PADRA_INVALID_ARGUMENT;
    if (kv->format < PADRA_KV_BF16 || kv->format > PADRA_KV_Q8_0_NOROT)
      return PADRA_INVALID_ARGUMENT;
    if (kv->format == PADRA_KV_Q8 && (!kv->scales || (reinterpret_cast<uintptr_t>(kv->scales) & 7u)))
      return PADRA_INVALID_ARGUMENT;
    if (pos->mode == PADRA_POS_DECODE && tokens > 1 && kv->seq_stride < kv->cap)
      return PADRA_INVALID_ARGUMENT;
    if (pos->mode != PADRA_POS_DECODE && tokens - kv->first > kv->cap)
      return PADRA_INVALID_ARGUMENT; // a local ring stores at most its last `cap` rows
  }
  return PADRA_OK;
}

template <class T>
QKArgs<T> make_qk(void *q, void *k, const void *v, const uint16_t *qn, const uint16_t *kn,
                  const uint16_t *table, int table_rows, const padra_Positions *pos, int tokens,
                  int q_heads, int kv_heads, float eps, const padra_KVCache *kv, int *bad) {
  QKArgs<T> a;
  a.q = static_cast<T *>(q);
  a.k = static_cast<T *>(k);
  a.v = static_cast<const T *>(v);
  a.qn = qn;
  a.kn = kn;
  a.table = table;
  a.table_rows = table_rows;
  a.tokens = tokens;
  a.hq = q_heads;
  a.hkv = kv_heads;
  a.eps = eps;
  a.pos = make_pos(*pos, tokens);
  a.kc = kv ? kv->k : nullptr;
  a.vc = kv ? kv->v : nullptr;
  a.scales = kv ? kv->scales : nullptr;
  a.cap = kv ? kv->cap : 0;
  a.first = kv ? kv->first : 0;
  a.seq_stride = kv ? kv->seq_stride : 0;
  a.bad = bad;
  return a;
}

template <class F> int with_format(const padra_KVCache *kv, F &&f) {
  if (!kv)
    return f(std::integral_constant<int, -1>{});
  switch (kv->format) {
  case PADRA_KV_BF16:
    return f(std::integral_constant<int, PADRA_KV_BF16>{});
  case PADRA_KV_Q8:
    return f(std::integral_constant<int, PADRA_KV_Q8>{});
  case PADRA_KV_Q8_0:
    return f(std::integral_constant<int, PADRA_KV_Q8_0>{});
  case PADRA_KV_Q8_0_NOROT:
    return f(std::integral_constant<int, PADRA_KV_Q8_0_NOROT>{});
  }
  return PADRA_INVALID_ARGUMENT;
}

} // namespace

extern "C" int padra_ResidualPostNorm(void *stream, void *x, const void *residual,
                                      void *normalized, const uint16_t *gamma, int rows,
                                      int hidden, float eps, int tree, float *statistics,
                                      int *bad, int act) {
  int st = check_norm(x, normalized, gamma, rows, hidden, eps, tree, bad, act);
  if (st)
    return st;
  if (residual && (!aligned16(residual) || residual == x))
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = (rows + rows_per_wave(tree) - 1) / rows_per_wave(tree);
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    NormArgs<T> a;
    a.x = static_cast<T *>(x);
    a.residual = static_cast<const T *>(residual);
    a.y = static_cast<T *>(normalized);
    a.gamma = gamma;
    a.stats = statistics;
    a.bad = bad;
    a.rows = rows;
    a.eps = eps;
    return norm_shape(tree, hidden / tree, [&](auto vt, auto j) -> int {
      if constexpr (std::is_same<T, uint16_t>::value && vt.value == 256) {
        if (residual && rows <= kNormWgRows) {
          hipLaunchKernelGGL((k_norm_small<vt.value, j.value>), dim3(rows), dim3(256), 0, s, a);
          return launched();
        }
      }
      if (residual) {
        hipLaunchKernelGGL((k_norm<vt.value, j.value, T, true>), dim3(grid), dim3(64), 0, s, a);
      } else {
        hipLaunchKernelGGL((k_norm<vt.value, j.value, T, false>), dim3(grid), dim3(64), 0, s, a);
      }
      return launched();
    });
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

extern "C" int padra_NormFP8(void *stream, const void *x, void *normalized,
                             const uint16_t *gamma, uint8_t *packed, float *scales, int rows,
                             int hidden, float eps, float *statistics, int *bad, int act) {
  int st = check_norm(x, normalized, gamma, rows, hidden, eps, 128, bad, act);
  if (st)
    return st;
  if (!packed || !scales || !aligned16(packed))
    return PADRA_INVALID_ARGUMENT;
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
    return norm_shape(128, hidden / 128, [&](auto, auto j) -> int {
      hipLaunchKernelGGL((k_norm_fp8<j.value, T>), dim3(rows), dim3(64), 0, s, a);
      return launched();
    });
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

// Device self-check of q8_code_fast: for every positive finite BF16 maximum amax whose
// scale amax / 127 passes q8_fast_ok (scale >= 2^-100), and every BF16 v with
// |v| <= amax (both signs), the code byte through the reciprocal equals the code of the correctly rounded quotient
// (2.1e9 pairs).  Mismatches are added to counts[0].
__global__ __launch_bounds__(256) void k_check_q8(unsigned long long *counts) {
  const uint32_t mb = blockIdx.x + 1; // BF16 bits of the maximum, 0x0001 .. 0x7f7f
  const float amax = __uint_as_float(mb << 16);
  const float scale = amax / 127.f, inverse = 1.f / scale;
  if (!q8_fast_ok(scale))
    return; // block-uniform
  unsigned long long bad = 0;
  for (uint32_t vb = threadIdx.x; vb <= mb; vb += blockDim.x) {
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      const float v = __uint_as_float((vb << 16) | (sg ? 0x80000000u : 0u));
      bad += ((q8_code_fast(v, scale, inverse) ^ q8_code(v, scale)) & 0xffu) != 0;
    }
  }
  if (bad)
    atomicAdd(&counts[0], bad);
}

extern "C" int padra_CheckQ8Path(void *stream, unsigned long long *counts) {
  if (!counts)
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_zero_u64, dim3(1), dim3(64), 0, s, counts, 1);
  hipLaunchKernelGGL(k_check_q8, dim3(0x7f7f), dim3(256), 0, s, counts);
  return launched();
}

extern "C" int padra_CheckFP8Paths(void *stream, unsigned long long *counts) {
  if (!counts)
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_zero_u64, dim3(1), dim3(64), 0, s, counts, 2);
  hipLaunchKernelGGL(k_check_fp8_hw, dim3(8192), dim3(256), 0, s, 2ull * 0x43f00000ull, counts);
  hipLaunchKernelGGL(k_check_fp8_quotient, dim3(0x7f7f), dim3(256), 0, s, counts);
  return launched();
}

extern "C" int padra_QKNormRopeStore(void *stream, void *q, void *k, const void *v,
                                     const uint16_t *qn, const uint16_t *kn,
                                     const uint16_t *table, int table_rows,
                                     const padra_Positions *pos, int tokens, int q_heads,
                                     int kv_heads, int head_dim, float eps,
                                     const padra_KVCache *kv, int *bad, int act) {
  const int st = check_qk(q, k, v, qn, kn, table, table_rows, pos, tokens, q_heads, kv_heads,
                          head_dim, eps, kv, bad, act);
  if (st)
    return st;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    const QKArgs<T> a =
        make_qk<T>(q, k, v, qn, kn, table, table_rows, pos, tokens, q_heads, kv_heads, eps, kv, bad);
    return with_format(kv, [&](auto fmt) -> int {
      if (tokens <= head_wave_tokens<fmt.value, T>()) {
        const long long grid = qk_head_waves<fmt.value>(tokens, q_heads, kv_heads);
        hipLaunchKernelGGL((k_qk_heads<T, fmt.value>), dim3((unsigned)grid), dim3(64), 0, s, a);
        return launched();
      }
      const long long grid = qk_wave_count<fmt.value>(tokens, q_heads, kv_heads);
      hipLaunchKernelGGL((k_qk<T, fmt.value>), dim3((unsigned)grid), dim3(64), 0, s, a);
      return launched();
    });
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

namespace {

// The fused chain launch; with `gather` (non-null) the norm rows take x from the embedding
// table as padra_Embed would have written it.
int chain(hipStream_t s, const uint16_t *gather, int vocab, const int32_t *ids, void *x,
          const void *residual, void *normalized, const uint16_t *gamma, int hidden, int tree,
          float *statistics, void *q, void *k, const void *v, const uint16_t *qn,
          const uint16_t *kn, const uint16_t *table, int table_rows, const padra_Positions *pos,
          int tokens, int q_heads, int kv_heads, int head_dim, float eps,
          const padra_KVCache *kv, int *bad) {
  int st = check_norm(x, normalized, gamma, tokens, hidden, eps, tree, bad, PADRA_ACT_BF16);
  if (st)
    return st;
  if (!residual || !aligned16(residual) || residual == x)
    return PADRA_INVALID_ARGUMENT;
  st = check_qk(q, k, v, qn, kn, table, table_rows, pos, tokens, q_heads, kv_heads, head_dim, eps,
                kv, bad, PADRA_ACT_BF16);
  if (st)
    return st;
  NormArgs<uint16_t> n;
  n.x = static_cast<uint16_t *>(x);
  n.residual = static_cast<const uint16_t *>(residual);
  n.y = static_cast<uint16_t *>(normalized);
  n.gamma = gamma;
  n.stats = statistics;
  n.bad = bad;
  n.rows = tokens;
  n.eps = eps;
  if (gather) {
    // padra_Embed's token source for the same positions.
    if (vocab < 1 || !aligned16(gather))
      return PADRA_INVALID_ARGUMENT;
    n.gather = gather;
    n.ids = ids;
    n.vocab = vocab;
    n.src.mode = pos ? pos->mode : PADRA_POS_BASE;
    n.src.tokens = tokens;
    if (pos) {
      n.src.maximum = pos->maximum;
      n.src.vocab = pos->vocab;
      n.src.epoch = pos->binding_epoch;
      n.src.prefill = pos->prefill;
      n.src.decode = pos->decode;
    }
    if ((n.src.mode == PADRA_POS_BASE || n.src.mode == PADRA_POS_PREFILL) && !ids)
      return PADRA_INVALID_ARGUMENT;
  }
  const QKArgs<uint16_t> a = make_qk<uint16_t>(q, k, v, qn, kn, table, table_rows, pos, tokens,
                                               q_heads, kv_heads, eps, kv, bad);
  return chain_shape(tree, hidden / tree, [&](auto vt, auto j) -> int {
    return with_flag(gather != nullptr, [&](auto g) -> int {
      return with_format(kv, [&](auto fmt) -> int {
        constexpr int VT = vt.value, J = j.value, FMT = fmt.value;
        constexpr bool G = g.value;
        if (tokens <= head_wave_tokens<FMT>()) {
          const long long heads = qk_head_waves<FMT>(tokens, q_heads, kv_heads);
          if constexpr (VT == 256) {
            // One workgroup per norm row, then one per four head vectors.
            const dim3 grid((unsigned)(tokens + (heads + 3) / 4)), block(256);
            hipLaunchKernelGGL((k_chain_small<VT, J, FMT, G>), grid, block, 0, s, n, a,
                               (long long)tokens, heads);
          } else {
            const long long norm_waves = tokens, waves = norm_waves + heads;
            hipLaunchKernelGGL((k_chain_heads<VT, J, FMT, G>), dim3((unsigned)waves),
                               dim3(64), 0, s, n, a, norm_waves, waves);
          }
          return launched();
        }
        constexpr bool FAST = FMT <= PADRA_KV_BF16 && !G;
        const long long norm_waves = FAST ? (tokens + kChainRows - 1) / kChainRows : tokens;
        const long long waves = norm_waves + qk_wave_count<FMT>(tokens, q_heads, kv_heads);
        hipLaunchKernelGGL((k_chain<VT, J, FMT, G>), dim3((unsigned)waves), dim3(64), 0, s, n,
                           a, norm_waves, waves);
        return launched();
      });
    });
  });
}

} // namespace

namespace {
// The chain on fp32 activations (the reference's buffers): up to head_wave_tokens one
// launch of norm-row waves and per-head Q/K waves; above, the residual-norm launch, then
// the four-lanes-per-head Q/K launch.
int chain_f32(hipStream_t s, void *x, const void *residual, void *normalized,
              const uint16_t *gamma, int hidden, int tree, float *statistics, void *q, void *k,
              const void *v, const uint16_t *qn, const uint16_t *kn, const uint16_t *table,
              int table_rows, const padra_Positions *pos, int tokens, int q_heads, int kv_heads,
              int head_dim, float eps, const padra_KVCache *kv, int *bad) {
  int st = check_norm(x, normalized, gamma, tokens, hidden, eps, tree, bad, PADRA_ACT_F32);
  if (st)
    return st;
  if (!residual || !aligned16(residual) || residual == x)
    return PADRA_INVALID_ARGUMENT;
  st = check_qk(q, k, v, qn, kn, table, table_rows, pos, tokens, q_heads, kv_heads, head_dim, eps,
                kv, bad, PADRA_ACT_F32);
  if (st)
    return st;
  NormArgs<float> n;
  n.x = static_cast<float *>(x);
  n.residual = static_cast<const float *>(residual);
  n.y = static_cast<float *>(normalized);
  n.gamma = gamma;
  n.stats = statistics;
  n.bad = bad;
  n.rows = tokens;
  n.eps = eps;
  const QKArgs<float> a = make_qk<float>(q, k, v, qn, kn, table, table_rows, pos, tokens,
                                         q_heads, kv_heads, eps, kv, bad);
  const long long norm_waves = tokens;
  return chain_shape(tree, hidden / tree, [&](auto vt, auto j) -> int {
    return with_format(kv, [&](auto fmt) -> int {
      if (tokens <= head_wave_tokens<fmt.value, float>()) {
        const long long waves = norm_waves + qk_head_waves<fmt.value>(tokens, q_heads, kv_heads);
        hipLaunchKernelGGL((k_chain_heads<vt.value, j.value, fmt.value, false, float>),
                           dim3((unsigned)waves), dim3(64), 0, s, n, a, norm_waves, waves);
        return launched();
      }
      // Larger launches run the two halves as two kernels on the stream: one kernel would
      // give its norm rows the Q/K waves' registers (142 VGPRs, 3 waves per SIMD, against
      // 89 and 5 for the norm rows alone); config 1: 22.1 us in one kernel, 11.4 + 9.8 us
      // as two.
      hipLaunchKernelGGL((k_norm<vt.value, j.value, float, true>), dim3((unsigned)norm_waves),
                         dim3(64), 0, s, n);
      const int st2 = launched();
      if (st2)
        return st2;
      hipLaunchKernelGGL((k_qk<float, fmt.value>),
                         dim3((unsigned)qk_wave_count<fmt.value>(tokens, q_heads, kv_heads)),
                         dim3(64), 0, s, a);
      return launched();
    });
  });
}
} // namespace

extern "C" int padra_ResidualNormQKRopeStore(
    void *stream, void *x, const void *residual, void *normalized, const uint16_t *gamma,
    int hidden, int tree, float *statistics, void *q, void *k, const void *v,
    const uint16_t *qn, const uint16_t *kn, const uint16_t *table, int table_rows,
    const padra_Positions *pos, int tokens, int q_heads, int kv_heads, int head_dim, float eps,
    const padra_KVCache *kv, int *bad, int act) {
  if (act == PADRA_ACT_F32)
    return chain_f32(static_cast<hipStream_t>(stream), x, residual, normalized, gamma, hidden,
                     tree, statistics, q, k, v, qn, kn, table, table_rows, pos, tokens, q_heads,
                     kv_heads, head_dim, eps, kv, bad);
  if (act != PADRA_ACT_BF16)
    return PADRA_INVALID_ARGUMENT;
  return chain(static_cast<hipStream_t>(stream), nullptr, 0, nullptr, x, residual, normalized,
               gamma, hidden, tree, statistics, q, k, v, qn, kn, table, table_rows, pos, tokens,
               q_heads, kv_heads, head_dim, eps, kv, bad);
}

extern "C" int padra_EmbedResidualNormQKRopeStore(
    void *stream, const uint16_t *embed, int vocab, const int32_t *ids, void *x,
    const void *residual, void *normalized, const uint16_t *gamma, int hidden, int tree,
    float *statistics, void *q, void *k, const void *v, const uint16_t *qn, const uint16_t *kn,
    const uint16_t *table, int table_rows, const padra_Positions *pos, int tokens, int q_heads,
    int kv_heads, int head_dim, float eps, const padra_KVCache *kv, int *bad) {
  if (!embed)
    return PADRA_INVALID_ARGUMENT;
  return chain(static_cast<hipStream_t>(stream), embed, vocab, ids, x, residual, normalized,
               gamma, hidden, tree, statistics, q, k, v, qn, kn, table, table_rows, pos, tokens,
               q_heads, kv_heads, head_dim, eps, kv, bad);
}

// Streaming copy for the practical-ceiling measurement: 256-lane workgroups, 16 pieces of
// 16 bytes per lane, every load (non-temporal) issued before the first store (non-temporal).
// Of the copies measured on MI355X for a 61 MB move (workgroups of 64 to 1024 lanes, 4 to
// 16 pieces per lane, flat or persistent grids, plain, non-temporal or written-through
// stores) this shape is the fastest: 10.84 us, against 11.04-11.77 us for the others.
__global__ __launch_bounds__(256) void k_stream_copy(const uint4 *src, uint4 *dst, long long n) {
  constexpr int U = 16;
  const long long base = (long long)blockIdx.x * 256 * U + threadIdx.x;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    v[u] = ld_nt(src + min(base + 256LL * u, n - 1));
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (base + 256LL * u < n)
      st_nt(dst + base + 256LL * u, v[u]);
}

extern "C" int padra_StreamCopy(void *stream, void *dst, const void *src, long long bytes) {
  if (!dst || !src || bytes < 16 || bytes % 16 || !aligned16(dst) || !aligned16(src))
    return PADRA_INVALID_ARGUMENT;
  const long long n = bytes / 16;
  hipLaunchKernelGGL(k_stream_copy, dim3((unsigned)((n + 4095) / 4096)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4 *>(src),
                     static_cast<uint4 *>(dst), n);
  return launched();
}

extern "C" const char *padra_version(void) { return "padra-mi355x 0.1 gfx950 exact-fusions-v1"; }
