/*
 * padra_oracle.c -- CPU restatement of the reference arithmetic for Padra's
 * exact-fusions-v1 per-token layer path.  TEST INFRASTRUCTURE ONLY (the checker):
 * see padra_oracle.h.  Compile with -ffp-contract=off and without -ffast-math so
 * that every float operation below is one IEEE-754 binary32 operation with
 * round-to-nearest-even, as the reference's __fadd_rn/__fmul_rn/__fdiv_rn/
 * __fsqrt_rn intrinsics are.
 */
#include "padra_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t bits_of(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return b;
}
static float float_of(uint32_t b) {
  float x;
  memcpy(&x, &b, 4);
  return x;
}

/* ---- A1 -------------------------------------------------------------------- */

/* Round-to-nearest-even to BF16, as __float2bfloat16_rn (inference.cu:52-54) and the
 * reference's host form BHost (inference.cu:742-748).  NaN maps to the canonical
 * quiet NaN 0x7fff. */
uint16_t po_f32_to_bf16(float x) {
  uint32_t b = bits_of(x);
  if ((b & 0x7fffffffu) > 0x7f800000u)
    return 0x7fffu;
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}
float po_bf16_to_f32(uint16_t h) { return float_of((uint32_t)h << 16); }
float po_bf16_round(float x) { return po_bf16_to_f32(po_f32_to_bf16(x)); }

/* __float2half_rn: IEEE binary16, round to nearest even, gradual underflow. */
uint16_t po_f32_to_f16(float x) {
  const uint32_t b = bits_of(x);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x7f800000u)
    return sign | 0x7e00u;
  if (a >= 0x477ff000u) /* >= 65520 (midpoint above 65504, odd) rounds to infinity */
    return sign | 0x7c00u;
  if (a < 0x38800000u) { /* below 2^-14: binary16 subnormal, unit 2^-24 */
    const float scaled = float_of(a) * 16777216.0f; /* exact: power-of-two scaling */
    return sign | (uint16_t)lrintf(scaled);         /* default mode is RNE */
  }
  uint32_t h = ((((a >> 23) - 127u + 15u)) << 10) | ((a & 0x7fffffu) >> 13);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
    ++h;
  return sign | (uint16_t)h;
}
float po_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  if (e == 31)
    return float_of(sign | 0x7f800000u | (m << 13));
  return float_of(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

/* Neumaier step, inference.cu:103-109.  The branch picks the larger magnitude as
 * the Fast2Sum leader; the error term accumulates with one rounding per step. */
void po_accumulate(float value, float *sum, float *error) {
  const float s = *sum;
  const float next = s + value;
  const float residual = fabsf(s) >= fabsf(value) ? (s - next) + value : (value - next) + s;
  *error = *error + residual;
  *sum = next;
}

/* One warp-wide shuffle-down tree over 32 lanes (inference.cu:111-119): for d = 16..1
 * every lane l with l+d < 32 folds in lane l+d's (sum, error) as read before the step.
 * Lane 0 ends with the result. */
static void warp_tree(float *sum, float *error) {
  for (int d = 16; d; d /= 2) {
    float os[32], oe[32];
    memcpy(os, sum, sizeof os);
    memcpy(oe, error, sizeof oe);
    for (int l = 0; l + d < 32; ++l) {
      po_accumulate(os[l + d], &sum[l], &error[l]);
      po_accumulate(oe[l + d], &sum[l], &error[l]);
    }
  }
}

/* Block-wide compensated sum of squares.  Thread t accumulates v[t], v[t+threads], ...
 * in order (Norm inference.cu:197-198; ResidualPostNormWideExact
 * residual_norm_wide_exact.cuh:24-33 with threads = 256), each warp reduces with
 * warp_tree, warp results land in lanes 0..threads/32-1 of one warp (other lanes zero)
 * and that warp reduces again (inference.cu:120-135; residual_norm_wide_exact.cuh:
 * 45-58); the result is sum + error (inference.cu:135). */
float po_sumsq_tree(const float *v, int n, int threads) {
  float sum[256], error[256];
  const int warps = threads / 32;
  for (int t = 0; t < threads; ++t) {
    sum[t] = 0.f;
    error[t] = 0.f;
    for (int i = t; i < n; i += threads)
      po_accumulate(v[i] * v[i], &sum[t], &error[t]);
  }
  float ws[32], we[32];
  for (int l = 0; l < 32; ++l)
    ws[l] = we[l] = 0.f;
  for (int w = 0; w < warps; ++w) {
    warp_tree(sum + 32 * w, error + 32 * w);
    ws[w] = sum[32 * w];
    we[w] = error[32 * w];
  }
  warp_tree(ws, we);
  return ws[0] + we[0];
}

/* variance = S/n, inv = 1/sqrt(variance + eps); inference.cu:203-205. */
void po_rms_inv(float sumsq, int n, float eps, float *variance, float *inv) {
  const float var = sumsq / (float)n;
  *variance = var;
  *inv = 1.0f / sqrtf(var + eps);
}

/* ExpRN: fp64 exp rounded once to fp32 (inference.cu:57-59). */
float po_exp_rn(float x) { return (float)exp((double)x); }

static void set_bad(int *bad) {
  if (bad)
    *bad = 1;
}
static int finite_f(float x) { return isfinite(x) != 0; }

/* ---- A2 / A3 ------------------------------------------------------------------ */

/* Add (inference.cu:475-481) followed by Norm (inference.cu:188-214) for threads=128,
 * or ResidualPostNormWideExact (residual_norm_wide_exact.cuh:6-80) for threads=256:
 * v = B(x + r) is written back to x, y = B(B(v*inv) * gamma).  bad: a non-finite v
 * (Add, inference.cu:479) or row sum; with threads=256 also a non-finite output. */
void po_residual_rmsnorm(uint16_t *x, const uint16_t *residual, uint16_t *y,
                         const uint16_t *gamma, int rows, int hidden, float eps, int threads,
                         float *stats, int *bad) {
  float v[8192];
  for (int r = 0; r < rows; ++r) {
    uint16_t *xr = x + (long long)r * hidden;
    const uint16_t *rr = residual + (long long)r * hidden;
    uint16_t *yr = y + (long long)r * hidden;
    for (int i = 0; i < hidden; ++i) {
      v[i] = po_bf16_round(po_bf16_to_f32(xr[i]) + po_bf16_to_f32(rr[i]));
      xr[i] = po_f32_to_bf16(v[i]);
      if (!finite_f(v[i]))
        set_bad(bad);
    }
    const float s = po_sumsq_tree(v, hidden, threads);
    if (!finite_f(s))
      set_bad(bad);
    float var, inv;
    po_rms_inv(s, hidden, eps, &var, &inv);
    if (stats) {
      stats[2 * r] = var;
      stats[2 * r + 1] = inv;
    }
    for (int i = 0; i < hidden; ++i) {
      const float o = po_bf16_round(po_bf16_round(v[i] * inv) * po_bf16_to_f32(gamma[i]));
      yr[i] = po_f32_to_bf16(o);
      if (!finite_f(o) && threads == 256) /* residual_norm_wide_exact.cuh:77 */
        set_bad(bad);
    }
  }
}

/* Norm without residual (inference.cu:188-214; norm half of NormFP8Exact
 * norm_fp8_exact.cuh:22-45 and NormFP8WideExact norm_fp8_wide_exact.cuh:22-50). */
void po_rmsnorm(const uint16_t *x, uint16_t *y, const uint16_t *gamma, int rows, int hidden,
                float eps, int threads, float *stats, int *bad) {
  float v[8192];
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (long long)r * hidden;
    uint16_t *yr = y + (long long)r * hidden;
    for (int i = 0; i < hidden; ++i)
      v[i] = po_bf16_to_f32(xr[i]);
    const float s = po_sumsq_tree(v, hidden, threads);
    float var, inv;
    po_rms_inv(s, hidden, eps, &var, &inv);
    if (stats) {
      stats[2 * r] = var;
      stats[2 * r + 1] = inv;
    }
    for (int i = 0; i < hidden; ++i) {
      const float o = po_bf16_round(po_bf16_round(v[i] * inv) * po_bf16_to_f32(gamma[i]));
      yr[i] = po_f32_to_bf16(o);
      if (!finite_f(o))
        set_bad(bad);
    }
  }
}

/* ---- A3 FP8 E4M3 row encoding ---------------------------------------------------- */

/* E4M3 per the OCP 8-bit floating point specification: normals 2^-6 .. 448 with three
 * mantissa bits, subnormals k * 2^-9.  Written from the format definition. */
uint8_t po_e4m3(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u)
    return 0x7f; /* one NaN code whatever the input NaN's sign and payload */
  float a;
  memcpy(&a, &mag, 4);
  if (a >= 448.f)
    return (uint8_t)(sign | 0x7e);
  if (a < 0.015625f) /* 2^-6: subnormal codes k = RNE(a * 2^9), k = 8 is the least normal */
    return (uint8_t)(sign | (uint8_t)rintf(a * 512.f));
  /* normal: keep 3 of 23 mantissa bits, ties to even; a carry moves into the exponent */
  const uint32_t rounded = mag + 0x7ffffu + ((mag >> 20) & 1u);
  const uint32_t code = (rounded >> 20) - ((127u - 7u) << 3);
  return (uint8_t)(sign | (code > 0x7eu ? 0x7eu : code));
}

/* fp8_exact_reciprocal.cuh:5-11 */
int po_fp8_needs_division(uint32_t b) {
  if (b < 0x3a800000u)
    return b >= 0x3a800000u - 4u;
  const uint32_t e = b >> 23, shift = e < 121u ? 140u - e : 19u;
  const uint32_t residue = b & ((1u << (shift + 1)) - 1u), midpoint = 1u << shift;
  return residue >= midpoint - 4u && residue <= midpoint + 4u;
}

/* fp8_exact_reciprocal.cuh:12-21 */
uint8_t po_fp8_encode(float value, float scale, float inverse) {
  uint32_t ib;
  memcpy(&ib, &inverse, 4);
  ib &= 0x7fffffffu;
  if ((ib & 0x7f800000u) == 0 || (ib & 0x7f800000u) == 0x7f800000u)
    return po_e4m3(value / scale);
  float q = value * inverse;
  uint32_t b;
  memcpy(&b, &q, 4);
  if (po_fp8_needs_division(b & 0x7fffffffu))
    q = value / scale;
  return po_e4m3(q);
}

/* norm_fp8_exact.cuh:19-61 (MaxReduce inference.cu:257-268: fmaxf drops NaN operands). */
void po_norm_fp8(const uint16_t *x, uint16_t *normalized, const uint16_t *gamma,
                 uint8_t *packed, float *scales, int rows, int hidden, float eps, float *stats,
                 int *bad) {
  float v[8192], y[8192];
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (long long)r * hidden;
    for (int i = 0; i < hidden; ++i)
      v[i] = po_bf16_to_f32(xr[i]);
    const float s = po_sumsq_tree(v, hidden, 128);
    float var, inv;
    po_rms_inv(s, hidden, eps, &var, &inv);
    if (stats && r == 0) {
      stats[0] = var;
      stats[1] = inv;
    }
    float maximum = 0.f;
    for (int i = 0; i < hidden; ++i) {
      y[i] = po_bf16_round(po_bf16_round(v[i] * inv) * po_bf16_to_f32(gamma[i]));
      normalized[(long long)r * hidden + i] = po_f32_to_bf16(y[i]);
      if (!finite_f(y[i]))
        set_bad(bad);
      maximum = fmaxf(maximum, fabsf(y[i]));
    }
    const float scale = maximum == 0.f ? 1.f : maximum / 448.f;
    const float inverse = 1.f / scale;
    scales[r] = scale;
    for (int i = 0; i < hidden; ++i)
      packed[(long long)r * hidden + i] = po_fp8_encode(y[i], scale, inverse);
  }
}

/* prefill.cuh:46-66 */
void po_quantize_fp8(const float *x, uint8_t *packed, float *scales, int rows, int cols,
                     int *bad) {
  for (int r = 0; r < rows; ++r) {
    const float *xr = x + (long long)r * cols;
    float amax = 0.f;
    for (int c = 0; c < cols; ++c) {
      if (!finite_f(xr[c]))
        set_bad(bad);
      amax = fmaxf(amax, fabsf(xr[c]));
    }
    const float scale = amax == 0.f ? 1.f : amax / 448.f;
    scales[r] = scale;
    for (int c = 0; c < cols; ++c)
      packed[(long long)r * cols + c] = po_e4m3(xr[c] / scale);
  }
}

unsigned long long po_round_away_mismatches(uint64_t lo, uint64_t hi) {
  unsigned long long bad = 0;
  for (uint64_t b = lo; b < hi; ++b) {
    const uint32_t u = (uint32_t)b;
    float x;
    memcpy(&x, &u, 4);
    if (!finite_f(x) || fabsf(x) >= 8388608.f)
      continue;
    volatile float s = x + copysignf(0.49999997f, x); /* one float addition, RNE */
    bad += (int)s != (int)roundf(x);
  }
  return bad;
}

/* ---- Expert combine -------------------------------------------------------------- */

/* inference.cu:580-590; expert_exl3_prefill_packed_activations.cuh:86-102 */
void po_combine(uint16_t *x, const uint16_t *down, const float *weights, int rows, int hidden,
                int experts, int residual, int *bad) {
  for (int t = 0; t < rows; ++t)
    for (int i = 0; i < hidden; ++i) {
      float c = 0.f;
      for (int e = 0; e < experts; ++e) {
        const float d = po_bf16_to_f32(down[((long long)t * experts + e) * hidden + i]);
        c = po_bf16_round(c + po_bf16_round(d * weights[t * experts + e]));
      }
      uint16_t *xi = x + (long long)t * hidden + i;
      const float value = residual ? po_bf16_round(po_bf16_to_f32(*xi) + c) : c;
      if (!finite_f(value))
        set_bad(bad);
      *xi = po_f32_to_bf16(value);
    }
}

/* combine_norm_exact.cuh:22-71 */
void po_combine_norm(uint16_t *x, const uint16_t *down, const float *weights,
                     uint16_t *normalized, const uint16_t *gamma, uint8_t *packed,
                     float *scales, int rows, int hidden, int experts, float eps, float *stats,
                     int *bad) {
  float v[8192], y[8192];
  for (int t = 0; t < rows; ++t) {
    uint16_t *xr = x + (long long)t * hidden;
    po_combine(xr, down + (long long)t * experts * hidden, weights + (long long)t * experts, 1,
               hidden, experts, 1, bad);
    for (int i = 0; i < hidden; ++i)
      v[i] = po_bf16_to_f32(xr[i]);
    const float s = po_sumsq_tree(v, hidden, 128);
    float var, inv;
    po_rms_inv(s, hidden, eps, &var, &inv);
    if (stats && t == 0) {
      stats[0] = var;
      stats[1] = inv;
    }
    float maximum = 0.f;
    for (int i = 0; i < hidden; ++i) {
      y[i] = po_bf16_round(po_bf16_round(v[i] * inv) * po_bf16_to_f32(gamma[i]));
      normalized[(long long)t * hidden + i] = po_f32_to_bf16(y[i]);
      if (!finite_f(y[i]))
        set_bad(bad);
      maximum = fmaxf(maximum, fabsf(y[i]));
    }
    if (packed) {
      const float scale = maximum != 0.f ? maximum / 448.f : 1.f;
      const float inverse = 1.f / scale;
      scales[t] = scale;
      for (int i = 0; i < hidden; ++i)
        packed[(long long)t * hidden + i] = po_fp8_encode(y[i], scale, inverse);
    }
  }
}

/* ---- A5 -------------------------------------------------------------------------- */

/* RopeTable (inference.cu:764-785), with theta, head_dim and the YaRN constants as
 * parameters.  Float/double mix and evaluation order as in the reference. */
void po_rope_table(float *table, int positions, int head_dim, float theta, int yarn,
                   float factor, int original_context) {
  const int half = head_dim / 2;
  const double pi = acos(-1.0), base = (double)theta;
  const float low = (float)fmax(
      0., floor(head_dim * log(original_context / (32 * 2 * pi)) / (2 * log(base))));
  const float high = (float)fmin(
      (double)(head_dim - 1),
      ceil(head_dim * log(original_context / (2 * pi)) / (2 * log(base))));
  float frequencies[512];
  for (int i = 0; i < half; ++i) {
    const float freq = powf(theta, (float)(2 * i) / (float)head_dim);
    float ramp = ((float)i - low) / (high - low);
    ramp = ramp < 0.f ? 0.f : (ramp > 1.f ? 1.f : ramp);
    const float extra = 1 - ramp;
    frequencies[i] = !yarn ? 1 / freq
                           : (1 / (factor * freq)) * (1 - extra) + (1 / freq) * extra;
  }
  const float scale = !yarn ? 1.f : (float)(1 + 0.1 * log((double)factor));
  for (int p = 0; p < positions; ++p)
    for (int i = 0; i < half; ++i) {
      const float angle = (float)p * frequencies[i];
      table[(long long)p * head_dim + i] = po_bf16_round(cosf(angle) * scale);
      table[(long long)p * head_dim + half + i] = po_bf16_round(sinf(angle) * scale);
    }
}

/* ---- A4 / A6 ---------------------------------------------------------------------- */

/* QKNormRopeStoreControlled / QKNormRope / QKNormRopePair64 per head
 * (qk_rope_store_exact.cuh:27-44, qknorm_rope.cuh:27-50, qknorm_rope_pair64.cuh:30-82):
 * a 128-thread AccurateReduce tree over the D squares, inv, o = B(B(x*inv)*w), then
 * lo = B(B(a*c) + B((-b)*s)), hi = B(B(b*c) + B(a*s)) for each pair (i, i+D/2). */
void po_qk_norm_rope_head(uint16_t *x, const uint16_t *weight, const uint16_t *table_row,
                          int head_dim, float eps, int *bad) {
  float v[1024], o[1024];
  if (head_dim < 2 || head_dim > 1024 || head_dim % 2) { /* outside the local arrays */
    set_bad(bad);
    return;
  }
  const int half = head_dim / 2;
  for (int i = 0; i < head_dim; ++i)
    v[i] = po_bf16_to_f32(x[i]);
  /* v[0..head_dim) is written above; GCC cannot see that head_dim >= 2 holds here */
#pragma GCC diagnostic push
#pragma GCC diagnostic ignored "-Wmaybe-uninitialized"
  const float s = po_sumsq_tree(v, head_dim, 128);
#pragma GCC diagnostic pop
  float var, inv;
  po_rms_inv(s, head_dim, eps, &var, &inv);
  for (int i = 0; i < head_dim; ++i)
    o[i] = po_bf16_round(po_bf16_round(v[i] * inv) * po_bf16_to_f32(weight[i]));
  for (int i = 0; i < half; ++i) {
    const float c = po_bf16_to_f32(table_row[i]), sn = po_bf16_to_f32(table_row[half + i]);
    const float a = o[i], b = o[i + half];
    const float lo = po_bf16_round(po_bf16_round(a * c) + po_bf16_round((-b) * sn));
    const float hi = po_bf16_round(po_bf16_round(b * c) + po_bf16_round(a * sn));
    x[i] = po_f32_to_bf16(lo);
    x[i + half] = po_f32_to_bf16(hi);
    if (!finite_f(lo) || !finite_f(hi))
      set_bad(bad);
  }
}

void po_qk_norm_rope(uint16_t *q, uint16_t *k, const uint16_t *qn, const uint16_t *kn,
                     const uint16_t *table, const int *positions, int tokens, int q_heads,
                     int kv_heads, int head_dim, float eps, int *bad) {
  for (int t = 0; t < tokens; ++t) {
    const uint16_t *row = table + (long long)positions[t] * head_dim;
    for (int h = 0; h < q_heads; ++h)
      po_qk_norm_rope_head(q + ((long long)t * q_heads + h) * head_dim, qn, row, head_dim, eps,
                           bad);
    for (int h = 0; h < kv_heads; ++h)
      po_qk_norm_rope_head(k + ((long long)t * kv_heads + h) * head_dim, kn, row, head_dim, eps,
                           bad);
  }
}

void po_kv_store_bf16(const uint16_t *k, const uint16_t *v, uint16_t *kc, uint16_t *vc,
                      const int *positions, int tokens, int features, int cap, int first) {
  for (int t = first; t < tokens; ++t) {
    const long long slot = (long long)(positions[t] % cap) * features;
    memcpy(kc + slot, k + (long long)t * features, (size_t)features * 2);
    memcpy(vc + slot, v + (long long)t * features, (size_t)features * 2);
  }
}

/* ---- A7 ----------------------------------------------------------------------------- */

static int8_t q8_code(float value, float scale) { /* kv_q8.cuh:12-14 */
  long c = lrintf(value / scale); /* __float2int_rn(__fdiv_rn(value, scale)) */
  if (c > 127)
    c = 127;
  if (c < -127)
    c = -127;
  return (int8_t)c;
}

/* kv_q8::Encode<Controlled> (kv_q8.cuh:28-74) per (token, head) written straight to
 * slot pos%cap, as Encode followed by Commit (kv_q8.cuh:75-98) leaves the ring.
 * A head whose K or V values are non-finite or not BF16-exact sets bad and writes
 * nothing (the BF16-exactness holds by construction for BF16 inputs). */
void po_kv_q8_encode(const uint16_t *k, const uint16_t *v, int8_t *codes_k, int8_t *codes_v,
                     float *scales, const int *positions, int tokens, int kv_heads,
                     int head_dim, int cap, int first, int *bad) {
  const int features = kv_heads * head_dim;
  for (int t = first; t < tokens; ++t) {
    const long long slot = positions[t] % cap;
    for (int h = 0; h < kv_heads; ++h) {
      const uint16_t *kh = k + (long long)t * features + h * head_dim;
      const uint16_t *vh = v + (long long)t * features + h * head_dim;
      float km = 0.f, vm = 0.f;
      int invalid = 0;
      for (int i = 0; i < head_dim; ++i) {
        const float a = po_bf16_to_f32(kh[i]), b = po_bf16_to_f32(vh[i]);
        invalid |= !finite_f(a) || !finite_f(b);
        km = fmaxf(km, fabsf(a));
        vm = fmaxf(vm, fabsf(b));
      }
      if (invalid) {
        set_bad(bad);
        continue;
      }
      const float ks = km == 0 ? 1.f : km / 127.f, vs = vm == 0 ? 1.f : vm / 127.f;
      if (!finite_f(ks) || !finite_f(vs) || ks <= 0 || vs <= 0) {
        set_bad(bad);
        continue;
      }
      scales[(slot * kv_heads + h) * 2] = ks;
      scales[(slot * kv_heads + h) * 2 + 1] = vs;
      for (int i = 0; i < head_dim; ++i) {
        codes_k[slot * features + h * head_dim + i] = q8_code(po_bf16_to_f32(kh[i]), ks);
        codes_v[slot * features + h * head_dim + i] = q8_code(po_bf16_to_f32(vh[i]), vs);
      }
    }
  }
}

/* kv_q8::Decode (kv_q8.cuh:15-27): returns 0 and sets bad-equivalent on rejection. */
int po_kv_q8_decode(int8_t code, float scale, uint16_t *out) {
  if (code == -128 || !finite_f(scale) || scale <= 0) {
    *out = 0x7fffu;
    return 0;
  }
  const float product = (float)code * scale;
  const uint16_t value = po_f32_to_bf16(product);
  if (!finite_f(product) || (value & 0x7f80u) == 0x7f80u) {
    *out = 0x7fffu;
    return 0;
  }
  *out = value;
  return 1;
}

/* ---- A8 ------------------------------------------------------------------------------- */

/* q8_native::Rotate<W> (kv_q8_native.cuh:22-45).  Feature f = lane + 32*r; the lane
 * butterflies (d = 1..16) are stages on bits 0..4 of f and the register butterflies
 * (d = 1, 2) stages on bits 5, 6, in that order.  Each stage sets
 * lower' = lower + upper, upper' = lower - upper; then every value is scaled. */
void po_hadamard(float *x, int n, float scale) {
  for (int bit = 1; bit < n; bit *= 2)
    for (int f = 0; f < n; ++f)
      if (!(f & bit)) {
        const float lower = x[f], upper = x[f | bit];
        x[f] = lower + upper;
        x[f | bit] = lower - upper;
      }
  for (int f = 0; f < n; ++f)
    x[f] = x[f] * scale;
}

int po_q8_0_row_bytes(int features) {
  const int raw = 2 * (features / 32) + features;
  return (raw + 15) / 16 * 16;
}

/* q8_native::Code (kv_q8_native.cuh:46-48): roundf (half away from zero) of v * (1/ad). */
static int8_t q8_0_code(float value, float inverse) {
  /* The reference's (int) of the rounded float is CUDA's saturating conversion (NaN to 0,
   * out-of-range values to the int limits), then the clamp to +-127; C leaves the
   * conversion of infinities and NaN undefined, so those cases are written out.  An
   * infinite product comes from a block whose 1/ad overflows (ad subnormal). */
  const float r = roundf(value * inverse);
  int c;
  if (r != r)
    c = 0;
  else if (r >= 127.f)
    c = 127;
  else if (r <= -127.f)
    c = -127;
  else
    c = (int)r;
  return (int8_t)c;
}

/* q8_native::EncodeKV (kv_q8_native.cuh:52-101) written straight to slot pos%cap as
 * EncodeKV + Commit (kv_q8_native.cuh:440-463) leave the ring.  K gets a normalized
 * 128-point transform (scale 0.08838834764831845f), V two 64-point transforms (0.125).
 * Blocks are encoded in order r = 0..D/32-1, K and V together; a block whose amax or
 * fp16 scale is not finite sets bad and stops that head, as the reference returns. */
void po_kv_q8_0_encode(const uint16_t *k, const uint16_t *v, uint8_t *rows_k, uint8_t *rows_v,
                       const int *positions, int tokens, int kv_heads, int head_dim, int cap,
                       int first, int rotate, int *bad) {
  const int features = kv_heads * head_dim, nd = features / 32, per = head_dim / 32;
  const int row_bytes = po_q8_0_row_bytes(features);
  for (int t = first; t < tokens; ++t) {
    const long long slot = positions[t] % cap;
    uint8_t *rk = rows_k + slot * row_bytes, *rv = rows_v + slot * row_bytes;
    for (int h = 0; h < kv_heads; ++h) {
      float a[1024], b[1024];
      int invalid = 0;
      for (int i = 0; i < head_dim; ++i) {
        a[i] = po_bf16_to_f32(k[(long long)t * features + h * head_dim + i]);
        b[i] = po_bf16_to_f32(v[(long long)t * features + h * head_dim + i]);
        invalid |= !finite_f(a[i]) || !finite_f(b[i]);
      }
      if (invalid) {
        set_bad(bad);
        continue;
      }
      if (rotate) {
        po_hadamard(a, head_dim, .08838834764831845f);
        for (int s = 0; s < head_dim; s += 64)
          po_hadamard(b + s, 64, .125f);
      }
      for (int r = 0; r < per; ++r) {
        float am = 0.f, bm = 0.f;
        for (int l = 0; l < 32; ++l) {
          am = fmaxf(am, fabsf(a[r * 32 + l]));
          bm = fmaxf(bm, fabsf(b[r * 32 + l]));
        }
        const float ad = am / 127.f, bd = bm / 127.f;
        const uint16_t ah = po_f32_to_f16(ad), bh = po_f32_to_f16(bd);
        if (!finite_f(am) || !finite_f(bm) || !finite_f(po_f16_to_f32(ah)) ||
            !finite_f(po_f16_to_f32(bh))) {
          set_bad(bad);
          break;
        }
        memcpy(rk + 2 * (h * per + r), &ah, 2);
        memcpy(rv + 2 * (h * per + r), &bh, 2);
        const float ia = ad == 0.f ? 0.f : 1.f / ad, ib = bd == 0.f ? 0.f : 1.f / bd;
        for (int l = 0; l < 32; ++l) {
          rk[2 * nd + h * head_dim + r * 32 + l] = (uint8_t)q8_0_code(a[r * 32 + l], ia);
          rv[2 * nd + h * head_dim + r * 32 + l] = (uint8_t)q8_0_code(b[r * 32 + l], ib);
        }
      }
    }
  }
}

/* q8_native::Dequantize (kv_q8_native.cuh:366-390) to BF16 output. */
void po_kv_q8_0_dequantize(const uint8_t *rows_k, const uint8_t *rows_v, uint16_t *out_k,
                           uint16_t *out_v, int rows, int features, int *bad) {
  const int nd = features / 32, row_bytes = po_q8_0_row_bytes(features);
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < features; ++i) {
      const uint8_t *rk = rows_k + (long long)r * row_bytes, *rv = rows_v + (long long)r * row_bytes;
      uint16_t hk, hv;
      memcpy(&hk, rk + 2 * (i / 32), 2);
      memcpy(&hv, rv + 2 * (i / 32), 2);
      const float kd = po_f16_to_f32(hk), vd = po_f16_to_f32(hv);
      const int8_t ck = (int8_t)rk[2 * nd + i], cv = (int8_t)rv[2 * nd + i];
      if ((i % 32 == 0 && (!finite_f(kd) || !finite_f(vd) || kd < 0 || vd < 0)) || ck == -128 ||
          cv == -128)
        set_bad(bad);
      out_k[(long long)r * features + i] = po_f32_to_bf16((float)ck * kd);
      out_v[(long long)r * features + i] = po_f32_to_bf16((float)cv * vd);
    }
}

/* ---- A10 -------------------------------------------------------------------------------- */

/* exl3_silu_lut::Rounded (exl3_silu_lut.cuh:5-8): B(g / (1 + RN32(exp64(-g)))). */
uint16_t po_silu_bf16(uint16_t gate) {
  const float g = po_bf16_to_f32(gate);
  const float denominator = 1.f + (float)exp(-(double)g);
  return po_f32_to_bf16(g / denominator);
}
void po_silu_table(uint16_t *table) {
  for (uint32_t i = 0; i < 65536u; ++i)
    table[i] = po_silu_bf16((uint16_t)i);
}

/* exl3_silu_lut::Activate (exl3_silu_lut.cuh:15-31): non-finite gate or up sets bad and
 * leaves the element; otherwise out = B(s*u).  The direct form (inference.cu:575-579)
 * yields the same bits for finite inputs. */
void po_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out, long long count,
               int *bad) {
  for (long long i = 0; i < count; ++i) {
    const float g = po_bf16_to_f32(gate[i]), u = po_bf16_to_f32(up[i]);
    if (!finite_f(g) || !finite_f(u)) {
      set_bad(bad);
      continue;
    }
    const float s = po_bf16_to_f32(po_silu_bf16(gate[i]));
    const float value = po_bf16_round(s * u);
    if (!finite_f(value))
      set_bad(bad);
    out[i] = po_f32_to_bf16(value);
  }
}

/* ---- A11 ---------------------------------------------------------------------------------- */

void po_embed(const uint16_t *table, const int32_t *ids, uint16_t *out, int tokens, int hidden,
              int vocab, int *bad) {
  for (int t = 0; t < tokens; ++t) {
    const int32_t id = ids[t];
    if (id < 0 || id >= vocab) {
      set_bad(bad);
      continue;
    }
    memcpy(out + (long long)t * hidden, table + (long long)id * hidden, (size_t)hidden * 2);
  }
}

/* ---- A12 ------------------------------------------------------------------------------------ */

int po_decode_ready(const po_DecodeState *s, int maximum, int vocab) {
  return maximum > 0 && maximum <= 131072 && s && !s->stopped && !s->eos && s->remaining > 0 &&
         s->token >= 0 && s->token < vocab && s->capacity > 0 && s->capacity <= maximum &&
         s->position >= 0 && s->position < s->capacity && s->global_valid == s->position &&
         s->local_valid == (s->position < 1024 ? s->position : 1024);
}

int po_valid_prefill_state(const po_PrefillState *s, int active_tokens, int capacity,
                           uint32_t binding_epoch, int maximum) {
  return s->valid == 1 && s->binding_epoch == binding_epoch && s->request_epoch != 0 &&
         maximum > 0 && maximum <= 131072 && s->capacity == capacity && capacity > 0 &&
         capacity <= maximum && s->tokens == active_tokens && active_tokens > 0 &&
         active_tokens <= 2048 && s->base >= 0 && s->base <= capacity - active_tokens &&
         s->committed == s->base && s->prompt_offset >= 0 &&
         s->prompt_offset <= capacity - active_tokens;
}

/* ---- Local-ring checkpoint capture ------------------------------------------------ */

/* kv_checkpoint.cuh:12-25 */
void po_kv_checkpoint_plane(const uint8_t *old_rows, const uint8_t *current_rows,
                            uint8_t *saved_rows, int row_bytes, int base, int anchor) {
  for (int slot = 0; slot < 1024; ++slot) {
    const int position = anchor - 1 - ((anchor - 1 - slot + 1024) % 1024);
    uint8_t *dst = saved_rows + (long long)slot * row_bytes;
    if (position >= base)
      memcpy(dst, current_rows + (long long)(position - base) * row_bytes, (size_t)row_bytes);
    else if (position >= 0)
      memcpy(dst, old_rows + (long long)slot * row_bytes, (size_t)row_bytes);
    else
      memset(dst, 0, (size_t)row_bytes);
  }
}

/* kv_checkpoint.cuh:33-38 */
int po_kv_checkpoint_admitted(const po_PrefillState *s, int tokens, int anchor,
                              uint32_t binding_epoch, int maximum) {
  return po_valid_prefill_state(s, tokens, s->capacity, binding_epoch, maximum) &&
         s->capacity >= 1024 && anchor > s->base && anchor <= s->base + tokens;
}

/* ---- Decode attention -------------------------------------------------------------- */

/* __shfl_xor butterfly sum over 32 lanes (levels 16, 8, 4, 2, 1): every lane ends with
 * the same value; this is lane 0's. */
static float butterfly_sum32(const float *x) {
  float v[32], w[32];
  memcpy(v, x, sizeof v);
  for (int d = 16; d; d /= 2) {
    for (int l = 0; l < 32; ++l)
      w[l] = v[l] + v[l ^ d];
    memcpy(v, w, sizeof v);
  }
  return v[0];
}

int po_decode_attention(const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int cap,
                        int position, int local, int hq, int hkv, int splits, uint16_t *out,
                        int *bad) {
  const int D = 128, G = hq / hkv, features = hkv * D;
  const float scale = .08838834764831845f;
  const int n = local ? (position + 1 < 1024 ? position + 1 : 1024) : position + 1;
  const int first = position + 1 - n, tiles = (n + 31) / 32;
  if (splits <= 0) {
    splits = (cap + 31) / 32;
    if (splits > (local ? 16 : 32))
      splits = local ? 16 : 32;
  }
  const int active = splits < tiles ? splits : tiles;
  float *partial = (float *)calloc((size_t)active * hq * D, sizeof(float));
  float *lse = (float *)calloc((size_t)active * hq, sizeof(float));
  for (int sp = 0; sp < active; ++sp) {
    const int begin = tiles * sp / active, end = tiles * (sp + 1) / active;
    for (int head = 0; head < hq; ++head) {
      const int kv = head / G;
      float qf[128], accum[128], maximum = -INFINITY, denominator = 0.f;
      for (int d = 0; d < D; ++d) {
        qf[d] = po_bf16_to_f32(q[head * D + d]);
        accum[d] = 0.f;
      }
      for (int tile = begin; tile < end; ++tile) {
        float s[32], prob[32], p[32], mx = -INFINITY;
        int row[32];
        for (int j = 0; j < 32; ++j) {
          const int offset = tile * 32 + j;
          row[j] = offset < n ? (first + offset) % cap : -1;
          if (row[j] < 0) {
            s[j] = -INFINITY;
            continue;
          }
          float dot = 0.f;
          for (int d = 0; d < D; ++d)
            dot += qf[d] * po_bf16_to_f32(kc[(long long)row[j] * features + kv * D + d]);
          s[j] = dot * scale;
          if (!finite_f(s[j]))
            set_bad(bad);
          mx = fmaxf(mx, s[j]);
        }
        const float next = fmaxf(maximum, mx);
        const float a = finite_f(maximum) ? expf(maximum - next) : 0.f;
        for (int j = 0; j < 32; ++j) {
          prob[j] = finite_f(s[j]) ? expf(s[j] - next) : 0.f;
          p[j] = po_bf16_round(prob[j]);
        }
        const float total = butterfly_sum32(prob);
        maximum = next;
        denominator = fmaf(denominator, a, total);
        for (int d = 0; d < D; ++d) {
          float acc = accum[d] * a;
          for (int j = 0; j < 32; ++j)
            if (row[j] >= 0)
              acc += p[j] * po_bf16_to_f32(vc[(long long)row[j] * features + kv * D + d]);
          accum[d] = acc;
        }
      }
      for (int d = 0; d < D; ++d) {
        const float value = accum[d] / denominator;
        partial[((long long)sp * hq + head) * D + d] = value;
        if (!finite_f(value))
          set_bad(bad);
      }
      lse[sp * hq + head] = maximum + logf(denominator);
      if (!finite_f(lse[sp * hq + head]))
        set_bad(bad);
    }
  }
  for (int head = 0; head < hq; ++head) {
    float v[32], w[32], weights[32], mx = -INFINITY;
    for (int l = 0; l < 32; ++l) {
      v[l] = l < active ? lse[l * hq + head] : -INFINITY;
      mx = fmaxf(mx, v[l]);
    }
    for (int l = 0; l < 32; ++l)
      w[l] = l < active ? expf(v[l] - mx) : 0.f;
    const float den = butterfly_sum32(w);
    for (int l = 0; l < active; ++l) {
      weights[l] = w[l] / den;
      if (!finite_f(weights[l]))
        set_bad(bad);
    }
    for (int d = 0; d < D; ++d) {
      float sum = 0.f;
      for (int sp = 0; sp < active; ++sp)
        sum = fmaf(weights[sp], partial[((long long)sp * hq + head) * D + d], sum);
      const float value = po_bf16_round(sum);
      out[head * D + d] = po_f32_to_bf16(value);
      if (!finite_f(value))
        set_bad(bad);
    }
  }
  free(partial);
  free(lse);
  return active;
}

/* ---- Decode attention over a q8_0 cache ----------------------------------------------- */

static float half_bits_to_f32(const uint8_t *p) {
  uint16_t h;
  memcpy(&h, p, 2);
  return po_f16_to_f32(h);
}

/* kv_q8_native.cuh:103-148, 198-363 */
int po_decode_attention_q8_0(const uint16_t *q, const uint8_t *kc, const uint8_t *vc, int cap,
                             int position, int local, int hq, int hkv, int splits, uint16_t *out,
                             int *bad) {
  const int D = 128, G = hq / hkv, features = hkv * D, rb = po_q8_0_row_bytes(features);
  const int dbytes = 2 * (features / 32);
  const float scale = .08838834764831845f;
  if (local ? cap != 1024 : position >= cap) { /* the ring the reference admits */
    set_bad(bad);
    return -1;
  }
  /* EncodeQuery */
  int8_t qcode[64][128];
  float qd[64][4];
  for (int h = 0; h < hq; ++h) {
    float x[128];
    for (int d = 0; d < D; ++d) {
      x[d] = po_bf16_to_f32(q[h * D + d]);
      if (!finite_f(x[d])) {
        set_bad(bad);
        return -1;
      }
    }
    po_hadamard(x, 128, .08838834764831845f);
    for (int b = 0; b < 4; ++b) {
      float m = 0.f;
      for (int i = 0; i < 32; ++i)
        m = fmaxf(m, fabsf(x[32 * b + i]));
      const float d = m / 127.f;
      if (!finite_f(d)) {
        set_bad(bad);
        return -1;
      }
      qd[h][b] = d;
      for (int i = 0; i < 32; ++i)
        qcode[h][32 * b + i] = q8_0_code(x[32 * b + i], d == 0.f ? 0.f : 1.f / d);
    }
  }
  const int n = local ? (position + 1 < 1024 ? position + 1 : 1024) : position + 1;
  const int first = position + 1 - n, tiles = (n + 127) / 128;
  if (splits <= 0)
    splits = local ? 16 : 32;
  const int active = splits < tiles ? splits : tiles;
  float *partial = (float *)calloc((size_t)active * hq * D, sizeof(float));
  float *lse = (float *)calloc((size_t)active * hq, sizeof(float));
  for (int sp = 0; sp < active; ++sp) {
    const int begin = tiles * sp / active, end = tiles * (sp + 1) / active;
    for (int head = 0; head < hq; ++head) {
      const int kv = head / G;
      float mx[4], den[4][32], accum[4][128];
      for (int s = 0; s < 4; ++s) {
        mx[s] = -INFINITY;
        for (int l = 0; l < 32; ++l)
          den[s][l] = 0.f;
        for (int d = 0; d < D; ++d)
          accum[s][d] = 0.f;
      }
      for (int tile = begin; tile < end; ++tile)
        for (int s = 0; s < 4; ++s) {
          float own[32], p[32], ks[32][4], vs[32][4];
          const int8_t *kq[32], *vq[32];
          static const int8_t zeros[128];
          float top = -INFINITY;
          for (int k = 0; k < 32; ++k) {
            const int offset = tile * 128 + s * 32 + k;
            if (offset < n) {
              const int row = local ? (first + offset) & 1023 : first + offset;
              const uint8_t *kr = kc + (long long)row * rb, *vr = vc + (long long)row * rb;
              for (int b = 0; b < 4; ++b) {
                ks[k][b] = half_bits_to_f32(kr + 2 * (kv * 4 + b));
                vs[k][b] = half_bits_to_f32(vr + 2 * (kv * 4 + b));
              }
              kq[k] = (const int8_t *)(kr + dbytes + kv * D);
              vq[k] = (const int8_t *)(vr + dbytes + kv * D);
            } else {
              for (int b = 0; b < 4; ++b)
                ks[k][b] = vs[k][b] = 0.f;
              kq[k] = vq[k] = zeros;
            }
            float part[4];
            for (int sub = 0; sub < 4; ++sub) {
              float dot = 0.f;
              for (int b = 0; b < 4; ++b) {
                int sum = 0;
                for (int half = 0; half < 2; ++half) {
                  const int word = b * 8 + sub + 4 * half; /* 4-code group of block b */
                  for (int i = 0; i < 4; ++i)
                    sum += kq[k][4 * word + i] * qcode[head][4 * word + i];
                }
                dot = fmaf((float)sum, ks[k][b] * qd[head][b], dot);
              }
              part[sub] = dot;
            }
            const float dot = (part[0] + part[1]) + (part[2] + part[3]);
            own[k] = offset < n ? dot * scale : -INFINITY;
            top = fmaxf(top, own[k]);
          }
          const float next = fmaxf(mx[s], top);
          const float alpha = finite_f(mx[s]) ? expf(mx[s] - next) : 0.f;
          for (int k = 0; k < 32; ++k) {
            p[k] = finite_f(own[k]) ? expf(own[k] - next) : 0.f;
            den[s][k] = fmaf(den[s][k], alpha, p[k]);
          }
          mx[s] = next;
          for (int d = 0; d < D; ++d) {
            float acc = accum[s][d] * alpha;
            for (int k = 0; k < 32; ++k)
              acc = fmaf(p[k] * vs[k][d / 32], (float)vq[k][d], acc);
            accum[s][d] = acc;
          }
        }
      float total = 0.f, sum[128], top = -INFINITY;
      for (int s = 0; s < 4; ++s) {
        const float d = butterfly_sum32(den[s]);
        mx[s] = d > 0 ? mx[s] + logf(d) : -INFINITY;
        for (int i = 0; i < D; ++i)
          accum[s][i] = d > 0 ? accum[s][i] / d : 0.f;
      }
      top = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
      for (int i = 0; i < D; ++i)
        sum[i] = 0.f;
      for (int s = 0; s < 4; ++s) {
        const float w = finite_f(mx[s]) ? expf(mx[s] - top) : 0.f;
        total += w;
        for (int i = 0; i < D; ++i)
          sum[i] = fmaf(w, accum[s][i], sum[i]);
      }
      if (!(total > 0.f) || !finite_f(total)) {
        set_bad(bad);
        continue;
      }
      for (int i = 0; i < D; ++i)
        partial[((long long)sp * hq + head) * D + i] = sum[i] / total;
      lse[sp * hq + head] = top + logf(total);
    }
  }
  for (int head = 0; head < hq; ++head) {
    float v[32], w[32], weights[32], mx = -INFINITY, x[128];
    for (int l = 0; l < 32; ++l) {
      v[l] = l < active ? lse[l * hq + head] : -INFINITY;
      mx = fmaxf(mx, v[l]);
    }
    for (int l = 0; l < 32; ++l)
      w[l] = l < active ? expf(v[l] - mx) : 0.f;
    const float den = butterfly_sum32(w);
    for (int l = 0; l < active; ++l)
      weights[l] = w[l] / den;
    for (int d = 0; d < D; ++d) {
      float acc = 0.f;
      for (int sp = 0; sp < active; ++sp)
        acc = fmaf(weights[sp], partial[((long long)sp * hq + head) * D + d], acc);
      x[d] = acc;
    }
    po_hadamard(x, 64, .125f);
    po_hadamard(x + 64, 64, .125f);
    for (int d = 0; d < D; ++d) {
      if (!finite_f(x[d]))
        set_bad(bad);
      out[head * D + d] = po_f32_to_bf16(x[d]);
    }
  }
  free(partial);
  free(lse);
  return active;
}
