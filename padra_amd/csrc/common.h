// Device primitives shared by the gfx950 kernels of the per-token layer path.
//
// Arithmetic contract (reference: /root/reference/src/cuda/inference.cu:52-59, 103-135):
//  - B(x): round-to-nearest-even to BF16 and back.  gfx950 has a native RNE
//    conversion (v_cvt_pk_bf16_f32), two values per instruction.
//  - every + - * / sqrt is one correctly rounded binary32 operation: the build uses
//    -ffp-contract=off and HIP's default correctly rounded division and sqrt.
//  - compensated (Neumaier) accumulation with the reference's exact step and tree
//    order, so sums of squares match bit for bit.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "padra_hip.h"

namespace padra {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// BF16 halves of a packed word (element 2w in the low half, 2w+1 in the high half).
__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// RNE-convert two floats to one packed BF16 word (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2_t f = {a, b};
  const bf16x2_t h = __builtin_convertvector(f, bf16x2_t);
  return __builtin_bit_cast(uint32_t, h);
}
// B(x) of inference.cu:52-54, in one instruction: the packed conversion of (0, x) puts
// the RNE BF16 of x in the high half over a zero low half, which is B(x)'s bit pattern.
__device__ __forceinline__ float B(float x) { return __uint_as_float(pack2(0.f, x)); }

// Neumaier step, inference.cu:103-109: the larger magnitude leads the Fast2Sum.
__device__ __forceinline__ void acc(float value, float &sum, float &error) {
  const float next = sum + value;
  const bool lead = fabsf(sum) >= fabsf(value);
  const float big = lead ? sum : value, small = lead ? value : sum;
  error = error + ((big - next) + small);
  sum = next;
}
// The same step when sum >= 0 and value >= 0 (squares and their partial sums): then
// |sum| >= |value| <=> sum >= value, so max/min pick the same operands.
// (AccumulatePositiveExact, positive_accumulate_exact.cuh:3-9, is this form.)
__device__ __forceinline__ void acc_pos(float value, float &sum, float &error) {
  const float next = sum + value;
  error = error + ((fmaxf(sum, value) - next) + fminf(sum, value));
  sum = next;
}
// Fold partner partial (s2, e2) into (s, e) as one shuffle-down step does
// (inference.cu:113-117): first the partner's sum, then its error.
//
// For sums of squares the second step never needs the reference's magnitude test
// (inference.cu:105): every residual of a step is at most 2^-24 of the partial sum it
// came from, partial sums only grow (non-negative terms, monotone rounding), and no
// partial takes more than ~40 steps, so |e2| < 2^-18 * s2 <= s after the first step.
// The test would always pick its first arm, (s - next) + e2, which is what is computed.
__device__ __forceinline__ void fold(float s2, float e2, float &s, float &e) {
  acc_pos(s2, s, e);
  const float next = s + e2;
  e = e + ((s - next) + e2);
  s = next;
}

// Value of lane (lane ^ M) for M a power of two below 64, through VALU exchanges instead
// of an LDS round trip (ds_bpermute): DPP quad permutes for 1 and 2; for 4 the half-row
// mirror (lane i of 8 reads 7 - i) then the quad reversal (i reads i ^ 3),
// 7 - (i ^ 3) = i ^ 4; for 8 a row rotation by 8.  For 16, v_permlane16_swap of the value
// with itself swaps rows 1 and 3 of the first operand with rows 0 and 2 of the second, so
// the first result holds row r - 1 in the odd rows and the second row r + 1 in the even
// ones; for 32, v_permlane32_swap does the same with the 32-lane halves.  The values are
// those of __shfl_xor(v, M): only the route differs.
template <int M> __device__ __forceinline__ uint32_t lane_xor_u(uint32_t v) {
  static_assert(M >= 1 && M <= 32 && (M & (M - 1)) == 0, "lane xor of a power of two below 64");
  const int i = (int)v;
  if constexpr (M == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0xb1 /* quad_perm [1,0,3,2] */, 0xf, 0xf, true);
  } else if constexpr (M == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0x4e /* quad_perm [2,3,0,1] */, 0xf, 0xf, true);
  } else if constexpr (M == 4) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(
        __builtin_amdgcn_mov_dpp(i, 0x141 /* row_half_mirror */, 0xf, 0xf, true),
        0x1b /* quad_perm [3,2,1,0] */, 0xf, 0xf, true);
  } else if constexpr (M == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0x128 /* row_ror:8 */, 0xf, 0xf, true);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(i, i, false, false);
    return (uint32_t)((threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(i, i, false, false);
    return (uint32_t)((threadIdx.x & 32) ? r[0] : r[1]);
  }
}
template <int M> __device__ __forceinline__ float lane_xor(float v) {
  return __uint_as_float(lane_xor_u<M>(__float_as_uint(v)));
}
template <int M> __device__ __forceinline__ int lane_xor(int v) {
  return (int)lane_xor_u<M>((uint32_t)v);
}
template <int M> __device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  return lane_xor_u<M>(v);
}
template <int M> __device__ __forceinline__ double lane_xor(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint64_t lo = lane_xor_u<M>((uint32_t)b), hi = lane_xor_u<M>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)((hi << 32) | lo));
}
// Lane 0's value, as a wave-uniform scalar.
__device__ __forceinline__ float lane0(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}
// The butterfly v = op(v, lane ^ d) for d = TOP, TOP / 2, ..., 1, in that order (the
// order of a shuffle-xor reduction loop from TOP down).
template <int TOP, class V, class Op> __device__ __forceinline__ V xor_reduce(V v, Op op) {
  if constexpr (TOP >= 1)
    return xor_reduce<TOP / 2>(op(v, lane_xor<TOP>(v)), op);
  else
    return v;
}
// ---------------------------------------------------------------------------------------
// Sum of squares without the reference's order, rounded to the reference's result when
// that result is certain.
//
// The reference sums the fp32 squares p_i >= 0 of a row (or head) with Accumulate
// (inference.cu:103-109) over a fixed tree: each thread folds its m squares in order,
// then ten shuffle-down levels (a warp's five, then five over the warp partials), two
// Accumulate steps per level, and it returns RN32(s + e) (inference.cu:134).  In every
// Accumulate step the new sum is RN(sum + value) and its rounding error is recovered
// exactly (Fast2Sum with the larger magnitude first); only `error = RN(error +
// residual)` rounds.  So s + e = S - sum_k delta_k exactly, S = sum p_i, where delta_k is
// the rounding error of the k-th error update, |delta_k| <= u |e_k|, u = 2^-24.
// Bound, for S < 2^126 (no partial overflows):
//  - every residual is at most u |next| of its step; along the tree that feeds the
//    result the steps' |next| add up to at most (m + 20) S (1 + 2^-20): each thread's
//    m partial sums are below its share of S, and each of the ten levels adds two steps
//    per receiving lane whose sums are disjoint parts of S;
//  - a residual enters at most D = m + 20 error updates on its way to the result (the
//    thread's m, then two per level), so sum_k |e_k| <= D (1 + 2^-20) sum |residual|;
//  - hence |s + e - S| <= 1.003 (m + 20)^2 u^2 S.
// The fp64 sum S64 of the same p_i (each exact in fp64), in any order whose longest
// chain of additions is `depth`, is within 1.001 depth 2^-53 S of S.  If RN32 maps both
// ends of [S64 (1 - c), S64 (1 + c)] to the same float f, with c above the sum of both
// bounds (and the rounding of the two ends), then S and s + e lie inside that interval,
// and RN32 being monotone, the reference's RN32(s + e) = f.
// Squares of BF16 values are exact in fp32 except below 2^-126, where RN32 moves each by at
// most 2^-150; with S >= 2^-60 that is under 2^-77 S for any row here, inside the 2^-51
// slack of the margin.
// Otherwise (a result near an fp32 rounding midpoint, about 2 c / 2^-23.5 of rows, or S
// outside [2^-60, 2^126), or a non-finite square) the caller replays the reference tree.
// m: squares per reference thread; depth: the fp64 summation's longest chain.
__host__ __device__ constexpr double sumsq_margin(int m, int depth) {
  return 1.01 * (1.003 * (m + 20.0) * (m + 20.0) * 0x1p-48 + 1.001 * depth * 0x1p-53) +
         0x1p-51;
}
// RN32 of an fp64 sum of squares when it is certain to equal the reference's compensated
// result (`out`), else false.  A NaN or infinite s fails the tests.
__device__ __forceinline__ bool certified_sum(double s, double margin, float &out) {
  const float lo = (float)__builtin_fma(-margin, s, s);
  const float hi = (float)__builtin_fma(margin, s, s);
  out = hi;
  return (lo == hi) & (s >= 0x1p-60) & (s < 0x1p126);
}
// acc + v^2 in fp64 for a BF16-exact v (v^2 has at most 16 significant bits: exact).
__device__ __forceinline__ double sq64(float v, double acc) {
  return __builtin_fma((double)v, (double)v, acc);
}
// acc + RN32(v * v) in fp64, for any fp32 v (the reference's __fmul_rn square).
__device__ __forceinline__ double sq64_rn(float v, double acc) { return acc + (double)(v * v); }
// The wave's total of an fp64 value, in every lane (xor butterfly: each level adds the
// same two values in every lane, so all lanes end equal).
__device__ __forceinline__ double wave_sum64(double v) {
  return xor_reduce<32>(v, [](double a, double b) { return a + b; });
}

// One Hadamard stage on lane bit log2(M): lower' = lower + upper, upper' = lower - upper,
// as one fused multiply-add with the lane's sign (+-1 products are exact, so the sum is
// rounded once, as the add or subtract is).
template <int M> __device__ __forceinline__ float hadamard_lane(float v, int lane) {
  const float o = lane_xor<M>(v);
  return __builtin_fmaf((lane & M) ? -1.f : 1.f, v, o);
}

// An empty use of v at this point of the program: its load is issued before here and is
// not sunk past a later branch.
__device__ __forceinline__ void pin(const uint4 &v) {
  asm volatile("" : : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}
__device__ __forceinline__ void pin(uint32_t v) { asm volatile("" : : "v"(v)); }
// A point that the compiler moves no instruction across: memory accesses written before it
// stay before (the clobber), and the machine scheduler moves nothing over it (a
// sched_barrier with an empty mask), so loads written before it are issued before any
// instruction written after it.
__device__ __forceinline__ void issue_point() {
  asm volatile("" : : : "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Streaming (non-temporal) global accesses for data each launch touches once: the
// activations, the KV rows.  On gfx950 these bypass the normal cache allocation policy;
// a plain store stream loses up to half its bandwidth to cache write-allocation when
// every load of a wave is issued before its stores.  Norm weights and the RoPE table
// are re-read by many waves and use ordinary loads.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t ld_nt(const uint32_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint2 ld_nt(const uint2 *p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(uint32_t *p, uint32_t v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_nt(uint2 *p, uint2 v) {
  const u32x2_t t = {v.x, v.y};
  __builtin_nontemporal_store(t, reinterpret_cast<u32x2_t *>(p));
}
__device__ __forceinline__ void st_nt(uint4 *p, uint4 v) {
  const u32x4_t t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t *>(p));
}
// Stores written through with the sc1 cache policy (global_store ... sc1).  For a kernel
// that streams each byte once this measured faster than non-temporal stores in some
// kernels (the expert combine + norm: 22.8 -> 21.5 us) and slower in others (the fused
// chain), so the choice is made per kernel.
__device__ __forceinline__ void st_wt(uint32_t *p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_wt(uint2 *p, uint2 v) {
  const u32x2_t t = {v.x, v.y};
  asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(t) : "memory");
}
// A store of more than 8 bytes reads its data VGPRs one cycle after it issues, so a VALU
// write to them needs one wait state in between.  The compiler inserts it after its own
// stores but cannot see into an asm block, so the block carries the s_nop itself; without
// it a following VALU write reused the data registers and 16 lanes stored stale words.
__device__ __forceinline__ void st_wt(uint4 *p, uint4 v) {
  const u32x4_t t = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 0" : : "v"(p), "v"(t) : "memory");
}
// Non-temporal (WT false) or written-through (WT true) streaming store.
template <bool WT, class P, class V> __device__ __forceinline__ void st_stream(P *p, V v) {
  if constexpr (WT)
    st_wt(p, v);
  else
    st_nt(p, v);
}
__device__ __forceinline__ float ld_nt(const float *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(float *p, float v) { __builtin_nontemporal_store(v, p); }

// 16-byte vector loads/stores of activations.  Eight consecutive elements map to one
// uint4 of BF16 or two uint4 of fp32.
template <class T> struct ActIO;
template <> struct ActIO<uint16_t> {
  static __device__ __forceinline__ void load8(const uint16_t *p, float (&v)[8]) {
    const uint4 w = ld_nt(reinterpret_cast<const uint4 *>(p));
    v[0] = lo16(w.x); v[1] = hi16(w.x); v[2] = lo16(w.y); v[3] = hi16(w.y);
    v[4] = lo16(w.z); v[5] = hi16(w.z); v[6] = lo16(w.w); v[7] = hi16(w.w);
  }
  template <bool WT = false>
  static __device__ __forceinline__ void store8(uint16_t *p, const uint32_t (&w)[4]) {
    st_stream<WT>(reinterpret_cast<uint4 *>(p), make_uint4(w[0], w[1], w[2], w[3]));
  }
};
template <> struct ActIO<float> {
  static __device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const uint4 a = ld_nt(reinterpret_cast<const uint4 *>(p));
    const uint4 b = ld_nt(reinterpret_cast<const uint4 *>(p + 4));
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  template <bool WT = false>
  static __device__ __forceinline__ void store8(float *p, const uint32_t (&w)[4]) {
    st_stream<WT>(reinterpret_cast<uint4 *>(p), make_uint4(w[0] << 16, w[0] & 0xffff0000u,
                                                           w[1] << 16, w[1] & 0xffff0000u));
    st_stream<WT>(reinterpret_cast<uint4 *>(p + 4), make_uint4(w[2] << 16, w[2] & 0xffff0000u,
                                                               w[3] << 16, w[3] & 0xffff0000u));
  }
};
__device__ __forceinline__ void load8_bf16(const uint16_t *p, float (&v)[8]) {
  ActIO<uint16_t>::load8(p, v);
}

// True when x stays finite after rounding to BF16: 0x7f7f8000 is the midpoint between the
// largest finite BF16 (0x7f7f, odd) and infinity, and it rounds to infinity.
__device__ __forceinline__ bool bf16_finite(float x) {
  return fabsf(x) < __uint_as_float(0x7f7f8000u);
}

// Ring slot of a non-negative position: the division runs only when the position has
// wrapped (pos >= cap), which a global cache (cap = capacity > pos) never does.
__device__ __forceinline__ int ring_slot(int pos, int cap) {
  if (pos >= cap)
    pos %= cap;
  return pos;
}

// Sets the caller's sticky error flag (reference: atomicExch(bad, 1)).
__device__ __forceinline__ void raise_bad(int *bad) {
  if (bad)
    atomicExch(bad, 1);
}

// The codes below are returned as a word whose low byte is the int8 code (two's
// complement); callers use that byte only.

// q8 code (kv_q8.cuh:12-14): RNE of the correctly rounded quotient, clamped to +-127.
__device__ __forceinline__ uint32_t q8_code(float value, float scale) {
  return (uint32_t)max(-127, min(127, (int)rintf(value / scale)));
}
// The same code through the head's cached reciprocal: q = v * inverse, r = q * scale - v
// (one fused multiply-add), q - r * inverse; three instructions where the correctly
// rounded division takes ten.  RNE then takes one addition: with |q| < 2^22, the float sum
// q + 1.5 * 2^23 lies in [2^23, 2^24), where the spacing is 1, so it is rounded to
// 1.5 * 2^23 + RNE(q) (1.5 * 2^23 is even, so ties go as RNE(q)'s), whose low byte is
// RNE(q) mod 256.  Here |v| <= amax and scale = RN(amax / 127), so |q| is within a few
// ulps of 127 at most and needs no clamp.  For every BF16 value v with |v| <= amax, amax a
// BF16 maximum whose scale = amax / 127 is at least 2^-100 (q8_fast_ok: then r, whose size
// is about 2^-24 |v|, loses at most 2^-150 to the subnormal range, which moves
// q - r * inverse by at most 2^-43), its code byte equals q8_code's: padra_CheckQ8Path
// compares the two on every such (amax, v) pair on the device.  With smaller scales the
// two differ (a scale of 2^-125 puts an exact 63.5 quotient at 63.499996).
__device__ __forceinline__ uint32_t q8_code_fast(float value, float scale, float inverse) {
  const float q = value * inverse;
  const float r = __builtin_fmaf(q, scale, -value);
  return __float_as_uint(__builtin_fmaf(-r, inverse, q) + 12582912.f);
}
__device__ __forceinline__ bool q8_fast_ok(float scale) { return scale >= 0x1p-100f; }
// q8_0 code (kv_q8_native.cuh:46-48): roundf (half away from zero) of v * inverse.
// roundf(v) (half away from zero) is (int)(v + copysign(0.49999997, v)) with the float
// sum rounded to nearest even and the conversion truncating, for every finite |v| < 2^23
// (0.49999997 is the float below 0.5; the oracle's po_round_away_mismatches checks all of
// them): three instructions instead of roundf's seven.
__device__ __forceinline__ uint32_t q8_0_code(float value, float inverse) {
  const float v = value * inverse;
  return (uint32_t)max(-127, min(127, (int)(v + __builtin_copysignf(0.49999997f, v))));
}
// The same without the clamp, for a value of a block whose inverse = 1 / (amax / 127) is
// finite: |value| <= amax puts |v| within a few ulps of 127, so the sum stays below 128
// and the truncation gives at most 127.  (An infinite inverse, amax below about 2^-121,
// needs the clamp.)
__device__ __forceinline__ uint32_t q8_0_code_in_range(float value, float inverse) {
  const float v = value * inverse;
  return (uint32_t)(int)(v + __builtin_copysignf(0.49999997f, v));
}
// Four codes (the low bytes of c0..c3) as one word, c0 in the lowest byte: three byte
// permutes instead of a mask, a shift and an or per code.
__device__ __forceinline__ uint32_t pack_codes4(uint32_t c0, uint32_t c1, uint32_t c2,
                                                uint32_t c3) {
  const uint32_t lo = __builtin_amdgcn_perm(c1, c0, 0x0c0c0400u); // c0, c1, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm(c3, c2, 0x0c0c0400u); // c2, c3, 0, 0
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);             // c0, c1, c2, c3
}
// A 32-byte control record read as eight words issued together: the checks below then
// work on registers, instead of one dependent load per field under short-circuit tests.
template <class S> __device__ __forceinline__ S load_state(const S *p) {
  static_assert(sizeof(S) == 32, "control records are 32 bytes");
  const uint32_t *w = reinterpret_cast<const uint32_t *>(p);
  uint32_t r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    r[i] = w[i];
  S s;
  __builtin_memcpy(&s, r, sizeof(S));
  return s;
}

// DecodeReadyAtLimit (context_admission.cuh:5-11) with the vocabulary bound a parameter.
// Bitwise '&' keeps the test branch-free.
__device__ __forceinline__ bool decode_ready(const padra_DecodeState &s, int maximum, int vocab) {
  return (maximum > 0) & (maximum <= 131072) & !s.stopped & !s.eos & (s.remaining > 0) &
         (s.token >= 0) & (s.token < vocab) & (s.capacity > 0) & (s.capacity <= maximum) &
         (s.position >= 0) & (s.position < s.capacity) & (s.global_valid == s.position) &
         (s.local_valid == min(s.position, 1024));
}
// ValidPrefillState (src/runtime/prefill_state.h:16-24).
__device__ __forceinline__ bool prefill_valid(const padra_PrefillState &s, int active_tokens,
                                              int capacity, uint32_t binding_epoch,
                                              int maximum) {
  return (s.valid == 1) & (s.binding_epoch == binding_epoch) & (s.request_epoch != 0) &
         (maximum > 0) & (maximum <= 131072) & (s.capacity == capacity) & (capacity > 0) &
         (capacity <= maximum) & (s.tokens == active_tokens) & (active_tokens > 0) &
         (active_tokens <= 2048) & (s.base >= 0) & (s.base <= capacity - active_tokens) &
         (s.committed == s.base) & (s.prompt_offset >= 0) &
         (s.prompt_offset <= capacity - active_tokens);
}

// Position source passed by value to kernels.
struct PosSrc {
  int mode, base, maximum, vocab, tokens;
  uint32_t epoch;
  const padra_PrefillState *prefill;
  const padra_DecodeState *decode;
};

// The token of embedding row t (Embed / EmbedPrefillControlled / EmbedControlled,
// inference.cu:181-187, prefill_control.cuh:3-22, decode_control.cuh:68-79): ids[t]
// (PADRA_POS_BASE), ids[prompt_offset + t] under a valid PrefillState, or the ready
// DecodeState t's token.  ok is false for an invalid state or a token outside [0, vocab).
__device__ __forceinline__ int embed_token(const PosSrc &src, const int32_t *ids, int t,
                                           int vocab, bool &ok) {
  int token = -1;
  ok = true;
  if (src.mode == PADRA_POS_BASE) {
    token = ids[t];
  } else if (src.mode == PADRA_POS_PREFILL) {
    const padra_PrefillState s = load_state(src.prefill);
    ok = prefill_valid(s, src.tokens, s.capacity, src.epoch, src.maximum);
    token = ok ? ids[s.prompt_offset + t] : -1;
  } else {
    const padra_DecodeState s = load_state(src.decode + t);
    ok = decode_ready(s, src.maximum, src.vocab);
    token = ok ? s.token : -1;
  }
  ok = ok && token >= 0 && token < vocab;
  return token;
}

// The control record token t's position depends on (PADRA_POS_PREFILL: the chunk's
// PrefillState; PADRA_POS_DECODE: sequence t's DecodeState).  Fetched apart from
// resolve_position so that a kernel can put the load in flight before its data loads.
union PosState {
  padra_PrefillState prefill;
  padra_DecodeState decode;
};
__device__ __forceinline__ PosState fetch_state(const PosSrc &p, int t) {
  PosState s;
  if (p.mode == PADRA_POS_PREFILL)
    s.prefill = load_state(p.prefill);
  else if (p.mode == PADRA_POS_DECODE)
    s.decode = load_state(p.decode + t);
  else
    s.prefill = padra_PrefillState{};
  return s;
}

// Resolves token t's absolute position; `ok` false means the unit must write nothing
// and the caller raises the flag.  With a cache binding (cap > 0) the state must admit
// the ring: cap <= capacity (StorePrefillControlled prefill_control.cuh:27-29,
// QKNormRopeStoreControlled qk_rope_store_exact.cuh:8), and for the quantized formats
// (`ring_exact`) cap is the capacity or the 1024-row local ring and `first` is the
// chunk rows that do not fit (kv_q8.cuh:36-38, 80-82; kv_q8_native.cuh:447-450).
__device__ __forceinline__ int resolve_position(const PosSrc &p, const PosState &st, int t,
                                                int cap, int first, bool ring_exact, bool &ok) {
  ok = true;
  if (p.mode == PADRA_POS_BASE)
    return p.base + t;
  if (p.mode == PADRA_POS_PREFILL) {
    const padra_PrefillState &s = st.prefill;
    ok = prefill_valid(s, p.tokens, s.capacity, p.epoch, p.maximum);
    if (cap > 0) {
      ok = ok & (cap <= s.capacity);
      if (ring_exact)
        ok = ok && (cap == s.capacity || cap == min(1024, s.capacity)) &&
             first == (cap == s.capacity ? 0 : max(0, p.tokens - cap));
    }
    return s.base + t;
  }
  const padra_DecodeState &s = st.decode;
  ok = decode_ready(s, p.maximum, p.vocab);
  if (cap > 0) {
    ok = ok & (cap <= s.capacity);
    if (ring_exact)
      ok = ok & ((cap == s.capacity) | (cap == min(1024, s.capacity)));
  }
  return ok ? s.position : 0;
}
__device__ __forceinline__ int resolve_position(const PosSrc &p, int t, int cap, int first,
                                                bool ring_exact, bool &ok) {
  return resolve_position(p, fetch_state(p, t), t, cap, first, ring_exact, ok);
}

} // namespace padra
