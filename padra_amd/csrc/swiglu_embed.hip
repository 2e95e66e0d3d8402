// SwiGLU at the expert boundary and the embedding gather.
#include <stdio.h>

#include <algorithm>

#include "common.h"

using namespace padra;

namespace {

int launched(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fprintf(stderr, "padra: %s launch failed: %s\n", what, hipGetErrorString(e));
    return PADRA_INTERNAL;
  }
  return PADRA_OK;
}
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- SiLU table ---------------------------------------------------------------------------
//
// exl3_silu_lut::Build / Rounded (exl3_silu_lut.cuh:5-14): entry i is the BF16 bits of
// B(g / (1 + RN32(exp64(-g)))) for the gate g whose BF16 bits are i.
__global__ __launch_bounds__(256) void k_silu_table(uint16_t *table) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= 65536u)
    return;
  const float g = __uint_as_float(i << 16);
  const float e = (float)exp(-(double)g); // double exp, one rounding to fp32
  const float den = 1.f + e;
  table[i] = (uint16_t)(pack2(g / den, 0.f) & 0xffffu);
}

// Gates whose table entry is not a closed form: |g| in [2^-25, 256), both signs.  Below
// 2^-25, RN32(exp(-g)) is exactly 1 and the entry is B(g/2); from 256 up, exp(-g) is 0
// (g > 0: the entry is g) or overflows (g < 0: the entry is -0).  The span is staged in LDS.
constexpr unsigned kLutLo = 102u << 7, kLutHi = 135u << 7, kLutSpan = kLutHi - kLutLo;

__device__ __forceinline__ float silu_entry(uint32_t gb, const uint16_t *lut) {
  const float g = __uint_as_float(gb << 16);
  const uint32_t e = (gb >> 7) & 0xffu, sign = gb >> 15, mag = gb & 0x7fffu;
  if (e < 102u)
    return B(g * 0.5f);
  if (e >= 135u)
    return sign ? -0.f : g;
  return __uint_as_float((uint32_t)lut[sign * kLutSpan + (mag - kLutLo)] << 16);
}

// exl3_silu_lut::Activate (exl3_silu_lut.cuh:15-31): out = B(s * up), s the table entry of
// the gate.  A non-finite gate or up raises the flag and leaves the gate value in `out`
// (the reference skips the element of its in-place output); a non-finite product raises
// the flag and is written.
template <class T>
__global__ __launch_bounds__(512) void k_swiglu(const T *gate, const T *up, T *out,
                                                long long groups, const uint16_t *table,
                                                int *bad) {
  __shared__ uint16_t lut[2 * kLutSpan];
  for (unsigned i = threadIdx.x; i < kLutSpan / 8; i += blockDim.x) {
    reinterpret_cast<uint4 *>(lut)[i] = reinterpret_cast<const uint4 *>(table + kLutLo)[i];
    reinterpret_cast<uint4 *>(lut + kLutSpan)[i] =
        reinterpret_cast<const uint4 *>(table + 0x8000u + kLutLo)[i];
  }
  __syncthreads();
  bool fine = true;
  for (long long gi = blockIdx.x * (long long)blockDim.x + threadIdx.x; gi < groups;
       gi += (long long)gridDim.x * blockDim.x) {
    float g[8], u[8];
    ActIO<T>::load8(gate + gi * 8, g);
    ActIO<T>::load8(up + gi * 8, u);
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float r[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float gv = g[2 * p + q], uv = u[2 * p + q];
        const uint32_t bits = __float_as_uint(gv);
        if (!isfinite(gv) || !isfinite(uv) || (bits & 0xffffu)) {
          fine = false;
          r[q] = gv;
          continue;
        }
        const float value = silu_entry(bits >> 16, lut) * uv;
        fine = fine && bf16_finite(value);
        r[q] = value;
      }
      w[p] = pack2(r[0], r[1]);
    }
    ActIO<T>::store8(out + gi * 8, w);
  }
  if (!fine)
    raise_bad(bad);
}

// ---- embedding gather -------------------------------------------------------------------
//
// EmbedControlled / EmbedPrefillControlled / Embed (decode_control.cuh:68-79,
// prefill_control.cuh:3-22, inference.cu:181-187): out[t] = table[token_t].  The token
// comes from ids[t] (PADRA_POS_BASE), prompt ids[prompt_offset + t] after
// ValidPrefillState (PADRA_POS_PREFILL), or DecodeState t (PADRA_POS_DECODE).  An
// invalid state or a token outside [0, vocab) raises the flag and writes nothing.
template <class O>
__global__ __launch_bounds__(64) void k_embed(const uint16_t *table, const int32_t *ids, O *out,
                                              int hidden, int vocab, PosSrc src, int *bad) {
  const int t = blockIdx.x, lane = threadIdx.x & 63;
  bool ok;
  const int token = embed_token(src, ids, t, vocab, ok);
  if (!ok) {
    if (lane == 0)
      raise_bad(bad);
    return;
  }
  const uint4 *row = reinterpret_cast<const uint4 *>(table + (size_t)token * hidden);
  O *dst = out + (size_t)t * hidden;
  const int chunks = hidden / 8;
  for (int c = lane; c < chunks; c += 64) {
    const uint4 w = row[c];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    ActIO<O>::store8(dst + 8 * c, words);
  }
}

} // namespace

extern "C" int padra_SiluTableBuild(void *stream, uint16_t *table) {
  if (!table || !aligned16(table))
    return PADRA_INVALID_ARGUMENT;
  hipLaunchKernelGGL(k_silu_table, dim3(256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     table);
  return launched("SiluTableBuild");
}

extern "C" int padra_SwiGLU(void *stream, const void *gate, const void *up, void *out,
                            long long count, const uint16_t *table, int *bad, int act) {
  if (!gate || !up || !out || !table || !bad || count < 1 || count % 8 != 0 ||
      !aligned16(gate) || !aligned16(up) || !aligned16(out) || !aligned16(table) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  const long long groups = count / 8;
  // 512-thread workgroups, at most 1024 of them: each stages the SiLU table span (16.9 KB)
  // once, so fewer, larger workgroups halve that traffic against 256 x 2048 (config 3:
  // 19.7 -> 19.0 us); 768 or 512 workgroups, or 1024 threads, measured slower.
  const unsigned grid = (unsigned)std::min<long long>((groups + 511) / 512, 1024);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == PADRA_ACT_BF16)
    hipLaunchKernelGGL((k_swiglu<uint16_t>), dim3(grid), dim3(512), 0, s,
                       static_cast<const uint16_t *>(gate), static_cast<const uint16_t *>(up),
                       static_cast<uint16_t *>(out), groups, table, bad);
  else
    hipLaunchKernelGGL((k_swiglu<float>), dim3(grid), dim3(512), 0, s,
                       static_cast<const float *>(gate), static_cast<const float *>(up),
                       static_cast<float *>(out), groups, table, bad);
  return launched("SwiGLU");
}

extern "C" int padra_Embed(void *stream, const uint16_t *table, int vocab, int hidden,
                           const int32_t *ids, const padra_Positions *src, int tokens, void *out,
                           int *bad, int act) {
  if (!table || !out || !bad || vocab < 1 || hidden < 8 || hidden % 8 || tokens < 1 ||
      !aligned16(table) || !aligned16(out) || (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  PosSrc p{};
  p.mode = src ? src->mode : PADRA_POS_BASE;
  p.tokens = tokens;
  if (src) {
    p.maximum = src->maximum;
    p.vocab = src->vocab;
    p.epoch = src->binding_epoch;
    p.prefill = src->prefill;
    p.decode = src->decode;
  }
  if ((p.mode == PADRA_POS_BASE && !ids) || (p.mode == PADRA_POS_PREFILL && (!ids || !p.prefill)) ||
      (p.mode == PADRA_POS_DECODE && !p.decode) || p.mode < 0 || p.mode > PADRA_POS_DECODE)
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == PADRA_ACT_BF16)
    hipLaunchKernelGGL((k_embed<uint16_t>), dim3(tokens), dim3(64), 0, s, table, ids,
                       static_cast<uint16_t *>(out), hidden, vocab, p, bad);
  else
    hipLaunchKernelGGL((k_embed<float>), dim3(tokens), dim3(64), 0, s, table, ids,
                       static_cast<float *>(out), hidden, vocab, p, bad);
  return launched("Embed");
}
