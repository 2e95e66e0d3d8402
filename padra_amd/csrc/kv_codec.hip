// KV-cache writers that run apart from the Q/K norm: the store/encode of already rotated
// K rows and V rows, the commit of an encoded chunk into the ring, the q8_0 decode back to
// BF16, and the Hadamard row rotation used around q8_0 prefill attention.
#include <stdio.h>

#include <algorithm>
#include <type_traits>

#include "qk_quad.h"

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

PosSrc pos_src(const padra_Positions &p, int tokens) {
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

int check_positions(const padra_Positions *pos, int tokens) {
  if (!pos || tokens < 1)
    return PADRA_INVALID_ARGUMENT;
  switch (pos->mode) {
  case PADRA_POS_BASE:
    return pos->base < 0 || (long long)pos->base + tokens > 0x7fffffffLL ? PADRA_INVALID_ARGUMENT
                                                                          : PADRA_OK;
  case PADRA_POS_PREFILL:
    return !pos->prefill || tokens > 2048 || pos->maximum < 1 || pos->maximum > 131072
               ? PADRA_INVALID_ARGUMENT
               : PADRA_OK;
  case PADRA_POS_DECODE:
    return !pos->decode || pos->maximum < 1 || pos->maximum > 131072 || pos->vocab < 1
               ? PADRA_INVALID_ARGUMENT
               : PADRA_OK;
  }
  return PADRA_INVALID_ARGUMENT;
}

// ---- store / encode of K and V rows ----------------------------------------------------
//
// A wave covers 8 (token, KV head) pairs, four lanes per head vector (lane g of a quad:
// features 32g .. 32g+31, one q8_0 block): lanes 0-31 hold the K vectors, lanes 32-63 the
// V vectors of the same pairs, so that the pair's K and V quads (lane ^ 32) can decide
// together what is written, as the reference's one warp per (token, head) does.  Both
// halves run one instruction stream: the q8_0 rotation's K-only stage (feature bit 6) takes
// its partner through a DPP move that is enabled in the K rows of the wave only (V lanes
// read 0), with the per-lane sign and scale making it the identity plus the 1/8 scale for
// V.  BF16 rows are a plain copy.
// `write` (equal in the K and V quads of a pair): false for a pair that writes nothing,
// whose lanes still take part in the exchanges (with zeros in x).
template <int FMT, class A>
__device__ __forceinline__ void encode_quad_rt(const A &a, float (&x)[32], long long slot,
                                               int h, int g, bool isv, bool write) {
  constexpr int D = 128;
  const int features = a.hkv * D;
  bool invalid = false;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    invalid |= !isfinite(x[i]);
    if constexpr (FMT == PADRA_KV_Q8) // q8 also rejects values that are not BF16-exact
      invalid |= (__float_as_uint(x[i]) & 0xffffu) != 0;
  }
  // an invalid K or V vector: neither is written (every lane runs the exchanges)
  uint32_t bad_any = invalid ? 1u : 0u;
  bad_any |= quad_xor1(bad_any);
  bad_any |= quad_xor2(bad_any);
  bad_any |= lane_xor<32>(bad_any);
  if (bad_any) {
    if (write && g == 0 && !isv)
      raise_bad(a.bad);
    return;
  }
  if constexpr (FMT == PADRA_KV_Q8) {
    // kv_q8::Encode (kv_q8.cuh:56-73): scale = amax/127 (1 for an all-zero head), codes
    // RNE(x / scale) clamped to +-127; the (k, v) scale pair as one 8-byte store.
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      m = fmaxf(m, fabsf(x[i]));
    m = fmaxf(m, fquad_xor1(m));
    m = fmaxf(m, fquad_xor2(m));
    const float scale = m == 0.f ? 1.f : m / 127.f, inverse = 1.f / scale;
    const bool fast = q8_fast_ok(scale); // quad-uniform
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      auto code = [&](float v) { return fast ? q8_code_fast(v, scale, inverse) : q8_code(v, scale); };
      w[i] = pack_codes4(code(x[4 * i]), code(x[4 * i + 1]), code(x[4 * i + 2]),
                         code(x[4 * i + 3]));
    }
    const float vscale = lane_xor<32>(scale);
    if (!write)
      return;
    store_codes32(static_cast<int8_t *>(isv ? a.vc : a.kc) + slot * features + h * D + 32 * g, w);
    if (g == 0 && !isv)
      reinterpret_cast<float2 *>(a.scales)[slot * a.hkv + h] = make_float2(scale, vscale);
  } else {
    if constexpr (FMT == PADRA_KV_Q8_0) {
      // q8_native::Rotate (kv_q8_native.cuh:22-45): feature bits 0-4 in the lane, bit 5
      // across lanes g ^ 1, bit 6 (K only) across lanes g ^ 2, then the scale.
      // Both quad stages in the signed form (hadamard_quad_signed): the value held is the
      // rotated one times -1 per stage taken on an upper lane, and that sign rides in the
      // scale multiply (codes do not see the sign of a zero).
      hadamard32(x);
      hadamard_quad_signed<1>(x, g);
      const bool neg2 = !isv && (g & 2);
      const float sgn = neg2 ? -1.f : 1.f;
      const float sc = ((g & 1) != neg2) ? (isv ? -.125f : -.08838834764831845f)
                                         : (isv ? .125f : .08838834764831845f);
#pragma unroll
      for (int f = 0; f < 32; ++f) {
        // lane g ^ 2's value in the K rows (rows 0 and 1 of the wave), 0 in the V rows
        const float other = __int_as_float(__builtin_amdgcn_update_dpp(
            0, __float_as_int(x[f]), 0x4e /* quad_perm [2,3,0,1] */, 0x3, 0xf, false));
        x[f] = __builtin_fmaf(other, sgn, x[f]) * sc;
      }
    }
    // Block g (kv_q8_native.cuh:84-99): d = half(amax/127), codes roundf(x * (1/d_fp32)).
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      am = fmaxf(am, fabsf(x[i]));
    const float ad = am / 127.f;
    const __half dh = __float2half(ad);
    const bool fail = !isfinite(am) || !isfinite(__half2float(dh));
    // A failing block stops the reference at that block, in K and V together.
    uint32_t stop = fail ? (uint32_t)g : 4u;
    stop = min(stop, quad_xor1(stop));
    stop = min(stop, quad_xor2(stop));
    stop = min(stop, lane_xor<32>(stop));
    if (!write)
      return;
    if (stop < 4u && g == 0 && !isv)
      raise_bad(a.bad);
    if ((uint32_t)g >= stop)
      return;
    const float inverse = ad == 0.f ? 0.f : 1.f / ad;
    uint32_t w[8];
    q8_0_codes32(x, inverse, w);
    const int row_bytes = ((2 * (features / 32) + features) + 15) / 16 * 16;
    uint8_t *row = static_cast<uint8_t *>(isv ? a.vc : a.kc) + slot * row_bytes;
    reinterpret_cast<uint16_t *>(row)[h * 4 + g] = __half_as_ushort(dh);
    store_codes32(reinterpret_cast<int8_t *>(row + 2 * (features / 32) + h * D + 32 * g), w);
  }
}

template <class T, int FMT>
__global__ __launch_bounds__(64) void k_kv_store(QKArgs<T> a) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, g = lane & 3;
  const bool isv = lane >= 32;
  const unsigned nk = (unsigned)a.tokens * (unsigned)a.hkv;
  const unsigned idx = blockIdx.x * 8u + (unsigned)((lane >> 2) & 7);
  if (blockIdx.x * 8u >= nk)
    return; // wave-uniform
  // Pairs past the end run on the last pair's data (the exchanges need every lane) and
  // write nothing.
  const bool live = idx < nk; // quad-uniform, and equal in the K and V quads of a pair
  const unsigned ci = live ? idx : nk - 1u;
  const int t = (int)(ci / (unsigned)a.hkv), h = (int)(ci % (unsigned)a.hkv);
  const PosState ps = fetch_state(a.pos, t);
  Act32<T> xv;
  xv.load((isv ? a.v : a.k) + (size_t)ci * D + 32 * g);
  bool ok;
  const int pos = resolve_position(a.pos, ps, t, a.cap, a.first, FMT > PADRA_KV_BF16, ok);
  const bool write = live && ok && pos >= 0 && t >= a.first; // pair-uniform
  if (live && !(ok && pos >= 0) && g == 0 && !isv)
    raise_bad(a.bad);
  const long long seq = a.pos.mode == PADRA_POS_DECODE ? t : 0;
  const long long slot = seq * a.seq_stride + (write ? pos % a.cap : 0);
  if constexpr (FMT == PADRA_KV_BF16) {
    if (!write)
      return;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      w[i] = pack2(xv.get(2 * i), xv.get(2 * i + 1));
    store32_bf16(static_cast<uint16_t *>(isv ? a.vc : a.kc) + slot * (a.hkv * D) + h * D + 32 * g,
                 w);
  } else {
    float x[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
      x[i] = xv.get(i);
    // Quads that write nothing still take part in the exchanges with zeros.
    if (!write) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        x[i] = 0.f;
    }
    if (__ballot(write) == 0)
      return; // wave-uniform
    encode_quad_rt<FMT>(a, x, slot, h, g, isv, write);
  }
}

// ---- commit: encoded chunk rows -> ring slots ----------------------------------------
//
// Row r of the chunk (r >= first) goes to slot (base + r) % cap; one wave per row, every
// tensor of the format copied as 16-byte words (rows are 16-byte multiples except the q8
// scale pairs, copied as 8-byte words).
struct CommitArgs {
  const uint8_t *src[3];
  uint8_t *dst[3];
  int row_bytes[3];
  int tensors, tokens, cap, first, strict;
  PosSrc pos;
  int *bad;
};

__global__ __launch_bounds__(64) void k_kv_commit(CommitArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = a.first + (int)blockIdx.x;
  if (r >= a.tokens)
    return;
  bool ok;
  const int pos = resolve_position(a.pos, r, a.cap, a.first, a.strict != 0, ok);
  if (!ok || pos < 0) {
    if (lane == 0)
      raise_bad(a.bad);
    return;
  }
  const long long slot = pos % a.cap;
  for (int tn = 0; tn < a.tensors; ++tn) {
    const int rb = a.row_bytes[tn];
    const uint8_t *s = a.src[tn] + (long long)r * rb;
    uint8_t *d = a.dst[tn] + slot * rb;
    if ((rb & 15) == 0) {
      for (int w = lane; w < rb / 16; w += 64)
        st_nt(reinterpret_cast<uint4 *>(d) + w, ld_nt(reinterpret_cast<const uint4 *>(s) + w));
    } else {
      for (int w = lane; w < rb / 8; w += 64)
        st_nt(reinterpret_cast<uint2 *>(d) + w, ld_nt(reinterpret_cast<const uint2 *>(s) + w));
    }
  }
}

// ---- q8_0 rows -> BF16 ----------------------------------------------------------------
//
// q8_native::Dequantize (kv_q8_native.cuh:366-390): out = bf16(code * float(d)); a -128
// code or a negative / non-finite scale raises the flag (the value is still written).
template <class O>
__global__ __launch_bounds__(256) void k_q8_0_dequant(const uint8_t *rk, const uint8_t *rv,
                                                      O *ok_out, O *ov_out, long long rows,
                                                      int features, int *bad,
                                                      PosSrc prefix, int cap) {
  const int nd = features / 32, rb = ((2 * nd + features) + 15) / 16 * 16;
  if (prefix.prefill) {
    // q8_native::DequantizePrefix (kv_q8_native.cuh:391-413): the ring's valid rows,
    // min(base, cap), after ValidPrefillState and the ring-capacity check.
    const padra_PrefillState st = load_state(prefix.prefill);
    if (!prefill_valid(st, prefix.tokens, st.capacity, prefix.epoch, prefix.maximum) ||
        (cap != st.capacity && cap != min(1024, st.capacity))) {
      if (blockIdx.x == 0 && threadIdx.x == 0)
        raise_bad(bad);
      return;
    }
    rows = min(st.base, cap);
  }
  const long long groups = rows * (features / 8); // 8 codes per thread-step
  for (long long g = blockIdx.x * (long long)blockDim.x + threadIdx.x; g < 2 * groups;
       g += (long long)gridDim.x * blockDim.x) {
    const bool isv = g >= groups;
    const long long gg = isv ? g - groups : g;
    const long long row = gg / (features / 8);
    const int c0 = (int)(gg % (features / 8)) * 8;
    const uint8_t *rowp = (isv ? rv : rk) + row * rb;
    const uint16_t dbits = reinterpret_cast<const uint16_t *>(rowp)[c0 / 32];
    const float d = __half2float(__ushort_as_half(dbits));
    const uint2 codes = *reinterpret_cast<const uint2 *>(rowp + 2 * nd + c0);
    bool flag = (c0 % 32 == 0) && (!isfinite(d) || d < 0.f);
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t src = p < 2 ? codes.x : codes.y;
      const int8_t c0v = (int8_t)((src >> (16 * (p & 1))) & 0xff);
      const int8_t c1v = (int8_t)((src >> (16 * (p & 1) + 8)) & 0xff);
      flag |= c0v == -128 || c1v == -128;
      w[p] = pack2((float)c0v * d, (float)c1v * d);
    }
    if (flag)
      raise_bad(bad);
    O *dst = (isv ? ov_out : ok_out) + row * features + c0;
    ActIO<O>::store8(dst, w);
  }
}

// ---- Hadamard row rotation -----------------------------------------------------------
//
// q8_native::RotateRows (kv_q8_native.cuh:391-412): each 128-wide row rotated with the K
// transform (VALUE false) or the two 64-point V transforms (VALUE true), output B(x).
// Four lanes per row (lane g: features 32g .. 32g+31), 16 rows per wave.
template <class T, bool VALUE>
__global__ __launch_bounds__(64) void k_rotate_rows(T *data, long long rows, int *bad) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, g = lane & 3;
  const long long r = blockIdx.x * 16ll + (lane >> 2);
  if (blockIdx.x * 16ll >= rows)
    return; // wave-uniform
  // rows past the end rotate the last row's values (the exchanges need every lane) and
  // store nothing
  const bool live = r < rows;
  T *p = data + (live ? r : rows - 1) * D + 32 * g;
  Act32<T> xv;
  xv.load(p);
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    x[i] = xv.get(i);
  hadamard32(x);        // feature bits 0..4
  hadamard_quad<1>(x, g); // bit 5
  if constexpr (!VALUE) {
    hadamard_quad<2>(x, g); // bit 6
#pragma unroll
    for (int i = 0; i < 32; ++i)
      x[i] *= .08838834764831845f;
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      x[i] *= .125f;
  }
  bool fine = true;
  uint32_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    fine = fine && isfinite(x[2 * i]) && isfinite(x[2 * i + 1]);
    w[i] = pack2(x[2 * i], x[2 * i + 1]);
  }
  if (!live)
    return;
  if (!fine)
    raise_bad(bad);
  store32<T>(p, w);
}

template <class F> int with_kv_format(int fmt, F &&f) {
  switch (fmt) {
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

int row_bytes_q8_0(int features) { return ((2 * (features / 32) + features) + 15) / 16 * 16; }

// ---- local-ring checkpoint capture -------------------------------------------------
//
// kv_checkpoint::CaptureEncoded / CaptureLocal (kv_checkpoint.cuh:27-89): a 1024-row snapshot
// of a local ring taken before the chunk's suffix commit, copying encoded bits only.  Slot
// s holds position p = anchor-1 - ((anchor-1 - s + 1024) % 1024): the chunk's row p - base
// when p >= base, the old ring's slot s when 0 <= p < base, zeros before position 0.  Up to
// three planes (K, V, and the q8 scale pairs); every row is a multiple of 16 bytes, so each
// thread moves one 16-byte word.
struct CheckpointArgs {
  const uint8_t *old_rows[3], *current_rows[3];
  uint8_t *saved[3];
  int row_bytes[3];
  int planes, tokens, anchor;
  PosSrc pos;
  int *bad;
};

__global__ __launch_bounds__(256) void k_kv_checkpoint(CheckpointArgs a) {
  __shared__ int admitted;
  if (threadIdx.x == 0) {
    const padra_PrefillState st = load_state(a.pos.prefill);
    const bool ok = prefill_valid(st, a.tokens, st.capacity, a.pos.epoch, a.pos.maximum) &&
                    st.capacity >= 1024 && a.anchor > st.base && a.anchor <= st.base + a.tokens;
    // A flag already raised by earlier work stops the capture (kv_checkpoint.cuh:43-44).
    const bool pending = __atomic_load_n(a.bad, __ATOMIC_RELAXED) != 0;
    if (!ok && blockIdx.x == 0)
      raise_bad(a.bad);
    admitted = ok && !pending ? st.base + 1 : 0;
  }
  __syncthreads();
  if (!admitted)
    return; // block-uniform
  const int base = admitted - 1;
  for (int pl = 0; pl < a.planes; ++pl) {
    const int words = a.row_bytes[pl] / 16, n = 1024 * words;
    const uint4 *old = reinterpret_cast<const uint4 *>(a.old_rows[pl]);
    const uint4 *cur = reinterpret_cast<const uint4 *>(a.current_rows[pl]);
    uint4 *saved = reinterpret_cast<uint4 *>(a.saved[pl]);
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
      const int slot = i / words, word = i - slot * words;
      const int position = a.anchor - 1 - ((a.anchor - 1 - slot + 1024) % 1024);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (position >= base)
        v = ld_nt(cur + (size_t)(position - base) * words + word);
      else if (position >= 0)
        v = ld_nt(old + i);
      st_nt(saved + i, v);
    }
  }
}

} // namespace

extern "C" int padra_KVStore(void *stream, const void *k, const void *v,
                             const padra_Positions *pos, int tokens, int kv_heads, int head_dim,
                             const padra_KVCache *kv, int *bad, int act) {
  if (!k || !v || !kv || !bad || kv_heads < 1 || !aligned16(k) || !aligned16(v) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  if (head_dim != 128)
    return PADRA_UNSUPPORTED;
  int st = check_positions(pos, tokens);
  if (st)
    return st;
  if (!kv->k || !kv->v || kv->cap < 1 || kv->first < 0 || kv->first >= tokens ||
      kv->seq_stride < 0 || kv->format < PADRA_KV_BF16 || kv->format > PADRA_KV_Q8_0_NOROT ||
      (kv->format == PADRA_KV_Q8 && !kv->scales) ||
      (pos->mode == PADRA_POS_DECODE && tokens > 1 && kv->seq_stride < kv->cap) ||
      (pos->mode != PADRA_POS_DECODE && tokens - kv->first > kv->cap))
    return PADRA_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const long long grid = ((long long)tokens * kv_heads + 7) / 8;
  auto launch = [&](auto tag) -> int {
    using T = decltype(tag);
    QKArgs<T> a{};
    a.k = const_cast<T *>(static_cast<const T *>(k));
    a.v = static_cast<const T *>(v);
    a.tokens = tokens;
    a.hq = 0;
    a.hkv = kv_heads;
    a.pos = pos_src(*pos, tokens);
    a.kc = kv->k;
    a.vc = kv->v;
    a.scales = kv->scales;
    a.cap = kv->cap;
    a.first = kv->first;
    a.seq_stride = kv->seq_stride;
    a.bad = bad;
    return with_kv_format(kv->format, [&](auto fmt) -> int {
      hipLaunchKernelGGL((k_kv_store<T, fmt.value>), dim3((unsigned)grid), dim3(64), 0, s, a);
      return launched("KVStore");
    });
  };
  return act == PADRA_ACT_BF16 ? launch(uint16_t{}) : launch(float{});
}

extern "C" int padra_KVCommit(void *stream, const padra_KVCache *chunk, const padra_KVCache *ring,
                              const padra_Positions *pos, int tokens, int kv_heads, int *bad) {
  if (!chunk || !ring || !bad || kv_heads < 1 || chunk->format != ring->format ||
      !chunk->k || !chunk->v || !ring->k || !ring->v || ring->cap < 1 || ring->first < 0 ||
      ring->first >= tokens || tokens - ring->first > ring->cap)
    return PADRA_INVALID_ARGUMENT;
  if (pos && pos->mode == PADRA_POS_DECODE)
    return PADRA_UNSUPPORTED; // commits are per prefill chunk
  int st = check_positions(pos, tokens);
  if (st)
    return st;
  const int features = kv_heads * 128;
  CommitArgs a{};
  a.tokens = tokens;
  a.cap = ring->cap;
  a.first = ring->first;
  a.strict = ring->format > PADRA_KV_BF16;
  a.pos = pos_src(*pos, tokens);
  a.bad = bad;
  a.src[0] = static_cast<const uint8_t *>(chunk->k);
  a.src[1] = static_cast<const uint8_t *>(chunk->v);
  a.dst[0] = static_cast<uint8_t *>(ring->k);
  a.dst[1] = static_cast<uint8_t *>(ring->v);
  a.tensors = 2;
  switch (ring->format) {
  case PADRA_KV_BF16:
    a.row_bytes[0] = a.row_bytes[1] = 2 * features;
    break;
  case PADRA_KV_Q8:
    if (!chunk->scales || !ring->scales)
      return PADRA_INVALID_ARGUMENT;
    a.row_bytes[0] = a.row_bytes[1] = features;
    a.src[2] = static_cast<const uint8_t *>(chunk->scales);
    a.dst[2] = static_cast<uint8_t *>(ring->scales);
    a.row_bytes[2] = 8 * kv_heads;
    a.tensors = 3;
    break;
  default:
    a.row_bytes[0] = a.row_bytes[1] = row_bytes_q8_0(features);
    break;
  }
  for (int t = 0; t < a.tensors; ++t)
    if (!aligned16(a.src[t]) || !aligned16(a.dst[t]))
      return PADRA_INVALID_ARGUMENT;
  hipLaunchKernelGGL(k_kv_commit, dim3(tokens - ring->first), dim3(64), 0,
                     static_cast<hipStream_t>(stream), a);
  return launched("KVCommit");
}

extern "C" int padra_KvQ8_0Dequantize(void *stream, const void *rows_k, const void *rows_v,
                                      void *out_k, void *out_v, long long rows, int kv_heads,
                                      int *bad, int act) {
  if (!rows_k || !rows_v || !out_k || !out_v || !bad || rows < 1 || kv_heads < 1 ||
      !aligned16(rows_k) || !aligned16(rows_v) || !aligned16(out_k) || !aligned16(out_v) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  const int features = kv_heads * 128;
  const long long work = 2 * rows * (features / 8);
  const unsigned grid = (unsigned)std::min<long long>((work + 255) / 256, 4096);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const PosSrc none{};
  if (act == PADRA_ACT_BF16)
    hipLaunchKernelGGL((k_q8_0_dequant<uint16_t>), dim3(grid), dim3(256), 0, s,
                       static_cast<const uint8_t *>(rows_k), static_cast<const uint8_t *>(rows_v),
                       static_cast<uint16_t *>(out_k), static_cast<uint16_t *>(out_v), rows,
                       features, bad, none, 0);
  else
    hipLaunchKernelGGL((k_q8_0_dequant<float>), dim3(grid), dim3(256), 0, s,
                       static_cast<const uint8_t *>(rows_k), static_cast<const uint8_t *>(rows_v),
                       static_cast<float *>(out_k), static_cast<float *>(out_v), rows, features,
                       bad, none, 0);
  return launched("KvQ8_0Dequantize");
}

extern "C" int padra_KvQ8_0DequantizePrefix(void *stream, const void *rows_k, const void *rows_v,
                                            void *out_k, void *out_v,
                                            const padra_Positions *prefill, int tokens, int cap,
                                            int kv_heads, int *bad) {
  if (!rows_k || !rows_v || !out_k || !out_v || !bad || !prefill ||
      prefill->mode != PADRA_POS_PREFILL || !prefill->prefill || tokens < 1 || tokens > 2048 ||
      cap < 1 || cap > 131072 || kv_heads < 1 || !aligned16(rows_k) || !aligned16(rows_v) ||
      !aligned16(out_k) || !aligned16(out_v))
    return PADRA_INVALID_ARGUMENT;
  const int features = kv_heads * 128;
  const long long work = 2ll * cap * (features / 8);
  const unsigned grid = (unsigned)std::min<long long>((work + 255) / 256, 4096);
  hipLaunchKernelGGL((k_q8_0_dequant<uint16_t>), dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(rows_k),
                     static_cast<const uint8_t *>(rows_v), static_cast<uint16_t *>(out_k),
                     static_cast<uint16_t *>(out_v), (long long)cap, features, bad,
                     pos_src(*prefill, tokens), cap);
  return launched("KvQ8_0DequantizePrefix");
}

extern "C" int padra_RotateRows(void *stream, void *data, long long rows, int value, int *bad,
                                int act) {
  if (!data || !bad || rows < 1 || !aligned16(data) ||
      (act != PADRA_ACT_BF16 && act != PADRA_ACT_F32))
    return PADRA_INVALID_ARGUMENT;
  const unsigned grid = (unsigned)((rows + 15) / 16);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == PADRA_ACT_BF16) {
    if (value)
      hipLaunchKernelGGL((k_rotate_rows<uint16_t, true>), dim3(grid), dim3(64), 0, s,
                         static_cast<uint16_t *>(data), rows, bad);
    else
      hipLaunchKernelGGL((k_rotate_rows<uint16_t, false>), dim3(grid), dim3(64), 0, s,
                         static_cast<uint16_t *>(data), rows, bad);
  } else {
    if (value)
      hipLaunchKernelGGL((k_rotate_rows<float, true>), dim3(grid), dim3(64), 0, s,
                         static_cast<float *>(data), rows, bad);
    else
      hipLaunchKernelGGL((k_rotate_rows<float, false>), dim3(grid), dim3(64), 0, s,
                         static_cast<float *>(data), rows, bad);
  }
  return launched("RotateRows");
}

extern "C" int padra_KVCheckpointCapture(void *stream, const padra_KVCache *ring,
                                         const padra_KVCache *chunk, const padra_KVCache *saved,
                                         const padra_Positions *prefill, int tokens, int anchor,
                                         int kv_heads, int *bad) {
  if (!ring || !chunk || !saved || !prefill || !bad || kv_heads < 1 ||
      prefill->mode != PADRA_POS_PREFILL || !prefill->prefill || tokens < 1 || tokens > 2048 ||
      prefill->maximum < 1 || prefill->maximum > 131072 || ring->format != chunk->format ||
      saved->format != ring->format || ring->format < PADRA_KV_BF16 ||
      ring->format > PADRA_KV_Q8_0_NOROT || !ring->k || !ring->v || !chunk->k || !chunk->v ||
      !saved->k || !saved->v)
    return PADRA_INVALID_ARGUMENT;
  const int features = kv_heads * 128;
  CheckpointArgs a{};
  a.tokens = tokens;
  a.anchor = anchor;
  a.pos = pos_src(*prefill, tokens);
  a.bad = bad;
  const void *olds[3] = {ring->k, ring->v, ring->scales};
  const void *curs[3] = {chunk->k, chunk->v, chunk->scales};
  void *outs[3] = {saved->k, saved->v, saved->scales};
  int rb;
  switch (ring->format) {
  case PADRA_KV_BF16:
    rb = 2 * features;
    a.planes = 2;
    break;
  case PADRA_KV_Q8:
    rb = features;
    a.planes = 3;
    if (!ring->scales || !chunk->scales || !saved->scales)
      return PADRA_INVALID_ARGUMENT;
    break;
  default:
    rb = row_bytes_q8_0(features);
    a.planes = 2;
    break;
  }
  for (int pl = 0; pl < a.planes; ++pl) {
    a.old_rows[pl] = static_cast<const uint8_t *>(olds[pl]);
    a.current_rows[pl] = static_cast<const uint8_t *>(curs[pl]);
    a.saved[pl] = static_cast<uint8_t *>(outs[pl]);
    a.row_bytes[pl] = pl == 2 ? 8 * kv_heads : rb;
    if (a.row_bytes[pl] % 16 || !aligned16(olds[pl]) || !aligned16(curs[pl]) ||
        !aligned16(outs[pl]))
      return PADRA_INVALID_ARGUMENT;
    // the snapshot may not alias any source plane (kv_checkpoint.cuh:37-38)
    for (int q = 0; q < 3; ++q)
      if (outs[pl] && (outs[pl] == olds[q] || outs[pl] == curs[q]))
        return PADRA_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_kv_checkpoint, dim3(128), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return launched("KVCheckpointCapture");
}
