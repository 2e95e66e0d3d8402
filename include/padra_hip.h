/*
 * padra_hip.h -- C-ABI of the MI355X (gfx950) kernels for Padra's exact-fusions-v1
 * per-token layer path: residual-add + RMSNorm, Q/K RMSNorm + NeoX RoPE + KV-cache
 * store (BF16, q8, q8_0), SwiGLU at the expert boundary and the embedding gather.
 *
 * The reference launches these as __global__ functions from RunCudaInferenceCore
 * (/root/reference/src/cuda/inference.cu:2988-3166 decode, :3421-3950 prefill); it
 * has no FFI of its own.  Each entry point below replaces one reference kernel family
 * (cited per function) with the same arithmetic, the same KV-cache byte layout
 * (/root/reference/docs/kv-cache.md, src/runtime/kv_cache_layout.h) and the same two
 * error channels:
 *   - a host-checkable shape/pointer problem returns a nonzero status and launches
 *     nothing (the reference throws std::runtime_error, prefill_kv_commit.cuh:6-9);
 *   - a device-detected problem (invalid DecodeState/PrefillState, non-finite value,
 *     token id out of range, -128 code) stores 1 to the caller's device int `bad`
 *     and the affected unit writes nothing (reference: atomicExch(bad, 1)).
 *
 * Conventions: every pointer except `stream` and the descriptor structs is a device
 * pointer owned by the caller.  Nothing here allocates, frees or synchronizes; all
 * work is ordered on `stream` (a hipStream_t, NULL = default stream) and may be
 * captured into a HIP graph: positions are read on the device when a state pointer
 * is given, so replays at new positions need no host update.
 * Activations (x, residual, normalized, q, k, v, gate, up) are BF16 bit patterns
 * (uint16_t) unless a function takes `act`; with act = PADRA_ACT_F32 they are fp32
 * words holding BF16-exact values, the reference's own buffer convention
 * (inference.cu:52-54).  16-byte alignment is required for every row base.
 */
#ifndef PADRA_HIP_H
#define PADRA_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, numbered as mellum16::StatusCode (include/mellum16/status.h:11-21). */
enum {
  PADRA_OK = 0,
  PADRA_INVALID_ARGUMENT = 1,
  PADRA_UNSUPPORTED = 5,
  PADRA_INTERNAL = 8
};

/* Activation storage. */
enum { PADRA_ACT_BF16 = 0, PADRA_ACT_F32 = 1 };

/* Reduction tree of the row norms (which reference kernel's bits to reproduce):
 * 128 = Norm / NormFP8Exact / NormFP8WideExact (inference.cu:188-214), 128 threads,
 *       thread t sums elements t, t+128, ...;
 * 256 = ResidualPostNormWideExact (residual_norm_wide_exact.cuh:6-80), 256 threads. */
enum { PADRA_TREE_128 = 128, PADRA_TREE_256 = 256 };

/* KV cache formats (src/runtime/kv_cache_layout.h:6). */
enum {
  PADRA_KV_BF16 = 0,       /* "bf16": K [cap][F] bf16, V [cap][F] bf16 */
  PADRA_KV_Q8 = 1,         /* "q8_token_head128_f32scale_v1": codes K [cap][F] int8,
                              codes V [cap][F] int8, scales [cap][Hkv] {float k, v} */
  PADRA_KV_Q8_0 = 2,       /* "q8_0_token512_block32_f16scale_rot_k128_v64_v2": K and V
                              [cap] rows of {fp16 d[F/32]; int8 qs[F]} (544 B for F=512) */
  PADRA_KV_Q8_0_NOROT = 3  /* the same row layout without the Hadamard rotation */
};

/* Device control state, byte-identical to the reference's structs. */
typedef struct padra_DecodeState { /* decode_control.cuh:3-6 */
  int32_t token, position, capacity, remaining, global_valid, local_valid, eos, stopped;
} padra_DecodeState;
typedef struct padra_PrefillState { /* src/runtime/prefill_state.h:8-11 */
  int32_t base, prompt_offset, tokens, capacity, committed;
  uint32_t binding_epoch, request_epoch, valid;
} padra_PrefillState;
typedef struct padra_Q8KVScalePair { float k, v; } padra_Q8KVScalePair; /* kv_cache_layout.h:48-51 */

/* Where token t's position comes from. */
enum {
  PADRA_POS_BASE = 0,     /* position = base + t (host-known chunk base; QKNormRope `position`) */
  PADRA_POS_PREFILL = 1,  /* position = prefill->base + t after ValidPrefillState
                             (prefill_state.h:16-24) with tokens = chunk rows */
  PADRA_POS_DECODE = 2    /* one token per sequence: position = decode[t].position after
                             DecodeReadyAtLimit (context_admission.cuh:5-11) */
};
typedef struct padra_Positions {
  int32_t mode;
  int32_t base;                        /* PADRA_POS_BASE */
  const padra_PrefillState *prefill;   /* device, PADRA_POS_PREFILL */
  const padra_DecodeState *decode;     /* device array [tokens], PADRA_POS_DECODE */
  int32_t maximum;                     /* context limit for state validation, <= 131072 */
  int32_t vocab;                       /* DecodeState token bound (reference: 98304) */
  uint32_t binding_epoch;              /* expected PrefillState.binding_epoch (reference: 1) */
} padra_Positions;

/* A KV cache binding for one layer (KVCacheView, kv_cache_layout.h:42-47). */
typedef struct padra_KVCache {
  int32_t format;        /* PADRA_KV_* */
  void *k, *v;           /* device */
  void *scales;          /* PADRA_KV_Q8 only */
  int32_t cap;           /* ring rows: capacity (global layer) or min(1024, capacity) (local) */
  int32_t first;         /* chunk rows before `first` are not stored: max(0, tokens-cap) for a
                            local ring narrower than the chunk, else 0 */
  int64_t seq_stride;    /* rows between consecutive sequences' caches (PADRA_POS_DECODE with
                            several sequences); 0 for one sequence */
} padra_KVCache;

/* ---- residual + RMSNorm / RMSNorm -------------------------------------------------
 * Replaces ResidualPostNormWideExact (residual_norm_wide_exact.cuh:6-80),
 * ResidualPostNormBF16 (residual_norm_bf16.cuh:3-40) and the prefill pair Add + Norm
 * (inference.cu:475-481, :188-214) fused in one pass:
 *   x[r][i] <- B(x + residual);  normalized[r][i] <- B(B(x*inv) * gamma[i]),
 *   inv = 1/sqrt(S/H + eps), S the compensated sum of squares in `tree` order.
 * residual may be NULL: then x is read only (Norm, and the norm half of NormFP8Exact /
 * NormFP8WideExact, norm_fp8_exact.cuh:6-45).  statistics (nullable, device float
 * [rows][2]) receives {variance, inv}.  gamma: BF16 [hidden].  hidden % tree == 0,
 * hidden / tree <= 36. */
int padra_ResidualPostNorm(void *stream, void *x, const void *residual, void *normalized,
                           const uint16_t *gamma, int rows, int hidden, float eps, int tree,
                           float *statistics, int *bad, int act);

/* padra_KVCheckpointCapture: kv_checkpoint::CaptureLocal / CaptureEncoded
 * (kv_checkpoint.cuh:27-89).  Before a chunk's suffix commit into a 1024-row local ring,
 * copies the ring as it will read at `anchor` into the snapshot `saved` (1024 rows per
 * plane, the ring's byte layout; encoded bits are copied, never decoded): slot s holds
 * position p = anchor-1 - ((anchor-1 - s + 1024) % 1024), taken from the chunk's row
 * p - base (chunk rows [tokens]) when p >= base, from the old ring's slot s when
 * 0 <= p < base, and zero before position 0.  Planes: K and V, plus the scale pairs for q8
 * (the reference's single CaptureEncoded buffer is saved->k, then saved->v at +1024 rows,
 * then saved->scales).  The capture runs only for a valid PrefillState (tokens rows,
 * prefill->binding_epoch; the reference passes 1) with capacity >= 1024 and
 * base < anchor <= base + tokens; otherwise *bad is raised.  If *bad is already set
 * nothing is copied.  ring, chunk and saved share one format; saved aliases no source. */
int padra_KVCheckpointCapture(void *stream, const padra_KVCache *ring,
                              const padra_KVCache *chunk, const padra_KVCache *saved,
                              const padra_Positions *prefill, int tokens, int anchor,
                              int kv_heads, int *bad);
/* padra_NormFP8: NormFP8Exact (norm_fp8_exact.cuh:6-62) and NormFP8WideExact
 * (norm_fp8_wide_exact.cuh:7-67), which give the same bytes: the 128-thread RMSNorm of each
 * row of x [rows][hidden] into normalized, plus its E4M3 encoding packed [rows][hidden]
 * (u8) with scales[row] = max|y|/448 (1 for an all-zero row), codes through
 * fp8_exact_reciprocal::Encode (fp8_exact_reciprocal.cuh:12-21).  statistics (2 floats,
 * may be NULL) receives {variance, inv} of row 0 only, as the reference writes it.  A
 * non-finite normalized value raises *bad; the row is still written.  hidden is a multiple
 * of 128 in {1024, 1152, 2048, 2304, 4096, 4608}; x, normalized, gamma and packed are
 * 16-byte aligned.  act: PADRA_ACT_BF16 or PADRA_ACT_F32 for x and normalized. */
int padra_NormFP8(void *stream, const void *x, void *normalized, const uint16_t *gamma,
                  uint8_t *packed, float *scales, int rows, int hidden, float eps,
                  float *statistics, int *bad, int act);
/* ---- RoPE table (host) --------------------------------------------------------------
 * Replaces RopeTable (inference.cu:764-785): fills the HOST buffer table[positions][D]
 * with BF16 bit patterns of cos (first D/2) and sin (last D/2), theta a parameter;
 * yarn != 0 selects the reference's global-layer ramp (factor, original_context).
 * The caller uploads it (the reference copies its table host-to-device once). */
int padra_RopeTable(uint16_t *table, int positions, int head_dim, float theta, int yarn,
                    float factor, int original_context);

/* ---- Q/K RMSNorm + RoPE (+ KV store) ------------------------------------------------
 * Replaces QKNormRope (qknorm_rope.cuh:4-50), QKNormRopePair64 (qknorm_rope_pair64.cuh:
 * 3-83), QKNormRopeControlled (decode_control.cuh:80-126) and, when kv != NULL,
 * QKNormRopeStoreControlled (qk_rope_store_exact.cuh:4-49) together with the cache
 * writers that follow it: StorePrefillControlled / Store (prefill_control.cuh:24-38,
 * inference.cu:248-256), kv_q8::Encode + Commit (kv_q8.cuh:28-98) and
 * q8_native::EncodeKV + Commit (kv_q8_native.cuh:52-101, :440-463).
 * q [T][Hq][D] and k [T][Hkv][D] are normalized and rotated in place (qn, kn: BF16 [D]);
 * table: BF16 [table_rows][D] from padra_RopeTable.  With kv: for every token t >= first
 * the rotated K row and the V row (v: [T][Hkv][D]) are stored at cache slot
 * position % cap in kv->format.  D must be 128 (the reference's block shape). */
int padra_QKNormRopeStore(void *stream, void *q, void *k, const void *v, const uint16_t *qn,
                          const uint16_t *kn, const uint16_t *table, int table_rows,
                          const padra_Positions *pos, int tokens, int q_heads, int kv_heads,
                          int head_dim, float eps, const padra_KVCache *kv, int *bad, int act);

/* ---- fused per-token chain ----------------------------------------------------------
 * One launch of padra_ResidualPostNorm over `tokens` rows and padra_QKNormRopeStore over
 * the same tokens (the two have no data dependence; exact-fusions-v1 runs them as
 * separate kernels: the prefill Add + Norm, inference.cu:475-481, 188-214, and
 * QKNormRopeStoreControlled, qk_rope_store_exact.cuh:4-49).  Arguments mean what they mean
 * there, act included (x, residual, normalized, q, k, v all of that type); results are
 * bit-identical to the two calls. */
int padra_ResidualNormQKRopeStore(void *stream, void *x, const void *residual,
                                  void *normalized, const uint16_t *gamma, int hidden,
                                  int tree, float *statistics, void *q, void *k,
                                  const void *v, const uint16_t *qn, const uint16_t *kn,
                                  const uint16_t *table, int table_rows,
                                  const padra_Positions *pos, int tokens, int q_heads,
                                  int kv_heads, int head_dim, float eps,
                                  const padra_KVCache *kv, int *bad, int act);
/* padra_EmbedResidualNormQKRopeStore: padra_Embed (BF16 output into x, same positions)
 * followed by padra_ResidualNormQKRopeStore, in one launch: the norm rows read row t of x
 * from embed[token_t] instead of from x.  The layer-0 decode step, EmbedControlled
 * (decode_control.cuh:68-79) then the residual norm and QKNormRopeStoreControlled;
 * exact-fusions-v1 runs them as separate kernels.  Results, including x and the flag for
 * an invalid token (that row reads x as it was), are bit-identical to the two calls. */
int padra_EmbedResidualNormQKRopeStore(void *stream, const uint16_t *embed, int vocab,
                                       const int32_t *ids, void *x, const void *residual,
                                       void *normalized, const uint16_t *gamma, int hidden,
                                       int tree, float *statistics, void *q, void *k,
                                       const void *v, const uint16_t *qn, const uint16_t *kn,
                                       const uint16_t *table, int table_rows,
                                       const padra_Positions *pos, int tokens, int q_heads,
                                       int kv_heads, int head_dim, float eps,
                                       const padra_KVCache *kv, int *bad);

/* ---- KV store, commit, decode ---------------------------------------------------------
 * padra_KVStore: the cache writers without the Q/K norm -- StorePrefillControlled /
 * Store / StoreControlled (prefill_control.cuh:24-38, inference.cu:248-256,
 * decode_control.cuh:213-224), kv_q8::Encode (kv_q8.cuh:28-74) and q8_native::EncodeKV
 * (kv_q8_native.cuh:52-101).  k and v [T][Hkv][128] (k already normalized and rotated)
 * go to slot position % kv->cap in kv->format; q8_0 applies its Hadamard rotation.  With
 * kv->cap = T and positions 0.. this fills an encoded chunk buffer, as the reference's
 * prefill encode does before attention. */
int padra_KVStore(void *stream, const void *k, const void *v, const padra_Positions *pos,
                  int tokens, int kv_heads, int head_dim, const padra_KVCache *kv, int *bad,
                  int act);
/* padra_KVCommit: kv_q8::Commit (kv_q8.cuh:75-98) and q8_native::Commit
 * (kv_q8_native.cuh:440-463), and the BF16 chunk commit: rows r >= ring->first of the
 * encoded chunk `chunk` (row r at index r, same format) are copied to ring slot
 * position(r) % ring->cap.  pos: PADRA_POS_BASE or PADRA_POS_PREFILL. */
int padra_KVCommit(void *stream, const padra_KVCache *chunk, const padra_KVCache *ring,
                   const padra_Positions *pos, int tokens, int kv_heads, int *bad);
/* padra_KvQ8_0Dequantize: q8_native::Dequantize (kv_q8_native.cuh:366-390): rows of q8_0
 * K and V (544 B each for 4 heads) to [rows][Hkv*128] bf16(code * d); a -128 code or a
 * negative / non-finite scale raises the flag. */
int padra_KvQ8_0Dequantize(void *stream, const void *rows_k, const void *rows_v, void *out_k,
                           void *out_v, long long rows, int kv_heads, int *bad, int act);
/* padra_KvQ8_0DequantizePrefix: q8_native::DequantizePrefix (kv_q8_native.cuh:391-413):
 * decodes the ring's first min(prefill->base, cap) rows to BF16, the row count read on
 * the device after ValidPrefillState (tokens = chunk rows) and the ring check (cap is the
 * capacity or min(1024, capacity)).  out_k / out_v hold cap rows. */
int padra_KvQ8_0DequantizePrefix(void *stream, const void *rows_k, const void *rows_v,
                                 void *out_k, void *out_v, const padra_Positions *prefill,
                                 int tokens, int cap, int kv_heads, int *bad);
/* padra_RotateRows: q8_native::RotateRows (kv_q8_native.cuh:391-412): rotates `rows`
 * 128-wide rows in place with the K transform (value = 0) or the two 64-point V
 * transforms (value = 1), output rounded to BF16. */
int padra_RotateRows(void *stream, void *data, long long rows, int value, int *bad, int act);

/* ---- SwiGLU ---------------------------------------------------------------------------
 * padra_SiluTableBuild: exl3_silu_lut::Build (exl3_silu_lut.cuh:9-14): table[65536] of the
 * BF16 bits of B(g / (1 + RN32(exp64(-g)))) per BF16 gate g.
 * padra_SwiGLU: exl3_silu_lut::Activate (exl3_silu_lut.cuh:15-31) and Activate
 * (inference.cu:575-579): out[i] = B(silu(gate[i]) * up[i]) over `count` elements
 * (count % 8 == 0; out may alias gate, as in the reference).  A non-finite gate or up
 * raises the flag and leaves the gate value in out. */
int padra_SiluTableBuild(void *stream, uint16_t *table);
int padra_SwiGLU(void *stream, const void *gate, const void *up, void *out, long long count,
                 const uint16_t *table, int *bad, int act);

/* ---- embedding gather ------------------------------------------------------------------
 * Embed / EmbedPrefillControlled / EmbedControlled (inference.cu:181-187,
 * prefill_control.cuh:3-22, decode_control.cuh:68-79): out[t][:] = table[token_t][:] for a
 * BF16 table [vocab][hidden].  The token is ids[t] (src NULL or PADRA_POS_BASE), the prompt
 * id ids[prompt_offset + t] (PADRA_POS_PREFILL), or decode[t].token (PADRA_POS_DECODE).  An
 * invalid state or a token outside [0, vocab) raises the flag and writes nothing. */
int padra_Embed(void *stream, const uint16_t *table, int vocab, int hidden, const int32_t *ids,
                const padra_Positions *src, int tokens, void *out, int *bad, int act);

/* padra_QuantizeFP8: QuantizeFP8 (prefill.cuh:46-66), the E4M3 row encoding of an
 * activation (the attention output before the O projection): per row of x [rows][cols],
 * scales[row] = max|x|/448 (1 for a zero row) and packed[row][c] = E4M3 of the correctly
 * rounded x/scale (saturating).  A non-finite value raises *bad (the row is still
 * written).  cols a multiple of 8; x 16-byte aligned, packed 8-byte aligned. */
int padra_QuantizeFP8(void *stream, const void *x, uint8_t *packed, float *scales, int rows,
                      int cols, int *bad, int act);
/* padra_Combine: Combine (inference.cu:580-590) and exl3_packed_activations::Combine
 * (expert_exl3_prefill_packed_activations.cuh:86-102).  For each row t and column i of
 * x [rows][hidden]: c = 0; for e = 0..experts-1: c = B(c + B(down[t][e][i] * weights[t][e]));
 * x = residual ? B(x + c) : c.  down is [rows][experts][hidden] in the activation type,
 * weights [rows][experts] fp32 routing weights.  A non-finite result raises *bad and is
 * still written.  experts must be 8; hidden a multiple of 8; x, down 16-byte aligned. */
int padra_Combine(void *stream, void *x, const void *down, const float *weights, int rows,
                  int hidden, int experts, int residual, int *bad, int act);
/* padra_CombineNorm: combine_norm_exact::CombineNorm (combine_norm_exact.cuh:7-72), one row
 * per row of x: the residual combine above, then the 128-thread RMSNorm of the new x into
 * normalized and, when packed != NULL, its E4M3 encoding as padra_NormFP8 writes it
 * (packed [rows][hidden], scales [rows]).  statistics (2 floats, may be NULL) receives
 * {variance, inv} of row 0.  Non-finite combined or normalized values raise *bad.  hidden
 * in {1024, 1152, 2048, 2304, 4096, 4608}; experts must be 8. */
int padra_CombineNorm(void *stream, void *x, const void *down, const float *weights,
                      void *normalized, const uint16_t *gamma, uint8_t *packed, float *scales,
                      int rows, int hidden, int experts, float eps, float *statistics, int *bad,
                      int act);
/* padra_DecodeAttention: decode attention, one token per sequence, for q_heads/kv_heads in
 * {1, 2, 4, 8} query heads per KV head.
 *  - BF16 cache: gqa8_fragment_validation::SplitBF16 (attention_gqa8_fragment_validation.cuh:
 *    79-214) and attention_perhead_exact::Merge (attention_perhead_exact.cuh:7-38).
 *  - q8 cache: gqa8_q8_attention::SplitBF16 (attention_gqa8_q8.cuh:112-277), its tiles
 *    decoded by kv_q8::Decode, with the per-head merge above.
 *  - q8_0 cache (rotated v2, 4 KV heads): q8_native::EncodeQuery, Split and Merge
 *    (kv_q8_native.cuh:103-148, 198-363); a local ring must have cap 1024.
 * q [seqs][q_heads][128] (BF16-exact), out likewise; kv: the cache binding (cap rows per
 * sequence, seq_stride rows apart); pos: PADRA_POS_DECODE states.  local != 0: a local
 * ring (BF16: cap = min(1024, capacity)), else cap must equal capacity.  splits: 1..32
 * split-K partitions, 0 for the reference's count (BF16: min(ceil(cap/32), local ? 16 : 32);
 * q8_0: local ? 16 : 32), -1 for the count tuned on MI355X (padra_DecodeAttentionSplits;
 * the same as 0 for global windows, fewer splits for a local ring with many sequences).
 * A count other than the reference's changes only the order in which the split partials
 * are merged.  scratch: device fp32 workspace of
 * padra_DecodeAttentionScratch(kv->format, seqs, q_heads, padra_DecodeAttentionSplits(...))
 * floats.  A sequence whose
 * state is not admitted raises *bad and writes nothing; non-finite queries, scores or
 * outputs raise *bad.  Results match the reference within the tolerance its tensor-core
 * accumulation order (BF16) and CUDA expf/logf leave. */
int padra_DecodeAttention(void *stream, const void *q, const padra_KVCache *kv, void *out,
                          const padra_Positions *pos, int seqs, int q_heads, int kv_heads,
                          int local, int splits, float *scratch, long long scratch_floats,
                          int *bad, int act);
/* padra_DecodeAttentionFP8: padra_DecodeAttention (BF16 or q8 cache) whose merge also
 * writes the E4M3 encoding of each sequence's output row, as
 * attention_o_wide_exact::MergeQuantize (attention_merge_quantize_wide_exact.cuh:9-66)
 * does after the reference's q8 split (attention_gqa8_q8.cuh:278-300): packed
 * [seqs][q_heads * 128] codes of the correctly rounded quotient out / scale, scales [seqs]
 * = max|out row| / 448 (1 for a zero row); the same bytes padra_QuantizeFP8 writes for out.
 * q_heads <= 32.  A q8_0 cache is PADRA_UNSUPPORTED (its reference merge has no FP8 form). */
int padra_DecodeAttentionFP8(void *stream, const void *q, const padra_KVCache *kv, void *out,
                             uint8_t *packed, float *scales, const padra_Positions *pos,
                             int seqs, int q_heads, int kv_heads, int local, int splits,
                             float *scratch, long long scratch_floats, int *bad, int act);
/* Floats of scratch padra_DecodeAttention needs for a cache format (splits as resolved,
 * 1..32); -1 if invalid. */
long long padra_DecodeAttentionScratch(int format, int seqs, int q_heads, int splits);
/* The split count padra_DecodeAttention runs for these arguments (splits 1..32 as given,
 * 0: the reference's, -1: the MI355X-tuned count); -1 if invalid.  No counterpart in the
 * reference, whose kernels fix their count: callers size the scratch with it. */
int padra_DecodeAttentionSplits(const padra_KVCache *kv, int seqs, int kv_heads, int local,
                                int splits);
/* padra_DecodeAttentionNoAlloc: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): padra_DecodeAttention with the same kernels and results, whose
 * workspace is a fixed device array of PADRA_DECODE_ATTENTION_STATIC_FLOATS floats
 * (18 MiB: 64 sequences x 16 query heads x 32 splits fit) instead of a caller buffer.  It
 * calls no allocator.  The array exists once per GPU and is held until the process ends;
 * its address is looked up on the first call on each device.  A launch that needs more
 * (padra_DecodeAttentionScratch) returns PADRA_INVALID_ARGUMENT with a message on stderr
 * and launches nothing.  Every call on one GPU uses that GPU's one array: calls ordered
 * on one stream are safe, calls that overlap on one GPU (several streams or threads)
 * race. */
#define PADRA_DECODE_ATTENTION_STATIC_FLOATS 4718592
int padra_DecodeAttentionNoAlloc(void *stream, const void *q, const padra_KVCache *kv,
                                 void *out, const padra_Positions *pos, int seqs, int q_heads,
                                 int kv_heads, int local, int splits, int *bad, int act);
/* ---- version / capability ----------------------------------------------------------- */
const char *padra_version(void);

#ifdef __cplusplus
}
#endif
#endif
