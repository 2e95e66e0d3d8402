/*
 * padra_oracle.h -- CPU restatement of Padra's exact-fusions-v1 per-token layer
 * arithmetic (the parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product in
 * padra_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product never links, loads or falls back to it.
 *
 * Every function restates the reference CUDA source in plain C11, operation by
 * operation (same rounding points, same reduction tree), citing the file:line of
 * /root/reference it follows.  Activations cross this interface as BF16 bit
 * patterns (uint16_t), the device I/O format of the product; the reference keeps
 * the same values in fp32 buffers (BF16-exact), which changes no arithmetic.
 *
 * Pinning (what checks each function against something other than itself) is
 * listed per function in tests/test_oracle.py.
 */
#ifndef PADRA_ORACLE_H
#define PADRA_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- A1 numeric primitives ------------------------------------------------ */
float po_bf16_round(float x);           /* B(x): inference.cu:52-54, BHost :742-748 */
uint16_t po_f32_to_bf16(float x);       /* __float2bfloat16_rn */
float po_bf16_to_f32(uint16_t h);
uint16_t po_f32_to_f16(float x);        /* __float2half_rn (RNE, subnormals) */
float po_f16_to_f32(uint16_t h);
void po_accumulate(float value, float *sum, float *error); /* inference.cu:103-109 */
/* Compensated sum of squares of n values with a block of `threads` threads
 * (128: AccurateReduce inference.cu:110-135 / Rms128In256Exact rms_wide_exact.cuh:3-31;
 *  256: ResidualPostNormWideExact residual_norm_wide_exact.cuh:24-63). */
float po_sumsq_tree(const float *v, int n, int threads);
/* variance and 1/sqrt(variance+eps), each step correctly rounded (inference.cu:203-205). */
void po_rms_inv(float sumsq, int n, float eps, float *variance, float *inv);
float po_exp_rn(float x);               /* ExpRN: inference.cu:57-59 */

/* ---- A2 residual + RMSNorm, A3 RMSNorm ------------------------------------ */
/* x <- B(x + r); y <- B(B(x*inv)*gamma).  stats (nullable) gets {variance, inv} per row. */
void po_residual_rmsnorm(uint16_t *x, const uint16_t *residual, uint16_t *y,
                         const uint16_t *gamma, int rows, int hidden, float eps,
                         int threads, float *stats, int *bad);
void po_rmsnorm(const uint16_t *x, uint16_t *y, const uint16_t *gamma, int rows, int hidden,
                float eps, int threads, float *stats, int *bad);

/* ---- A3 FP8 E4M3 row encoding (NormFP8Exact / NormFP8WideExact) ------------- */
/* OCP E4M3 (bias 7, max 448, no infinities, NaN S.1111.111) of x: round to nearest even,
 * finite overflow and infinities saturate to +-448, every NaN -> 0x7f. */
uint8_t po_e4m3(float x);
/* True when q's magnitude bits sit within 4 ulp of an E4M3 rounding midpoint
 * (fp8_exact_reciprocal.cuh:5-11). */
int po_fp8_needs_division(uint32_t magnitude_bits);
/* fp8_exact_reciprocal::Encode (fp8_exact_reciprocal.cuh:12-21): the code of value/scale
 * through the cached reciprocal, with a correctly rounded division near midpoints. */
uint8_t po_fp8_encode(float value, float scale, float inverse);
/* NormFP8Exact (norm_fp8_exact.cuh:6-62; the 256-thread NormFP8WideExact computes the
 * same bytes): per row the 128-thread norm, normalized = y, scales[row] = max|y|/448 (1 for
 * an all-zero row) and packed[row][i] = code of y_i.  stats (2 floats) from row 0 only. */
void po_norm_fp8(const uint16_t *x, uint16_t *normalized, const uint16_t *gamma,
                 uint8_t *packed, float *scales, int rows, int hidden, float eps, float *stats,
                 int *bad);

/* QuantizeFP8 (prefill.cuh:46-66): per row, scale = max|x|/448 (1 for a zero row; fmaxf
 * drops NaN), packed = E4M3 of x / scale (correctly rounded quotient, saturating); a
 * non-finite value raises *bad.  x is fp32 [rows][cols]. */
void po_quantize_fp8(const float *x, uint8_t *packed, float *scales, int rows, int cols,
                     int *bad);

/* Checker for the GPU's rounding of q8_0 codes: the number of floats with bit patterns in
 * [lo, hi) (finite, |x| < 2^23) where (int)(x + copysignf(0.49999997f, x)) differs from
 * (int)roundf(x). */
unsigned long long po_round_away_mismatches(uint64_t lo, uint64_t hi);

/* ---- Expert combine (+ residual) and combine + RMSNorm (+ FP8) ---------------- */
/* Combine (inference.cu:580-590) and exl3_packed_activations::Combine
 * (expert_exl3_prefill_packed_activations.cuh:86-102): per row t and column i,
 * c = 0; for e in 0..experts-1: c = B(c + B(down[t][e][i] * weights[t][e])); then
 * x[t][i] = residual ? B(x + c) : c, a non-finite result raising *bad (still written).
 * weights are fp32 routing weights [rows][experts]. */
void po_combine(uint16_t *x, const uint16_t *down, const float *weights, int rows, int hidden,
                int experts, int residual, int *bad);
/* combine_norm_exact::CombineNorm (combine_norm_exact.cuh:7-72), one row per row of x:
 * the residual combine above, then the 128-thread RMSNorm of the new x into normalized
 * (non-finite v or y raise *bad), and with packed != NULL the FP8 E4M3 encoding
 * (scales[row]).  stats (2 floats) from row 0. */
void po_combine_norm(uint16_t *x, const uint16_t *down, const float *weights,
                     uint16_t *normalized, const uint16_t *gamma, uint8_t *packed,
                     float *scales, int rows, int hidden, int experts, float eps, float *stats,
                     int *bad);

/* ---- A5 RoPE table --------------------------------------------------------- */
/* table[p][i] = B(cos(p*f_i)*scale), table[p][D/2+i] = B(sin(p*f_i)*scale), fp32 values.
 * yarn=0: plain NeoX f_i = 1/theta^(2i/D).  yarn=1: the reference's global-layer ramp
 * (inference.cu:764-785) with factor, original context, beta_fast 32, beta_slow 1. */
void po_rope_table(float *table, int positions, int head_dim, float theta, int yarn,
                   float factor, int original_context);

/* ---- A4 Q/K norm + RoPE (+ A6 BF16 store) ---------------------------------- */
/* One head vector in place: RMSNorm over D then NeoX half-split rotation with the
 * table row (D BF16 values, cos then sin).  qk_rope_store_exact.cuh:27-44,
 * qknorm_rope_pair64.cuh:30-82. */
void po_qk_norm_rope_head(uint16_t *x, const uint16_t *weight, const uint16_t *table_row,
                          int head_dim, float eps, int *bad);
/* q [T][Hq][D], k [T][Hkv][D] in place; positions[t] selects the table row. */
void po_qk_norm_rope(uint16_t *q, uint16_t *k, const uint16_t *qn, const uint16_t *kn,
                     const uint16_t *table, const int *positions, int tokens, int q_heads,
                     int kv_heads, int head_dim, float eps, int *bad);
/* kc[(pos_t % cap)][f] = k[t][f] (and v) for t >= first; prefill_control.cuh:24-38,
 * qk_rope_store_exact.cuh:45-48, prefill_kv_commit.cuh:4-13. */
void po_kv_store_bf16(const uint16_t *k, const uint16_t *v, uint16_t *kc, uint16_t *vc,
                      const int *positions, int tokens, int features, int cap, int first);

/* ---- A7 Q8 KV (q8_token_head128_f32scale_v1) -------------------------------- */
/* kv_q8.cuh:28-74 (Encode) + :75-98 (Commit), written straight to slot pos%cap.
 * scales: [cap][kv_heads] {k,v} pairs (fp32). */
void po_kv_q8_encode(const uint16_t *k, const uint16_t *v, int8_t *codes_k, int8_t *codes_v,
                     float *scales, const int *positions, int tokens, int kv_heads,
                     int head_dim, int cap, int first, int *bad);
int po_kv_q8_decode(int8_t code, float scale, uint16_t *out); /* kv_q8.cuh:15-27 */

/* ---- A8 Q8_0 KV (q8_0_token512_block32_f16scale_rot_k128_v64_v2) ------------ */
void po_hadamard(float *x, int n, float scale); /* kv_q8_native.cuh:22-45, stages bit0..bitlog2(n)-1 */
/* Row layout: uint16 d[F/32] (fp16), int8 qs[F], padded to 16 B (544 B for F=512).
 * rotate=1 is the reference v2 format (K: 128-point, V: 64-point transforms);
 * rotate=0 quantizes the BF16 values directly (no Hadamard). kv_q8_native.cuh:52-101. */
int po_q8_0_row_bytes(int features);
void po_kv_q8_0_encode(const uint16_t *k, const uint16_t *v, uint8_t *rows_k, uint8_t *rows_v,
                       const int *positions, int tokens, int kv_heads, int head_dim, int cap,
                       int first, int rotate, int *bad);
/* bf16(code * fp16 d) for rows [0, rows); kv_q8_native.cuh:366-390. */
void po_kv_q8_0_dequantize(const uint8_t *rows_k, const uint8_t *rows_v, uint16_t *out_k,
                           uint16_t *out_v, int rows, int features, int *bad);

/* ---- A10 SwiGLU -------------------------------------------------------------- */
uint16_t po_silu_bf16(uint16_t gate);   /* exl3_silu_lut.cuh:5-8 */
void po_silu_table(uint16_t *table);    /* 65536 entries, exl3_silu_lut.cuh:9-14 */
/* out = B(s*u), s = silu LUT of the BF16 gate; exl3_silu_lut.cuh:15-31, inference.cu:575-579. */
void po_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out, long long count,
               int *bad);

/* ---- A11 embedding gather --------------------------------------------------- */
/* out[t][:] = table[ids[t]][:]; ids outside [0, vocab) set bad and leave the row.
 * decode_control.cuh:68-79, prefill_control.cuh:3-22. */
void po_embed(const uint16_t *table, const int32_t *ids, uint16_t *out, int tokens, int hidden,
              int vocab, int *bad);

/* ---- A12 device state predicates ------------------------------------------- */
typedef struct {
  int32_t token, position, capacity, remaining, global_valid, local_valid, eos, stopped;
} po_DecodeState;
typedef struct {
  int32_t base, prompt_offset, tokens, capacity, committed;
  uint32_t binding_epoch, request_epoch, valid;
} po_PrefillState;
int po_decode_ready(const po_DecodeState *s, int maximum, int vocab); /* context_admission.cuh:5-11 */
int po_valid_prefill_state(const po_PrefillState *s, int active_tokens, int capacity,
                           uint32_t binding_epoch, int maximum); /* prefill_state.h:16-24 */

/* ---- Local-ring checkpoint capture (kv_checkpoint.cuh) --------------------------- */
/* CopyEncodedPlane / CaptureLocal's copy (kv_checkpoint.cuh:12-25, 70-88): slot s of the
 * 1024-row snapshot holds position p = anchor-1 - ((anchor-1 - s + 1024) % 1024): the
 * chunk's row p - base when p >= base, the old ring's slot s when 0 <= p < base, zeros
 * before position 0.  Rows of row_bytes bytes. */
void po_kv_checkpoint_plane(const uint8_t *old_rows, const uint8_t *current_rows,
                            uint8_t *saved_rows, int row_bytes, int base, int anchor);
/* The capture's admission (kv_checkpoint.cuh:33-38, 62-67): a valid PrefillState for
 * `tokens` rows, capacity >= 1024, base < anchor <= base + tokens. */
int po_kv_checkpoint_admitted(const po_PrefillState *s, int tokens, int anchor,
                              uint32_t binding_epoch, int maximum);

/* ---- Decode attention over a BF16 cache (split-K + per-head merge) ---------------- */
/* One sequence at `position`: gqa8_fragment_validation::SplitBF16
 * (attention_gqa8_fragment_validation.cuh:79-214) and attention_perhead_exact::Merge
 * (attention_perhead_exact.cuh:7-38), generalised to hq / hkv query heads per KV head.
 * Keys are positions first .. position (n = position + 1, or min(that, 1024) for a local
 * ring), cache row (first + offset) % cap of kc / vc [cap][hkv*128].  Splits of 32-key
 * tiles; per tile the online softmax with the score scale 1/sqrt(128) applied after the
 * dot product, BF16 probabilities in the PV product and fp32 ones in the denominator;
 * partial = accum / denominator, lse = max + log(denominator); then the merge:
 * weights exp(lse - max) / sum, out = B(sum_s w_s * partial_s) (fmaf, split order).
 * splits = 0 takes the reference's count, min(ceil(cap/32), local ? 16 : 32).  The dot
 * products and PV sums run sequentially in fp32 (the reference's tensor-core order is not
 * specified); expf/logf are the host libm's.  Returns the split count used. */
int po_decode_attention(const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int cap,
                        int position, int local, int hq, int hkv, int splits, uint16_t *out,
                        int *bad);

/* Decode attention over a q8_0 cache, one sequence: q8_native::EncodeQuery, Split and
 * Merge (kv_q8_native.cuh:103-148, 198-363) for hq / hkv query heads per KV head.  The
 * query is rotated (128-point) and coded per 32-block with an fp32 scale; scores are
 * integer code dot products scaled per block (fmaf order of the reference: four partial
 * sums, then ((p0 + p1) + (p2 + p3))); 128-key tiles run as four interleaved 32-key online
 * softmax streams (per-key denominators, fp32 probabilities in PV against V codes times
 * their block scale), joined per split; the merge rotates the result back (two 64-point
 * transforms) and rounds to BF16.  Rows are the 544-byte q8_0 cache rows [cap]; a local
 * ring has cap 1024.  splits = 0: the reference's 16 (local) or 32.  Returns the splits
 * used, or -1 (flag raised) for a non-finite query. */
int po_decode_attention_q8_0(const uint16_t *q, const uint8_t *kc, const uint8_t *vc, int cap,
                             int position, int local, int hq, int hkv, int splits, uint16_t *out,
                             int *bad);

#ifdef __cplusplus
}
#endif
#endif
