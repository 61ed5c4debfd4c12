/*
 * tq4_oracle.h -- CPU restatement of the TurboQuant TQ4 quantised-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * product in ascend-micro-harness_amd/csrc and the timed CPU baseline of
 * bench.py. Nothing on the product path may link, load or call it: the only
 * callers allowed are tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the fxslava/ascend-micro-harness checkout). What pins each function (golden
 * vectors from the reference's own header-only oracles, closed forms,
 * brute force) is listed beside it; a function with no pin says
 * "parity unpinned".
 *
 * Conventions shared with the product (the cache contract):
 *   key   nibble = ((page*H + head)*S + token)*d + channel            (token-major)
 *   value nibble = ((page*H + head)*S)*d + (token/16)*16*d
 *                  + channel*16 + token%16                             (strip-blocked)
 *   scale index  = ((plane*P + page)*H + head)*S + token, plane 0 = K, 1 = V
 *   nibbles: two per byte, low nibble first, signed INT4 in [-8, 7].
 *   reference: tests/common/turboquant_scatter_oracle.hpp:31-38,110-132
 */
#ifndef TQ4_ORACLE_H
#define TQ4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQ4O_STRIP 16u          /* strip height R */
#define TQ4O_MASKED (-3.0e38f)  /* kMaskedScore, turboquant_decode_tail.hpp:72 */

/* zero-row / absmax policy of the quantiser */
#define TQ4O_POLICY_PREFILL 0   /* absmax floored at 1.0 (turboquant_oracle.hpp:413) */
#define TQ4O_POLICY_EXACT 1     /* exact absmax, absmax==0 -> scale 1 (turboquant_scatter_oracle.hpp:192-200) */

/* input dtype of the writers */
#define TQ4O_IN_INT8 0
#define TQ4O_IN_BF16 1

/* ---------------------------------------------------------------- bf16 */
float tq4o_bf16_to_f32(uint16_t raw);
uint16_t tq4o_f32_to_bf16(float value);  /* RNE, quiet NaN kept */

/* ------------------------------------------------------------ index maps */
uint64_t tq4o_key_nibble(uint32_t H, uint32_t S, uint32_t d, uint32_t page, uint32_t head,
                         uint32_t token, uint32_t channel);
uint64_t tq4o_value_nibble(uint32_t H, uint32_t S, uint32_t d, uint32_t page, uint32_t head,
                           uint32_t token, uint32_t channel);
uint64_t tq4o_scale_index(uint32_t P, uint32_t H, uint32_t S, uint32_t plane, uint32_t page,
                          uint32_t head, uint32_t token);
int tq4o_read_nibble(const int8_t* cache, uint64_t nibble);
void tq4o_write_nibble(int8_t* cache, uint64_t nibble, int value);

/* -------------------------------------------------------------- rotation */
int tq4o_pi_sign(int channel);
void tq4o_canonical_signs(uint32_t d, float* signs);
void tq4o_build_tables_i8(uint32_t d, const float* signs, int8_t* tables);
int tq4o_signs_from_tables_i8(uint32_t d, const int8_t* tables, float* signs);
void tq4o_rotate_ingress(const float* x, const float* signs, uint32_t d, float* y);
void tq4o_rotate_egress(const float* x, const float* signs, uint32_t d, float* y);
void tq4o_rotate_dense(const float* x, const float* signs, uint32_t d, int transpose, double* y);

/* ------------------------------------------------------------- quantiser */
void tq4o_quantise_row(const float* y, uint32_t d, float inv_sqrt_len, int policy, int8_t* q,
                       float* scale);

/* --------------------------------------------------------------- writers */
int64_t tq4o_reshape_and_cache(int in_dtype, const void* key, const void* value,
                               int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                               const int32_t* slot_mapping, const float* pi_signs,
                               uint32_t num_tokens, uint32_t num_kv_heads, uint32_t head_size,
                               uint32_t block_size, uint32_t num_blocks, float inv_sqrt_len,
                               int policy);
int64_t tq4o_reshape_scatter(const uint16_t* key, const uint16_t* value, int8_t* key_cache,
                             int8_t* value_cache, float* scale_cache,
                             const int32_t* slot_mapping, const float* pi_signs,
                             const int32_t* cu_seqlens, uint32_t num_requests,
                             uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                             uint32_t num_blocks, uint32_t item_begin, uint32_t item_count,
                             float inv_sqrt_len);

/* ---------------------------------------------------------------- decode */
void tq4o_partition(uint32_t pages, uint32_t splits, uint32_t split, uint32_t* begin,
                    uint32_t* count);
uint32_t tq4o_active_in_strip(uint64_t token_base, uint32_t seq_len);
void tq4o_rotate_query(const uint16_t* q, const float* signs, uint32_t d, float inv_sqrt_len,
                       float scale, float* q_eff);
void tq4o_combine_step(float* m, float* l, float* acc, float m_t, float l_t, const float* acc_t,
                       uint32_t d);
/* decode flags: 1 = q already holds Pi q (BF16); 2 = round Pi q to BF16
 * before the score, the reference device's operand
 * (paged_decode_oracle.hpp:506-514); neither = FP32 q_rot. */
int tq4o_decode_partials(const uint16_t* q, const int8_t* key_cache, const int8_t* value_cache,
                         const float* scale_cache, const int32_t* block_tables,
                         const int32_t* context_lens, const float* pi_signs, float* workspace,
                         uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                         uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                         uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                         float inv_sqrt_len, uint32_t flags);
int tq4o_combine(const float* workspace, const float* pi_signs, const float* gate, uint16_t* out,
                 float* out_f32, uint32_t num_seqs, uint32_t num_heads, uint32_t head_size,
                 uint32_t num_splits, float inv_sqrt_len, uint32_t output_stage);
int tq4o_paged_decode(const uint16_t* q, const int8_t* key_cache, const int8_t* value_cache,
                      const float* scale_cache, const int32_t* block_tables,
                      const int32_t* context_lens, const float* pi_signs, const float* gate,
                      uint16_t* out, float* out_f32, uint32_t num_seqs, uint32_t num_heads,
                      uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                      uint32_t num_blocks, uint32_t max_blocks_per_seq, uint32_t num_splits,
                      float scale, float inv_sqrt_len, uint32_t output_stage, uint32_t flags,
                      uint32_t threads);
int tq4o_decode_reference_f64(const uint16_t* q, const int8_t* key_cache,
                              const int8_t* value_cache, const float* scale_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              const float* pi_signs, const float* gate, double* out,
                              uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                              uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, float scale, float inv_sqrt_len,
                              uint32_t output_stage, uint32_t flags);

/* record stride of one partial (m, l, pad, pad, acc[d]) in floats */
uint32_t tq4o_record_floats(uint32_t head_size);

/* multi-threaded writer for the CPU baseline: partitions strips over threads */
int64_t tq4o_reshape_and_cache_mt(int in_dtype, const void* key, const void* value,
                                  int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                                  const int32_t* slot_mapping, const float* pi_signs,
                                  uint32_t num_tokens, uint32_t num_kv_heads, uint32_t head_size,
                                  uint32_t block_size, uint32_t num_blocks, float inv_sqrt_len,
                                  int policy, uint32_t threads);

/* ------------------------------------------------------------- codebooks
 * The reference's codebook quantiser leaves: ICDF (scaled sigmoid -> signed
 * int4), Lloyd-Max and the Gaussian-CDF compander (2/4-bit unsigned codes,
 * packed low bits first). Pins: tests/golden/cb_* from the reference's own
 * fixtures and oracles, and the closed forms of the codebooks. */
#define TQ4O_BOOK_LLOYDMAX 0u
#define TQ4O_BOOK_GAUSSIAN_CDF 1u
float tq4o_codebook_centroid(uint32_t book, uint32_t bits, uint32_t q);
float tq4o_lloydmax_threshold(uint32_t bits, uint32_t i);
uint32_t tq4o_lloydmax_code(uint32_t bits, float x);
uint32_t tq4o_gaussian_cdf_code(uint32_t bits, float x);
void tq4o_codebook_pack(const uint32_t* q, uint64_t n, uint32_t bits, uint8_t* out);
int tq4o_codebook_quantize(uint32_t book, uint32_t bits, const float* x, uint64_t n, float* recon,
                           uint8_t* packed);
int tq4o_codebook_dequantize(uint32_t book, uint32_t bits, const uint8_t* packed, uint64_t n,
                             float* recon);
float tq4o_f16_to_f32(uint16_t h);
int tq4o_icdf_code(double x);
int tq4o_icdf_quantize(int in_bf16, const uint16_t* in, uint64_t n, uint8_t* packed);

/* ------------------------------------------------------------- RMS codec
 * The vllm-ascend baseline codec (TurboQuantCodec<4>) and its writer:
 * ApplyPi, RMS scale, 15-threshold levels, biased int8 packing, centroids. */
float tq4o_rms_threshold(uint32_t i);
float tq4o_rms_centroid(uint32_t level);
void tq4o_rms_apply_pi(float* x, const float* signs, float inv_sqrt_len, uint32_t n);
float tq4o_rms_scale(const float* y, uint32_t n, float inv_sqrt_len);
uint32_t tq4o_rms_level(float y, float rcp);
void tq4o_rms_quantize_row(const float* x, const float* signs, uint32_t n, float inv_sqrt_len,
                           uint8_t* levels, int8_t* packed, float* scale);
uint32_t tq4o_rms_scale_slot_floats(uint32_t num_kv_heads);
int64_t tq4o_rms_reshape_and_cache(int in_dtype, const uint16_t* key, const uint16_t* value,
                                   int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                                   const int32_t* slots, const float* signs, uint32_t num_tokens,
                                   uint32_t H, uint32_t d, uint32_t S, uint32_t P,
                                   uint32_t token_limit, float inv_sqrt_len);
void tq4o_rms_dequantize(const int8_t* packed, uint64_t n, float* out);

#ifdef __cplusplus
}
#endif

#endif
