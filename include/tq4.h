/*
 * tq4.h -- C ABI of the MI355X-native TurboQuant TQ4 quantised-KV hot path.
 *
 * One shared library, libtq4.so (ascend-micro-harness_amd/), exports every
 * symbol declared here. The entry points take plain device pointers, sizes
 * and a hipStream_t passed as void*; they allocate nothing (the caller owns
 * every buffer, including the decode workspace), never synchronise, and
 * never throw: each returns a tq4_status (0 = launched, negative = refused,
 * nothing launched). Work is stream-ordered and asynchronous.
 *
 * The cache contract (identical to the reference's, so caches are
 * interchangeable; d = head_size, H = num_kv_heads, S = block_size,
 * P = num_blocks, a strip is 16 tokens):
 *   key   nibble = ((page*H + head)*S + token)*d + channel            token-major
 *   value nibble = ((page*H + head)*S)*d + (token/16)*16*d
 *                  + channel*16 + token%16                             strip-blocked
 *   scale float  = ((plane*P + page)*H + head)*S + token    plane 0 key, 1 value
 *   nibbles: two per byte, low nibble first, signed INT4 in [-8, 7];
 *   stored value = nibble * scale, scale = 2^(e-2) * inv_sqrt_len.
 *   (reference: tests/common/turboquant_scatter_oracle.hpp:31-38,110-132,
 *    tests/common/turboquant_oracle.hpp:31-38)
 *
 * Supported shapes: head_size in {64, 128, 256}; block_size a multiple of
 * 16; decode GQA group num_heads / num_kv_heads in [1, 16].
 */
#ifndef TQ4_H
#define TQ4_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TQ4_OK = 0,
    TQ4_ERR_NULL_POINTER = -1,  /* a required pointer is NULL */
    TQ4_ERR_HEAD_SIZE = -2,     /* head_size not in {64, 128, 256} */
    TQ4_ERR_GEOMETRY = -3,      /* zero heads/blocks, block_size % 16, GQA group */
    TQ4_ERR_PARTIAL_STRIP = -4, /* num_tokens not a whole number of strips */
    TQ4_ERR_SPLITS = -5,        /* num_splits out of range */
    TQ4_ERR_WORKSPACE = -6,     /* workspace NULL, smaller than required or not 16-byte aligned */
    TQ4_ERR_OUTPUT_STAGE = -7,  /* output_stage > 2, or stage 2 without gate */
    TQ4_ERR_ROTATION = -8,      /* neither pi_signs nor tables given */
    TQ4_ERR_LAUNCH = -9,        /* the HIP runtime refused the launch */
    TQ4_ERR_RANGE = -10,        /* a size exceeds what the kernels index */
    TQ4_ERR_CODEBOOK = -11,     /* codebook leaf: bits, mode or element count */
    TQ4_ERR_FLAGS = -12,        /* unknown flag bits, or a test hook without its bound */
    TQ4_ERR_SCRATCH = -13       /* beyond the no-allocation entry's static scratch */
} tq4_status;

/* Human-readable name of a tq4_status. */
const char* tq4_status_string(int status);

/* ABI version: (major << 16) | minor. */
uint32_t tq4_version(void);

/* ----------------------------------------------------------------------
 * reshape_and_cache: rotate (randomised Hadamard M = (H_{d/32} (x) I32) .
 * diag(pi_signs) . (I_{d/32} (x) H32), butterflies in registers), quantise
 * to power-of-two-scaled INT4, pack and store whole 16-token strips.
 *
 * Slot contract per strip s (tokens 16s..16s+15): slot_mapping[16s+i] ==
 * slot_mapping[16s] + i, slot_mapping[16s] % 16 == 0 and page < num_blocks.
 * A strip that violates it writes nothing (the reference oracle's
 * bad-slot behaviour, tests/common/turboquant_oracle.hpp:274-287,489-494).
 * Quantiser: absmax floored at 1.0 (turboquant_oracle.hpp:412-448).
 * num_tokens must be a whole number of tokens_per_core strips
 * (TQ4_ERR_PARTIAL_STRIP otherwise), tokens_per_core a multiple of 16; it is
 * accepted for signature compatibility, the grid is chosen here.
 * num_kv_heads <= 65535 and 2 * num_tokens / 16 * num_kv_heads < 2^31
 * (TQ4_ERR_RANGE otherwise).
 * Rotation signs: pi_signs (float[head_size] of +-1) when non-NULL, else the
 * first column of `tables` (the reference's 2*(d/32) row-major 32x32 INT8
 * blocks, T[0][g][c0][0] = sign[g*32+c0]). reuse_mode4_flags selects an
 * Ascend cross-core flag policy and has no counterpart here (ignored).
 *
 * Replaces launch_turboquant_reshape_and_cache_a8
 * (kernels/ops/turboquant/turboquant_reshape_and_cache_a8.cpp:1578-1627).
 */
int tq4_reshape_and_cache_a8(void* stream, const int8_t* key, const int8_t* value,
                             int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                             const int32_t* slot_mapping, const float* pi_signs,
                             const int32_t* tables, uint32_t num_tokens, uint32_t num_kv_heads,
                             uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                             uint32_t tokens_per_core, float inv_sqrt_len,
                             bool reuse_mode4_flags);

/* Same contract with BF16 activations (uint16 bit patterns); `tables`, when
 * used, holds BF16 +-1 entries.
 * Replaces launch_turboquant_reshape_and_cache_bf16
 * (kernels/ops/turboquant/turboquant_reshape_and_cache_bf16.cpp:1993-2059). */
int tq4_reshape_and_cache_bf16(void* stream, const uint16_t* key, const uint16_t* value,
                               int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                               const int32_t* slot_mapping, const float* pi_signs,
                               const int32_t* tables, uint32_t num_tokens,
                               uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                               uint32_t num_blocks, uint32_t tokens_per_core,
                               float inv_sqrt_len, bool reuse_mode4_flags);

/* ----------------------------------------------------------------------
 * reshape_scatter: BF16 tokens at arbitrary slots (decode-step writes,
 * prefill tails). Work item = (request, kv_head) for item in
 * [item_begin, item_begin + item_count), item = request * num_kv_heads + head.
 * Request r owns tokens [cu_seqlens[r], cu_seqlens[r+1]) (cu_seqlens NULL =
 * one token per request); slot < 0 marks a padded token and is skipped.
 * The value strip is read-modify-written nibble-exactly: every nibble the
 * launch does not own is preserved. Quantiser: exact absmax, absmax == 0
 * gives codes 0 and scale 1.0 (turboquant_scatter_oracle.hpp:185-217).
 * block_dim is a grid-size hint (0 = one workgroup per item). When
 * launch_probe is non-NULL, workgroup 0 writes int32[32]: lanes 0-7 its
 * block index, 8-15 the grid size, 16-23 1, 24-31 item_count.
 * Two work items of one launch must not own tokens of the same strip.
 * Replaces launch_turboquant_reshape_scatter_aiv
 * (kernels/ops/turboquant/turboquant_reshape_scatter_aiv.cpp:760-773).
 */
int tq4_reshape_scatter(void* stream, uint32_t block_dim, const uint16_t* key,
                        const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                        float* scale_cache, const int32_t* slot_mapping, const float* pi_signs,
                        const int32_t* cu_seqlens, int32_t* launch_probe, uint32_t num_requests,
                        uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                        uint32_t num_blocks, uint32_t item_begin, uint32_t item_count,
                        float inv_sqrt_len);

/* ----------------------------------------------------------------------
 * Paged split-K decode over the TQ4 cache.
 *
 * q: [num_seqs][num_heads][head_size] BF16; q head j reads kv head
 * j / (num_heads / num_kv_heads). block_tables: [num_seqs][max_blocks_per_seq]
 * physical pages; context_lens: [num_seqs] live tokens (<= max_blocks_per_seq
 * * block_size). Scores are scale * (Pi q) . k_deq with Pi = M *
 * inv_sqrt_len; tokens at or past context_len are masked by overwrite.
 * Split k of num_splits owns logical pages Partition(max_blocks_per_seq, K, k)
 * of the block-table window (include/turboquant_splitk_contract.hpp:123-130,
 * as the reference AIC decode partitions its page window); a split with no
 * live token exports the neutral record m = -3e38, l = 0, acc = 0. Block-table
 * entries >= num_blocks contribute nothing (they are never dereferenced).
 * output_stage: 0 = normalised context in the rotated basis, 1 = rotated back
 * (Pi^T), 2 = rotated back and divided by 1 + exp(-gate), gate [num_seqs]
 * [num_heads][head_size] FP32. out: [num_seqs][num_heads][head_size] BF16 RNE.
 * flags: TQ4_DECODE_QUERY_ROTATED = q already holds Pi q (no rotation).
 */
#define TQ4_DECODE_QUERY_ROTATED 1u
/* tq4_paged_decode_partials only: FP32 scores and recurrence in the
 * reference's operation order, on the vector ALU, with the rotated query
 * rounded to BF16 first (the reference device's score operand,
 * tests/common/paged_decode_oracle.hpp:506-514; a pre-rotated q is BF16
 * already). Its records meet the reference rig's budgets
 * (tests/npu/turboquant_splitk_rigs.hpp:144-158); slower than the default
 * MFMA path, whose fp16 operands agree with them to about 2^-11. */
#define TQ4_DECODE_PRECISE 2u
/* Test hooks of the fused entry's bounded wait (never set in production):
 * TQ4_DECODE_TEST_POLL_BOUND cuts a combiner's record poll to 16 attempts
 * (from 2^20); TQ4_DECODE_TEST_WITHHOLD (accepted only together with the
 * bound) makes the split holding ticket 0 of every (seq, kv head) with more
 * than one live split skip its record, so that group's combiner gives up and
 * is counted (tq4_decode_poll_timeouts). Every workgroup still exits. */
#define TQ4_DECODE_TEST_POLL_BOUND (1u << 30)
#define TQ4_DECODE_TEST_WITHHOLD (1u << 31)
#define TQ4_MAX_SPLITS 256u
/* A split walks at most this many 16-token strips (its block-table window is
 * staged on chip): num_splits must be at least
 * ceil(max_blocks_per_seq * block_size / 16 / TQ4_MAX_SPLIT_STRIPS)
 * (TQ4_ERR_SPLITS). The cache must hold fewer than 2^32 (page, head, token)
 * rows: num_blocks * num_kv_heads * block_size < 2^32 (TQ4_ERR_RANGE). */
#define TQ4_MAX_SPLIT_STRIPS 2048u

/* Workspace bytes for num_splits (partial records plus the per-(seq, kv
 * head) tickets of the fused entry). */
size_t tq4_decode_workspace_bytes(uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                                  uint32_t head_size, uint32_t num_splits);

/* A split count for this geometry: at least two workgroups per compute unit
 * in flight, and splits of at most ~512 strips of 16 tokens. */
uint32_t tq4_decode_auto_splits(uint32_t num_seqs, uint32_t num_kv_heads,
                                uint32_t max_blocks_per_seq, uint32_t block_size);

/* Zero a workspace (a fill kernel, no memset node). The fused entry needs a
 * zeroed workspace before its first call and leaves it zeroed after every
 * call (its counters, and its records, which it consumes and clears); a
 * workspace that tq4_paged_decode_partials has written since must be zeroed
 * again before tq4_paged_decode uses it. */
/* tq4_decode_auto_splits for a caller that holds the context lengths on the
 * host (context_lens: num_seqs host integers; NULL gives the plain rule): a
 * ragged batch (longest >= 1.6 x mean) whose num_seqs * num_kv_heads lies
 * between 256 and 768 takes at least 3 splits. No reference counterpart (the
 * reference's callers pass their split count). */
uint32_t tq4_decode_auto_splits_lens(uint32_t num_seqs, uint32_t num_kv_heads,
                                     uint32_t max_blocks_per_seq, uint32_t block_size,
                                     const int32_t* context_lens);

int tq4_decode_workspace_init(void* stream, void* workspace, size_t workspace_bytes);

/* The fused entry's timeout count: rows (times 16-split record chunks) whose
 * combiner stopped polling at its bound with records still missing, summed
 * over every call since the workspace was last zeroed. Nonzero means those
 * calls' outputs include rows combined from incomplete records, and the
 * workspace no longer holds the all-zero state the next call needs: zero it
 * again (tq4_decode_workspace_init). The count is copied to *count
 * (host or device memory) in stream order; read it after synchronising the
 * stream. num_seqs and num_kv_heads are those the workspace was sized for.
 * Reports the reference's watchdog timeout to the host
 * (kernels/ops/turboquant/turboquant_splitk_reduce.cpp:34-45). */
int tq4_decode_poll_timeouts(void* stream, const void* workspace, size_t workspace_bytes,
                             uint32_t num_seqs, uint32_t num_kv_heads, uint32_t* count);

/* Fused decode: partials, then one workgroup of each (seq, kv head) -- the
 * last of its splits to start -- waits for the others' records, LSE-combines
 * them in split order, rotates back, gates and stores BF16 -- one launch.
 * The wait is bounded and only on workgroups already running, so the launch
 * completes whatever the number of workgroups in flight.
 * Splits that hold no live token of their sequence (those at or past
 * ceil(ceil(context_len / block_size) / ceil(max_blocks_per_seq /
 * num_splits))) write nothing and do not take part in the combine, so a
 * ragged batch can use many splits. Calls that overlap on one workspace
 * race. num_splits 0 = auto.
 * Modelled on turboquant_paged_attention_impl
 * (kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:773-793);
 * replaces the L2-spinlock accumulation
 * (kernels/ops/turboquant/turboquant_splitk_reduce.cpp:279-350,385-405). */
int tq4_paged_decode(void* stream, const uint16_t* q, const int8_t* key_cache,
                     const int8_t* value_cache, const float* scale_cache,
                     const int32_t* block_tables, const int32_t* context_lens,
                     const float* pi_signs, const float* gate, void* workspace,
                     size_t workspace_bytes, uint16_t* out, uint32_t num_seqs,
                     uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_size,
                     uint32_t block_size, uint32_t num_blocks, uint32_t max_blocks_per_seq,
                     uint32_t num_splits, float scale, float inv_sqrt_len,
                     uint32_t output_stage, uint32_t flags);

/* tq4_paged_decode without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. Same arguments and
 * result as tq4_paged_decode; the workspace is a static 16 MiB device array
 * inside libtq4.so, one per GPU, held until the process ends (zero when the
 * library's code object is loaded; its address is looked up at the first
 * call on each device, which launches nothing, so that call may be made
 * under graph capture; no allocation ever).
 * A call whose workspace (tq4_decode_workspace_bytes) exceeds 16 MiB is
 * refused with TQ4_ERR_SCRATCH (e.g. 64 sequences x 32 q heads at d = 128 fit
 * up to 15 splits). Every call on one GPU shares that array: calls that
 * overlap in time on one GPU (two streams, two threads) race and must be
 * serialised by the caller. The test hooks are refused (TQ4_ERR_FLAGS). A
 * combiner waits only for workgroups that are already running, so a poll
 * give-up (2^20 polls) means a stalled device; it is counted in the scratch
 * (tq4_paged_decode_noalloc_poll_timeouts) and leaves late records and the
 * count behind, which later calls of any geometry would read: after a
 * nonzero count, call tq4_paged_decode_noalloc_reset before the next call. */
int tq4_paged_decode_noalloc(void* stream, const uint16_t* q, const int8_t* key_cache,
                             const int8_t* value_cache, const float* scale_cache,
                             const int32_t* block_tables, const int32_t* context_lens,
                             const float* pi_signs, const float* gate, uint16_t* out,
                             uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                             uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                             uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                             float inv_sqrt_len, uint32_t output_stage, uint32_t flags);

/* The no-allocation decode's sticky poll-timeout count for the geometry of
 * its last call (num_seqs, num_kv_heads locate the count in the scratch), as
 * tq4_decode_poll_timeouts reads it (asynchronous on `stream`; `count` is a
 * host or device pointer). Allocates nothing. No counterpart in the
 * reference (it reports its watchdog the same way: README.md:65-76). */
int tq4_paged_decode_noalloc_poll_timeouts(void* stream, uint32_t num_seqs,
                                           uint32_t num_kv_heads, uint32_t* count);

/* Zero the whole no-allocation scratch of the current device (one fill
 * kernel on `stream`; allocates nothing): after a poll give-up, before the
 * next tq4_paged_decode_noalloc call. Calls on other streams must not
 * overlap it. No counterpart in the reference. */
int tq4_paged_decode_noalloc_reset(void* stream);

/* Partials only: workspace record (seq, q head, split) at float offset
 * ((seq*num_heads + head)*num_splits + split)*(head_size + 4) holds
 * [m, l, 0, 0, acc[head_size]] -- m the running max of the natural-log score,
 * l = sum exp(s - m), acc = sum exp(s - m) * v in the rotated basis.
 * Modelled on launch_turboquant_paged_decode_splitk_aic
 * (kernels/ops/turboquant/turboquant_paged_decode_attention.cpp:1727-1766):
 * the same Partition and recurrence, but not its argument list or record --
 * per-sequence context lengths instead of one seq_len and a page window, a
 * [num_seqs][max_blocks_per_seq] table, pi_signs instead of a 256 x 256
 * pi_table, one [m, l, 0, 0, acc] record per (seq, q head, split) instead of
 * [m(8) | l(8) | acc] per packed row. The default path feeds the MFMA an FP16
 * q operand and FP16 P * value-scale operands; with TQ4_DECODE_PRECISE the
 * records follow the reference's FP32 recurrence on a BF16 q_rot. workspace
 * holds at least num_seqs * num_heads * num_splits * (head_size + 4) floats. */
int tq4_paged_decode_partials(void* stream, const uint16_t* q, const int8_t* key_cache,
                              const int8_t* value_cache, const float* scale_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              const float* pi_signs, float* workspace, size_t workspace_bytes,
                              uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                              uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                              float inv_sqrt_len, uint32_t flags);

/* LSE combine of num_splits partial records per (seq, q head), then the
 * egress for output_stage. Replaces the reference's host-side / SyncAll
 * combine (tests/common/l2_atomic_oracle.hpp:156-176,
 * kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:733-740). */
int tq4_splitk_combine(void* stream, const float* workspace, const float* pi_signs,
                       const float* gate, uint16_t* out, uint32_t num_seqs, uint32_t num_heads,
                       uint32_t head_size, uint32_t num_splits, float inv_sqrt_len,
                       uint32_t output_stage);

/* ----------------------------------------------------------------------
 * Codebook quantiser leaves: standalone elementwise kernels over plain
 * device arrays (no cache layout). Codes pack low bits first: code i sits at
 * bit (i*bits) % 8 of byte i*bits/8.
 */

/* ICDF: FP16 (in_bf16 = 0) or BF16 values -> signed INT4
 * RNE(14 / (1 + exp(-x)) - 7) saturated to [-8, 7] (NaN -> 0), two per byte,
 * element 2j in bits [3:0] of byte j. `tiles` tiles of 1024 elements in,
 * 512 bytes out each. Replaces launch_camodel_icdf_quantize_fp16 / _bf16
 * (kernels/camodel/icdf_quantize.cpp:161-172); semantics of
 * routines/routine_vector_icdf_quantize.hpp:10-30. */
int tq4_icdf_quantize(void* stream, int in_bf16, const uint16_t* in, uint8_t* out,
                      uint32_t tiles);

/* The Lloyd-Max leaf and its companions over n*rows elements (a multiple of
 * 8; bits 2 or 4). mode:
 *   0, 1  Lloyd-Max: FP32 src -> codes = #{thresholds <= x} (NaN -> 0) and,
 *         when dst is not NULL, dst = the centroid of each code
 *         (include/routines/routine_vector_lloydmax_quantize.hpp:8-37);
 *   2     the Gaussian-CDF compander floor(2^b / (1 + exp(-(1.5976 +
 *         0.070565 x^2) x))) with the normal-quantile centroids
 *         (tests/common/lloydmax_oracle.hpp:19-28);
 *   3     the ICDF leaf on FP16 src (bits 4 only; codes as tq4_icdf_quantize,
 *         dst unused);
 *   4, 5  decode: src holds packed Lloyd-Max codes, dst = their centroids.
 * Modes 0/1 and 4/5 differ in the reference only by where the codebook table
 * lives on chip; here they are the same kernels. `guards` (the reference
 * rig's on-chip canary dump) is ignored and may be NULL.
 * Replaces launch_camodel_lloydmax_quantize
 * (kernels/camodel/lloydmax_quantize.cpp:96-99). */
int tq4_lloydmax_quantize(void* stream, const void* src, float* dst, uint8_t* codes,
                          uint32_t* guards, uint32_t bits, uint32_t mode, uint32_t n,
                          uint32_t rows);

/* ----------------------------------------------------------------------
 * The vllm-ascend RMS + threshold codec (TurboQuantCodec<4>) and its
 * baseline writer. Per (token, plane, kv head) vector x of head_size:
 *   y = Pi x, Pi = diag(pi_signs) H diag(pi_signs) * inv_sqrt_len (FWHT);
 *   scale = sqrt(sum y^2) * inv_sqrt_len + 1e-20;
 *   level = #{i : t_i < y / scale} over the 15 Lloyd-Max 4-bit thresholds t;
 *   byte = (level[2j] | level[2j+1] << 4) - 128 (int8).
 * Cache: key/value int8 [num_blocks * block_size slots][num_kv_heads]
 * [head_size / 2]; scale_cache float [slots][ceil(2 * num_kv_heads / 8) * 8]
 * = the K heads' scales, then the V heads', then zeros. type: 0 FP16, 1 BF16
 * (the reference's AscendType). Tokens whose slot is negative or past the
 * pool write nothing; when block_dim is not 0 only the first block_dim *
 * tokens_per_core tokens are written (the reference's grid covers those).
 * `tables` (the reference's gather/centroid tables) is not read. Summation
 * order of sum y^2: per 16th of the vector sequentially, then a pairwise tree.
 * Replaces turboquant_reshape_and_cache_impl of the baseline
 * (kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:754-771;
 * codec kernels/ops/turboquant/baseline/common/turboquant_codec_950.h:115-248). */
int tq4_rms_reshape_and_cache(void* stream, int type, uint32_t block_dim, const void* key,
                              const void* value, int8_t* key_cache, int8_t* value_cache,
                              float* scale_cache, const int32_t* slot_mapping,
                              const float* pi_signs, const int32_t* tables, uint32_t num_tokens,
                              uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                              uint32_t num_blocks, uint32_t tokens_per_core, float inv_sqrt_len);

/* The codec's decode: n (even) codes packed as above -> their centroids,
 * out[2j] from byte j's low nibble. Replaces TurboQuantCodec<4>::Dequantize4Bit
 * (kernels/ops/turboquant/baseline/common/turboquant_codec_950.h:165-172,251-285). */
int tq4_rms_dequantize(void* stream, const int8_t* packed, float* out, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* TQ4_H */
