/* tq4_kv4fp8.h -- C ABI of the KV4/FP8 64-token NZ-tiled cache decode.
 *
 * The second cache format the reference's vLLM layer ships: a 4-bit affine
 * cache read by its "fused decode opt" operator. Replaces
 *   launch_fused_decode_opt            include/turboquant_fused_decode_opt.hpp:186-188
 *   launch_fused_decode_opt_raw_query  include/turboquant_fused_decode_opt.hpp:192-194
 * (structs ascend_micro::fused_decode_opt::Launch / Buffers / RawQueryBuffers,
 * include/turboquant_fused_decode_opt.hpp:98-183).
 *
 * CACHE (per physical page of block_size rows, H = num_kv_heads <= 4, D = 256):
 *   key/value  int8 [page][block_size/64 tiles][H][4 column groups][64 rows][32 B];
 *              packed column c (0..127) of a row holds channel c in its low
 *              nibble and channel c + 128 in its high nibble, signed int4 n,
 *              level n + 0.5 (NzTiledPackedByte, turboquant_layout.h:81-92)
 *   scales     float [page][block_size rows][8]: lanes 0..H-1 the key scale
 *              of each KV head, lanes H..2H-1 the value scale
 *   element    K = (n + 0.5) * key_scale / kGain, V likewise
 *              (kGain = 2.9832882881, turboquant_mode.h:101)
 *
 * ARITHMETIC (the reference's, per (token, q head)): the query is put on the
 * FP8 e4m3 grid at 448 / (max|q| + 1e-20); 64-row tiles; logits
 * (Q8.K * key_scale * scale/kGain) / qScale; an online softmax; the
 * probabilities times value_scale/kGain are put on the FP8 grid at
 * 448 / (max + 1e-20) per tile, multiplied with V and divided back; the
 * context is normalised by 1 / (sum + 1e-20), optionally rotated back by
 * Pi = diag(s) H diag(s) / sqrt(D) (output_stage 1) and divided by
 * 1 + exp(-max(gate, -80)) (stage 2), then rounded to FP16 or BF16 (RNE).
 *
 * STATUS: 0 or a negative TQ4_ERR_* code (include/tq4.h); nothing is
 * launched when an argument is refused.
 */
#ifndef TQ4_KV4FP8_H
#define TQ4_KV4FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ascend_micro::fused_decode_opt::Launch, field for field, followed by three
 * fields of this library:
 *   num_blocks       physical pages in the key/value/scale caches; every page
 *                    index read from the block table is checked against it
 *                    (an entry < 0 or >= num_blocks: that page's rows are
 *                    skipped -- the reference refuses such a table in its
 *                    host tiling, build_decode_tiling's kUnmappedPage);
 *   workspace_bytes  the size of buffers->workspace
 *                    (>= tq4_kv4fp8_workspace_bytes(launch));
 *   test_flags       0 in production. Test hooks of the combiners' bounded
 *                    wait: TQ4_KV4FP8_TEST_POLL_BOUND cuts a combiner's
 *                    record poll to 16 attempts (from 2^20);
 *                    TQ4_KV4FP8_TEST_WITHHOLD (only with the bound) makes the
 *                    part holding ticket 0 of every group with more than one
 *                    live part skip its record exports, so the combiners that
 *                    need them give up and are counted
 *                    (tq4_kv4fp8_poll_timeouts). Every workgroup still exits.
 * grid, tasks_per_block and reduce_tasks_per_block are the NPU dispatch; they
 * are checked as valid_launch checks them (except its grid <= 32 bound) and
 * do not change the result. heads_per_task, splits and fused_context_limit
 * only partition the work in the reference; they are checked, and the result
 * does not depend on them (to FP32 rounding). probe_page/probe_tile are the
 * reference's diagnostic fields and are ignored. */
typedef struct tq4_kv4fp8_launch {
    uint32_t grid, tokens, heads, kv_heads;
    uint32_t head_size, block_size, max_blocks;
    uint32_t splits, heads_per_task, tasks_per_block;
    uint32_t reduce_tasks_per_block, fused_context_limit;
    float scale, inv_sqrt_len;
    uint32_t prologue_vectors_per_block, prologue_cube_chunk_vectors;
    uint32_t output_stage;
    uint32_t element_type; /* query/output/gate element: 0 FP16, 1 BF16 */
    uint32_t probe_page, probe_tile;
    uint32_t num_blocks;
    uint64_t workspace_bytes;
    uint32_t test_flags;
} tq4_kv4fp8_launch;

#define TQ4_KV4FP8_TEST_POLL_BOUND (1u << 30)
#define TQ4_KV4FP8_TEST_WITHHOLD (1u << 31)

/* ascend_micro::fused_decode_opt::Buffers. query: FP32 [tokens][heads][256]
 * in the rotated basis; block_table int32 [tokens][max_blocks];
 * context_lengths int32 [tokens]; output [tokens][heads][256] (element_type).
 * mode_tables and tiling are accepted and not read (this decode derives the
 * partition from context_lengths on the device). */
typedef struct tq4_kv4fp8_buffers {
    void *query, *key, *value, *scales, *block_table, *context_lengths;
    void *mode_tables, *workspace, *output;
    void* tiling;
} tq4_kv4fp8_buffers;

/* ascend_micro::fused_decode_opt::RawQueryBuffers. raw_query and gate are
 * element_type [tokens][heads][256]; pi_signs float [256] (+-1). The
 * rotated FP32 query is written to decode.query (as the reference's
 * prologue writes it) when that pointer is not NULL. rot_tables and h16 are
 * accepted and not read (the rotation runs as FP32 butterflies). */
typedef struct tq4_kv4fp8_raw_query_buffers {
    void *raw_query, *pi_signs, *rot_tables, *h16, *gate;
    tq4_kv4fp8_buffers decode;
} tq4_kv4fp8_raw_query_buffers;

/* Workspace this decode needs for `launch` (bytes, 256-aligned): a part
 * ticket per (token, kv head, 16-head chunk), the partial records of every
 * (token, q head, part) and a 256-byte status block (the poll-timeout count).
 * It must be zero before its first call
 * (tq4_kv4fp8_workspace_init); every call leaves it zero again, so one
 * workspace serves calls of any geometry it is large enough for. Calls that
 * overlap in time need their own workspaces. */
uint64_t tq4_kv4fp8_workspace_bytes(const tq4_kv4fp8_launch* launch);

/* Zero a workspace on `stream` (a fill kernel, so it may be captured in a
 * graph). workspace 16-byte aligned. No reference counterpart: the
 * reference's host code allocates its workspace per call. */
int tq4_kv4fp8_workspace_init(void* stream, void* workspace, uint64_t workspace_bytes);

/* The combiners' timeout count: rows whose bounded record poll gave up with
 * records still missing, summed over every call since the workspace was
 * zeroed. Nonzero means those calls' outputs include rows merged from
 * incomplete records (possible only when a combiner waits on a part that
 * cannot start, e.g. a process confined to fewer compute units than the
 * device reports), and the workspace must be zeroed again before the next
 * call. Copied to *count (host or device memory) in stream order; read it
 * after synchronising the stream. `launch` is the one the workspace was
 * sized for (workspace_bytes set). Reports the reference's watchdog timeout
 * to the host (kernels/ops/turboquant/turboquant_splitk_reduce.cpp:34-45). */
int tq4_kv4fp8_poll_timeouts(void* stream, const tq4_kv4fp8_launch* launch,
                             const void* workspace, uint32_t* count);

/* The pre-rotated entry (launch_fused_decode_opt): output_stage is not read. */
int tq4_kv4fp8_decode(void* stream, const tq4_kv4fp8_launch* launch,
                      const tq4_kv4fp8_buffers* buffers);

/* The raw-query entry (launch_fused_decode_opt_raw_query). */
int tq4_kv4fp8_decode_raw_query(void* stream, const tq4_kv4fp8_launch* launch,
                                const tq4_kv4fp8_raw_query_buffers* buffers);

/* The FP8 e4m3 operand rounding the decode applies to its query and
 * probability operands (round to nearest even on the OCP e4m3 grid), as f16
 * bits: out_f16[i] = f16(fp8(in[i])). n even. No reference counterpart: the
 * reference's CastToOperand (turboquant_codec_mx.h:349-359) is internal. */
int tq4_fp8_e4m3_round(void* stream, const float* in, uint16_t* out_f16, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
