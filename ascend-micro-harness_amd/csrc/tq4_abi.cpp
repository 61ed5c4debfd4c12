// tq4_abi.cpp -- the C ABI of libtq4.so (declared in include/tq4.h).
//
// Each entry point validates its geometry on the host, the way the
// reference launchers do (turboquant_reshape_and_cache_a8.cpp:1597-1609,
// turboquant_paged_decode_attention.cpp:1746-1759), but returns a tq4_status
// instead of throwing across the C boundary; nothing is launched on a
// refusal. Launches are asynchronous on the caller's stream.
#include <hip/hip_runtime.h>

#include "../../include/tq4.h"
#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace {

constexpr uint32_t kStrip = 16;

bool head_size_ok(uint32_t d) { return d == 64 || d == 128 || d == 256; }

int launched(hipError_t e) { return e == hipSuccess ? TQ4_OK : TQ4_ERR_LAUNCH; }

// Fused-decode workspace tail: one 1 KiB block holding the persistent
// kernel's work-queue counters (word 32x for sub-queue x, one 128-byte line
// each) and the sticky poll-timeout count (word 1), then one split ticket per
// (seq, kv head), each on its own 128-byte line: atomics on one line are
// served one after another, so counters that many workgroups hit at once
// must not share one.
constexpr size_t kQueueBytes = 1024;
constexpr uint32_t kFlagsKnown = TQ4_DECODE_QUERY_ROTATED | TQ4_DECODE_PRECISE |
                                 TQ4_DECODE_TEST_POLL_BOUND | TQ4_DECODE_TEST_WITHHOLD;
size_t ticket_bytes(uint32_t num_seqs, uint32_t num_kv_heads)
{
    return ((size_t)num_seqs * num_kv_heads * tq4::kTicketStride * sizeof(uint32_t) + 255) &
           ~(size_t)255;
}

int writer_checks(const void* key, const void* value, const int8_t* key_cache,
                  const int8_t* value_cache, const float* scale_cache, const int32_t* slots,
                  const float* pi_signs, const int32_t* tables, uint32_t num_tokens,
                  uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                  uint32_t num_blocks, uint32_t tokens_per_core)
{
    if (!head_size_ok(head_size)) return TQ4_ERR_HEAD_SIZE;
    if (num_kv_heads == 0 || num_blocks == 0 || block_size == 0 || block_size % kStrip)
        return TQ4_ERR_GEOMETRY;
    // WholeStrips (turboquant_wave_protocol.hpp:179-185): a partial trailing
    // strip would be silently dropped, so the geometry is refused.
    if (tokens_per_core == 0 || tokens_per_core % kStrip || num_tokens % tokens_per_core)
        return TQ4_ERR_PARTIAL_STRIP;
    if (num_tokens == 0) return TQ4_OK;
    if (!key || !value || !key_cache || !value_cache || !scale_cache || !slots)
        return TQ4_ERR_NULL_POINTER;
    if (!pi_signs && !tables) return TQ4_ERR_ROTATION;
    const uint64_t blocks = (uint64_t)(num_tokens / kStrip) * num_kv_heads * 2u;
    // the strip writer's grid is (strips, kv heads): at most 65535 heads
    if (blocks > 0x7fffffffull || num_kv_heads > 65535u) return TQ4_ERR_RANGE;
    return TQ4_OK;
}

}  // namespace

extern "C" {

const char* tq4_status_string(int status)
{
    switch (status) {
        case TQ4_OK: return "ok";
        case TQ4_ERR_NULL_POINTER: return "a required pointer is NULL";
        case TQ4_ERR_HEAD_SIZE: return "head_size must be 64, 128 or 256";
        case TQ4_ERR_GEOMETRY: return "invalid geometry (heads, blocks, block_size % 16, GQA group)";
        case TQ4_ERR_PARTIAL_STRIP:
            return "num_tokens must be a whole number of tokens_per_core strips (multiple of 16)";
        case TQ4_ERR_SPLITS: return "num_splits out of range";
        case TQ4_ERR_WORKSPACE: return "workspace missing or too small";
        case TQ4_ERR_OUTPUT_STAGE: return "output_stage must be 0, 1 or 2 (2 needs a gate)";
        case TQ4_ERR_ROTATION: return "neither pi_signs nor tables given";
        case TQ4_ERR_LAUNCH: return "the HIP runtime refused the launch";
        case TQ4_ERR_RANGE: return "a size exceeds the kernels' index range";
        case TQ4_ERR_CODEBOOK: return "codebook leaf: bits must be 2 or 4, mode 0..5, elements a multiple of 8";
        case TQ4_ERR_FLAGS: return "unknown flag bits, or a test hook without its poll bound";
        case TQ4_ERR_SCRATCH:
            return "the call needs more than the no-allocation entry's 16 MiB static scratch";
        default: return "unknown status";
    }
}

uint32_t tq4_version(void) { return (1u << 16) | 0u; }

int tq4_reshape_and_cache_a8(void* stream, const int8_t* key, const int8_t* value,
                             int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                             const int32_t* slot_mapping, const float* pi_signs,
                             const int32_t* tables, uint32_t num_tokens, uint32_t num_kv_heads,
                             uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                             uint32_t tokens_per_core, float inv_sqrt_len,
                             bool reuse_mode4_flags)
{
    (void)reuse_mode4_flags;
    const int rc = writer_checks(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                                 pi_signs, tables, num_tokens, num_kv_heads, head_size,
                                 block_size, num_blocks, tokens_per_core);
    if (rc != TQ4_OK || num_tokens == 0) return rc;
    return launched(tq4::launch_strip_writer((hipStream_t)stream, 0, key, value, key_cache,
                                             value_cache, scale_cache, slot_mapping, pi_signs,
                                             tables, num_tokens / kStrip, num_kv_heads, head_size,
                                             block_size, num_blocks, inv_sqrt_len));
}

int tq4_reshape_and_cache_bf16(void* stream, const uint16_t* key, const uint16_t* value,
                               int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                               const int32_t* slot_mapping, const float* pi_signs,
                               const int32_t* tables, uint32_t num_tokens,
                               uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                               uint32_t num_blocks, uint32_t tokens_per_core,
                               float inv_sqrt_len, bool reuse_mode4_flags)
{
    (void)reuse_mode4_flags;
    const int rc = writer_checks(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                                 pi_signs, tables, num_tokens, num_kv_heads, head_size,
                                 block_size, num_blocks, tokens_per_core);
    if (rc != TQ4_OK || num_tokens == 0) return rc;
    return launched(tq4::launch_strip_writer((hipStream_t)stream, 1, key, value, key_cache,
                                             value_cache, scale_cache, slot_mapping, pi_signs,
                                             tables, num_tokens / kStrip, num_kv_heads, head_size,
                                             block_size, num_blocks, inv_sqrt_len));
}

int tq4_reshape_scatter(void* stream, uint32_t block_dim, const uint16_t* key,
                        const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                        float* scale_cache, const int32_t* slot_mapping, const float* pi_signs,
                        const int32_t* cu_seqlens, int32_t* launch_probe, uint32_t num_requests,
                        uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                        uint32_t num_blocks, uint32_t item_begin, uint32_t item_count,
                        float inv_sqrt_len)
{
    if (!head_size_ok(head_size)) return TQ4_ERR_HEAD_SIZE;
    if (num_kv_heads == 0 || num_blocks == 0 || block_size == 0 || block_size % kStrip)
        return TQ4_ERR_GEOMETRY;
    if (item_count == 0 || num_requests == 0) return TQ4_OK;
    if (!key || !value || !key_cache || !value_cache || !scale_cache || !slot_mapping ||
        !pi_signs)
        return TQ4_ERR_NULL_POINTER;
    uint32_t grid = block_dim == 0 ? item_count : block_dim;
    if (grid > item_count) grid = item_count;
    if (grid > 65535u * 16u) grid = 65535u * 16u;
    return launched(tq4::launch_scatter_writer(
        (hipStream_t)stream, grid, key, value, key_cache, value_cache, scale_cache, slot_mapping,
        pi_signs, cu_seqlens, launch_probe, num_requests, num_kv_heads, head_size, block_size,
        num_blocks, item_begin, item_count, inv_sqrt_len));
}

size_t tq4_decode_workspace_bytes(uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                                  uint32_t head_size, uint32_t num_splits)
{
    if (num_splits == 0) num_splits = TQ4_MAX_SPLITS;
    return tq4::decode_records_bytes(num_seqs, num_heads, head_size, num_splits) +
           kQueueBytes + ticket_bytes(num_seqs, num_kv_heads);
}

uint32_t tq4_decode_auto_splits(uint32_t num_seqs, uint32_t num_kv_heads,
                                uint32_t max_blocks_per_seq, uint32_t block_size)
{
    // Workgroups for half the CUs (256); for one per CU while each split
    // still holds 16 strips (20 when that takes the fused combine past one
    // 16-split record chunk); for all their two slots when the splits would
    // still be long (> 64 strips); splits of at most ~512 strips; never
    // fewer than 16 strips per split, and at most 32 splits.
    // - Each extra item costs a table and a first-strip round trip, a merge
    //   and a record, and the persistent kernel orders the last splits
    //   longest first, so a batch that already fills the slots runs best
    //   with few, long items: 64 sequences x 8 KV heads, K = 1 beat K = 2 by
    //   20 % at ctx 4096; a spread of 1..32768 tokens wanted K = 4..8.
    // - One sequence (8 KV heads): K = 16 was best up to ctx 8192, K = 32
    //   from 12288 (16384: 10.7 against 11.6 us). Two sequences at ctx 4096
    //   and 8192, four at ctx 4096: one workgroup per CU, 11-16 % faster
    //   than half the CUs.
    // - More than 32 splits combine in two record chunks and measured 5-7 us
    //   slower than 32 at d = 128.
    const uint64_t strips = (uint64_t)max_blocks_per_seq * (block_size / kStrip);
    const uint64_t items = (uint64_t)num_seqs * num_kv_heads > 0
                               ? (uint64_t)num_seqs * num_kv_heads
                               : 1;
    uint64_t k = (128 + items - 1) / items;
    const uint64_t per_cu = 256 / items;
    if (per_cu > k && strips >= (per_cu > 16 ? 20 : 16) * per_cu) k = per_cu;
    if (strips > 64 * k) {
        uint64_t more = (512 + items - 1) / items;
        const uint64_t by_work = (strips + 63) / 64;
        if (more > by_work) more = by_work;
        if (k < more) k = more;
    }
    const uint64_t k_len = (strips + 511) / 512;
    if (k < k_len) k = k_len;
    const uint64_t by_len = strips / 16 > 0 ? strips / 16 : 1;
    if (k > by_len) k = by_len;
    if (k > 32) k = 32;
    // one split stages at most TQ4_MAX_SPLIT_STRIPS strips of its window
    const uint64_t k_min = (strips + TQ4_MAX_SPLIT_STRIPS - 1) / TQ4_MAX_SPLIT_STRIPS;
    if (k < k_min) k = k_min;
    if (k > TQ4_MAX_SPLITS) k = TQ4_MAX_SPLITS;
    if (k < 1) k = 1;
    return (uint32_t)k;
}

uint32_t tq4_decode_auto_splits_lens(uint32_t num_seqs, uint32_t num_kv_heads,
                                     uint32_t max_blocks_per_seq, uint32_t block_size,
                                     const int32_t* context_lens)
{
    uint32_t k = tq4_decode_auto_splits(num_seqs, num_kv_heads, max_blocks_per_seq, block_size);
    if (!context_lens || num_seqs == 0 || num_kv_heads == 0) return k;
    // A ragged batch (longest context >= 1.6 x the mean) whose (seq, kv head)
    // items fill the resident slots (512 at d <= 128) between half and one
    // and a half times: one item per (seq, kv head) leaves the launch waiting
    // on the longest sequences, so split them at least three ways. Measured
    // (64 x U[512, 8192]: 75.4 -> 72.3 us; 64 x U[128, 16384]: 133.3 ->
    // 125.2; 80 x U[512, 8192]: 96.5 -> 92.7), while a uniform or mildly
    // ragged batch (64 x 8192, 64 x U[2048, 8192]) runs best as it was.
    const uint64_t cap = (uint64_t)max_blocks_per_seq * block_size;
    uint64_t sum = 0, mx = 0;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        uint64_t c = context_lens[b] > 0 ? (uint64_t)context_lens[b] : 0;
        if (c > cap) c = cap;
        sum += c;
        if (c > mx) mx = c;
    }
    const uint64_t items = (uint64_t)num_seqs * num_kv_heads;
    if (sum > 0 && items * 2 > 512 && items * 2 <= 3 * 512 && mx * num_seqs * 5 >= sum * 8 &&
        k < 3 && max_blocks_per_seq >= 3)
        k = 3;
    return k;
}

int tq4_decode_workspace_init(void* stream, void* workspace, size_t workspace_bytes)
{
    if (!workspace) return TQ4_ERR_WORKSPACE;
    return launched(tq4::launch_fill_zero((hipStream_t)stream, workspace, workspace_bytes));
}

int tq4_decode_poll_timeouts(void* stream, const void* workspace, size_t workspace_bytes,
                             uint32_t num_seqs, uint32_t num_kv_heads, uint32_t* count)
{
    if (!workspace || !count) return TQ4_ERR_NULL_POINTER;
    const size_t tail = ticket_bytes(num_seqs, num_kv_heads) + kQueueBytes;
    if (num_seqs == 0 || num_kv_heads == 0 || workspace_bytes < tail ||
        ((uintptr_t)workspace & 15u))
        return TQ4_ERR_WORKSPACE;
    const char* word = (const char*)workspace + workspace_bytes - tail + sizeof(uint32_t);
    return launched(hipMemcpyAsync(count, word, sizeof(uint32_t), hipMemcpyDefault,
                                   (hipStream_t)stream));
}

namespace {

int decode_checks(const uint16_t* q, const int8_t* kc, const int8_t* vc, const float* sc,
                  const int32_t* tables, const int32_t* ctx, const float* pi_signs,
                  uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                  uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                  uint32_t max_blocks_per_seq, uint32_t flags)
{
    if (!head_size_ok(head_size)) return TQ4_ERR_HEAD_SIZE;
    if (num_seqs == 0 || num_kv_heads == 0 || num_heads == 0 || num_heads % num_kv_heads ||
        num_heads / num_kv_heads > 16 || block_size == 0 || block_size % kStrip ||
        num_blocks == 0 || max_blocks_per_seq == 0)
        return TQ4_ERR_GEOMETRY;
    if (!q || !kc || !vc || !sc || !tables || !ctx) return TQ4_ERR_NULL_POINTER;
    if (flags & ~kFlagsKnown) return TQ4_ERR_FLAGS;
    if ((flags & TQ4_DECODE_TEST_WITHHOLD) && !(flags & TQ4_DECODE_TEST_POLL_BOUND))
        return TQ4_ERR_FLAGS;
    if (!(flags & TQ4_DECODE_QUERY_ROTATED) && !pi_signs) return TQ4_ERR_ROTATION;
    // cache rows are indexed in 32 bits on the device
    if ((uint64_t)num_blocks * num_kv_heads * block_size > 0xffffffffull) return TQ4_ERR_RANGE;
    return TQ4_OK;
}

bool split_pages_ok(uint32_t max_blocks_per_seq, uint32_t block_size, uint32_t num_splits)
{
    const uint64_t pages = ((uint64_t)max_blocks_per_seq + num_splits - 1) / num_splits;
    return pages * (block_size / kStrip) <= TQ4_MAX_SPLIT_STRIPS;
}

tq4::DecodeParams make_params(const uint16_t* q, const int8_t* kc, const int8_t* vc,
                              const float* sc, const int32_t* tables, const int32_t* ctx,
                              const float* pi_signs, const float* gate, uint32_t num_seqs,
                              uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_size,
                              uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                              float inv_sqrt_len, uint32_t output_stage, uint32_t flags)
{
    tq4::DecodeParams p{};
    p.q = q;
    p.key_cache = kc;
    p.value_cache = vc;
    p.scale_cache = sc;
    p.block_tables = tables;
    p.context_lens = ctx;
    p.pi_signs = pi_signs;
    p.gate = gate;
    p.B = num_seqs;
    p.Hq = num_heads;
    p.Hkv = num_kv_heads;
    p.G = num_heads / num_kv_heads;
    p.D = head_size;
    p.S = block_size;
    p.P = num_blocks;
    p.max_blocks = max_blocks_per_seq;
    p.K = num_splits;
    p.scale = scale;
    p.inv_sqrt_len = inv_sqrt_len;
    p.output_stage = output_stage;
    p.flags = flags & TQ4_DECODE_QUERY_ROTATED;
    p.poll_limit = (flags & TQ4_DECODE_TEST_POLL_BOUND) ? tq4::kPollLimitTest : tq4::kPollLimit;
    p.withhold = (flags & TQ4_DECODE_TEST_WITHHOLD) ? 1u : 0u;
    return p;
}

}  // namespace

int tq4_paged_decode(void* stream, const uint16_t* q, const int8_t* key_cache,
                     const int8_t* value_cache, const float* scale_cache,
                     const int32_t* block_tables, const int32_t* context_lens,
                     const float* pi_signs, const float* gate, void* workspace,
                     size_t workspace_bytes, uint16_t* out, uint32_t num_seqs,
                     uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_size,
                     uint32_t block_size, uint32_t num_blocks, uint32_t max_blocks_per_seq,
                     uint32_t num_splits, float scale, float inv_sqrt_len,
                     uint32_t output_stage, uint32_t flags)
{
    int rc = decode_checks(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                           pi_signs, num_seqs, num_heads, num_kv_heads, head_size, block_size,
                           num_blocks, max_blocks_per_seq, flags);
    if (rc != TQ4_OK) return rc;
    if (flags & TQ4_DECODE_PRECISE) return TQ4_ERR_FLAGS;  // the partials entry's mode only
    if (!out) return TQ4_ERR_NULL_POINTER;
    if (output_stage > 2 || (output_stage == 2 && !gate)) return TQ4_ERR_OUTPUT_STAGE;
    if (output_stage >= 1 && !pi_signs) return TQ4_ERR_ROTATION;
    if (num_splits == 0)
        num_splits = tq4_decode_auto_splits(num_seqs, num_kv_heads, max_blocks_per_seq, block_size);
    if (num_splits > TQ4_MAX_SPLITS || !split_pages_ok(max_blocks_per_seq, block_size, num_splits))
        return TQ4_ERR_SPLITS;
    if ((uint64_t)num_seqs * num_kv_heads * num_splits > 0x7fffffffull) return TQ4_ERR_RANGE;
    tq4::DecodeParams p = make_params(q, key_cache, value_cache, scale_cache, block_tables,
                                      context_lens, pi_signs, gate, num_seqs, num_heads,
                                      num_kv_heads, head_size, block_size, num_blocks,
                                      max_blocks_per_seq, num_splits, scale, inv_sqrt_len,
                                      output_stage, flags);
    p.out = out;
    if (num_splits > 1) {
        const size_t need =
            tq4_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_size, num_splits);
        if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15u))
            return TQ4_ERR_WORKSPACE;
        p.records = (float*)workspace;
        // The tickets sit at the END of the workspace and the work-queue
        // counter just before them, so their place does not depend on
        // num_splits: a workspace zeroed once serves every split count.
        char* end = (char*)workspace + workspace_bytes;
        p.counters = (uint32_t*)(end - ticket_bytes(num_seqs, num_kv_heads));
        p.queue = (uint32_t*)(end - ticket_bytes(num_seqs, num_kv_heads) - kQueueBytes);
        p.timeouts = p.queue + 1;
    }
    return launched(tq4::launch_decode((hipStream_t)stream, p, 1));
}

int tq4_paged_decode_noalloc(void* stream, const uint16_t* q, const int8_t* key_cache,
                             const int8_t* value_cache, const float* scale_cache,
                             const int32_t* block_tables, const int32_t* context_lens,
                             const float* pi_signs, const float* gate, uint16_t* out,
                             uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                             uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                             uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                             float inv_sqrt_len, uint32_t output_stage, uint32_t flags)
{
    // Everything tq4_paged_decode refuses is refused here first, so a call
    // that would not fit the static scratch is refused before any HIP call.
    int rc = decode_checks(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                           pi_signs, num_seqs, num_heads, num_kv_heads, head_size, block_size,
                           num_blocks, max_blocks_per_seq, flags);
    if (rc != TQ4_OK) return rc;
    if (flags & ~TQ4_DECODE_QUERY_ROTATED) return TQ4_ERR_FLAGS;  // no test hooks here
    if (!out) return TQ4_ERR_NULL_POINTER;
    if (output_stage > 2 || (output_stage == 2 && !gate)) return TQ4_ERR_OUTPUT_STAGE;
    if (output_stage >= 1 && !pi_signs) return TQ4_ERR_ROTATION;
    if (num_splits == 0)
        num_splits = tq4_decode_auto_splits(num_seqs, num_kv_heads, max_blocks_per_seq, block_size);
    if (num_splits > TQ4_MAX_SPLITS || !split_pages_ok(max_blocks_per_seq, block_size, num_splits))
        return TQ4_ERR_SPLITS;
    if ((uint64_t)num_seqs * num_kv_heads * num_splits > 0x7fffffffull) return TQ4_ERR_RANGE;
    void* ws = nullptr;
    if (num_splits > 1) {
        if (tq4_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_size,
                                       num_splits) > tq4::kNoAllocScratchBytes)
            return TQ4_ERR_SCRATCH;
        if (tq4::noalloc_scratch(&ws) != hipSuccess) return TQ4_ERR_LAUNCH;
    }
    // The whole scratch is the workspace: its tail (queue, timeout word,
    // tickets) sits at the end whatever the geometry, and between calls
    // every word the decode uses is zero again, so calls of any geometry
    // can follow each other.
    return tq4_paged_decode(stream, q, key_cache, value_cache, scale_cache, block_tables,
                            context_lens, pi_signs, gate, ws, ws ? tq4::kNoAllocScratchBytes : 0,
                            out, num_seqs, num_heads, num_kv_heads, head_size, block_size,
                            num_blocks, max_blocks_per_seq, num_splits, scale, inv_sqrt_len,
                            output_stage, flags);
}

int tq4_paged_decode_noalloc_poll_timeouts(void* stream, uint32_t num_seqs,
                                           uint32_t num_kv_heads, uint32_t* count)
{
    if (!count) return TQ4_ERR_NULL_POINTER;
    if (num_seqs == 0 || num_kv_heads == 0) return TQ4_ERR_GEOMETRY;
    if (ticket_bytes(num_seqs, num_kv_heads) + kQueueBytes > tq4::kNoAllocScratchBytes)
        return TQ4_ERR_SCRATCH;
    void* ws = nullptr;
    if (tq4::noalloc_scratch(&ws) != hipSuccess) return TQ4_ERR_LAUNCH;
    return tq4_decode_poll_timeouts(stream, ws, tq4::kNoAllocScratchBytes, num_seqs, num_kv_heads,
                                    count);
}

int tq4_paged_decode_noalloc_reset(void* stream)
{
    void* ws = nullptr;
    if (tq4::noalloc_scratch(&ws) != hipSuccess) return TQ4_ERR_LAUNCH;
    return launched(tq4::launch_fill_zero((hipStream_t)stream, ws, tq4::kNoAllocScratchBytes));
}

int tq4_paged_decode_partials(void* stream, const uint16_t* q, const int8_t* key_cache,
                              const int8_t* value_cache, const float* scale_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              const float* pi_signs, float* workspace, size_t workspace_bytes,
                              uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                              uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                              float inv_sqrt_len, uint32_t flags)
{
    int rc = decode_checks(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                           pi_signs, num_seqs, num_heads, num_kv_heads, head_size, block_size,
                           num_blocks, max_blocks_per_seq, flags);
    if (rc != TQ4_OK) return rc;
    // no poll, no test hook
    if (flags & ~(TQ4_DECODE_QUERY_ROTATED | TQ4_DECODE_PRECISE)) return TQ4_ERR_FLAGS;
    if (num_splits == 0 || num_splits > TQ4_MAX_SPLITS ||
        !split_pages_ok(max_blocks_per_seq, block_size, num_splits))
        return TQ4_ERR_SPLITS;
    if ((uint64_t)num_seqs * num_kv_heads * num_splits > 0x7fffffffull) return TQ4_ERR_RANGE;
    // exactly the records [num_seqs][num_heads][num_splits][head_size + 4]
    // (the fused entry's size adds padding, tickets and counters)
    const size_t records =
        (size_t)num_seqs * num_heads * num_splits * (head_size + 4) * sizeof(float);
    if (!workspace || ((uintptr_t)workspace & 15u) || workspace_bytes < records)
        return TQ4_ERR_WORKSPACE;
    tq4::DecodeParams p = make_params(q, key_cache, value_cache, scale_cache, block_tables,
                                      context_lens, pi_signs, nullptr, num_seqs, num_heads,
                                      num_kv_heads, head_size, block_size, num_blocks,
                                      max_blocks_per_seq, num_splits, scale, inv_sqrt_len, 0,
                                      flags);
    p.records = workspace;
    if (flags & TQ4_DECODE_PRECISE)
        return launched(tq4::launch_decode_precise((hipStream_t)stream, p));
    return launched(tq4::launch_decode((hipStream_t)stream, p, 0));
}

int tq4_splitk_combine(void* stream, const float* workspace, const float* pi_signs,
                       const float* gate, uint16_t* out, uint32_t num_seqs, uint32_t num_heads,
                       uint32_t head_size, uint32_t num_splits, float inv_sqrt_len,
                       uint32_t output_stage)
{
    if (!head_size_ok(head_size)) return TQ4_ERR_HEAD_SIZE;
    if (num_seqs == 0 || num_heads == 0) return TQ4_ERR_GEOMETRY;
    if (num_splits == 0 || num_splits > TQ4_MAX_SPLITS) return TQ4_ERR_SPLITS;
    if (!workspace || !out) return TQ4_ERR_NULL_POINTER;
    if ((uintptr_t)workspace & 15u) return TQ4_ERR_WORKSPACE;
    if (output_stage > 2 || (output_stage == 2 && !gate)) return TQ4_ERR_OUTPUT_STAGE;
    if (output_stage >= 1 && !pi_signs) return TQ4_ERR_ROTATION;
    tq4::DecodeParams p{};
    p.records = const_cast<float*>(workspace);
    p.pi_signs = pi_signs;
    p.gate = gate;
    p.out = out;
    p.B = num_seqs;
    p.Hq = num_heads;
    p.D = head_size;
    p.K = num_splits;
    p.inv_sqrt_len = inv_sqrt_len;
    p.output_stage = output_stage;
    return launched(tq4::launch_combine((hipStream_t)stream, p));
}

}  // extern "C"

// ------------------------------------------------------------- RMS codec
extern "C" int tq4_rms_reshape_and_cache(void* stream, int type, uint32_t block_dim,
                                         const void* key, const void* value, int8_t* key_cache,
                                         int8_t* value_cache, float* scale_cache,
                                         const int32_t* slot_mapping, const float* pi_signs,
                                         const int32_t* tables, uint32_t num_tokens,
                                         uint32_t num_kv_heads, uint32_t head_size,
                                         uint32_t block_size, uint32_t num_blocks,
                                         uint32_t tokens_per_core, float inv_sqrt_len)
{
    (void)tables;  // the gather and centroid tables are built into the kernel
    if (type != 0 && type != 1) return TQ4_ERR_GEOMETRY;  // FP16 or BF16 activations
    if (!head_size_ok(head_size)) return TQ4_ERR_HEAD_SIZE;
    if (num_kv_heads == 0 || num_blocks == 0 || block_size == 0) return TQ4_ERR_GEOMETRY;
    // the reference's grid covers block_dim * tokens_per_core tokens
    uint64_t tokens = num_tokens;
    if (block_dim != 0 && (uint64_t)block_dim * tokens_per_core < tokens)
        tokens = (uint64_t)block_dim * tokens_per_core;
    if (tokens == 0) return TQ4_OK;
    if (!key || !value || !key_cache || !value_cache || !scale_cache || !slot_mapping ||
        !pi_signs)
        return TQ4_ERR_NULL_POINTER;
    if (tokens * 2u * num_kv_heads > 0x7fffffffull * 16u) return TQ4_ERR_RANGE;
    return launched(tq4::launch_rms_writer(
        (hipStream_t)stream, type, (const uint16_t*)key, (const uint16_t*)value, key_cache,
        value_cache, scale_cache, slot_mapping, pi_signs, (uint32_t)tokens, num_kv_heads,
        head_size, (uint64_t)num_blocks * block_size, inv_sqrt_len));
}

extern "C" int tq4_rms_dequantize(void* stream, const int8_t* packed, float* out, uint64_t n)
{
    if (n % 2) return TQ4_ERR_CODEBOOK;
    if (n == 0) return TQ4_OK;
    if (!packed || !out) return TQ4_ERR_NULL_POINTER;
    return launched(tq4::launch_rms_dequantize((hipStream_t)stream, packed, out, n / 2));
}

// ------------------------------------------------------------- codebooks
int tq4_icdf_quantize(void* stream, int in_bf16, const uint16_t* in, uint8_t* out, uint32_t tiles)
{
    if (tiles == 0) return TQ4_OK;
    if (!in || !out) return TQ4_ERR_NULL_POINTER;
    return launched(tq4::launch_icdf_quantize((hipStream_t)stream, in_bf16 ? 1 : 0, in, out,
                                              (uint64_t)tiles * 1024u));
}

int tq4_lloydmax_quantize(void* stream, const void* src, float* dst, uint8_t* codes,
                          uint32_t* guards, uint32_t bits, uint32_t mode, uint32_t n,
                          uint32_t rows)
{
    (void)guards;
    const uint64_t count = (uint64_t)n * rows;
    if ((bits != 2 && bits != 4) || mode > 5 || count % 8 || (mode == 3 && bits != 4))
        return TQ4_ERR_CODEBOOK;
    if (count == 0) return TQ4_OK;
    if (!src) return TQ4_ERR_NULL_POINTER;
    const hipStream_t st = (hipStream_t)stream;
    switch (mode) {
        case 0:
        case 1:
        case 2:
            if (!codes) return TQ4_ERR_NULL_POINTER;
            return launched(tq4::launch_codebook_quantize(st, mode == 2 ? 1u : 0u, bits,
                                                          (const float*)src, dst, codes, count));
        case 3:
            if (!codes) return TQ4_ERR_NULL_POINTER;
            return launched(
                tq4::launch_icdf_quantize(st, 0, (const uint16_t*)src, codes, count));
        default:
            if (!dst) return TQ4_ERR_NULL_POINTER;
            return launched(
                tq4::launch_codebook_dequantize(st, bits, (const uint8_t*)src, dst, count));
    }
}
