// tq4_internal.hpp -- launchers shared between the kernel translation units
// and the C ABI layer (tq4_abi.cpp). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tq4 {

hipError_t launch_strip_writer(hipStream_t stream, int in_bf16, const void* key,
                               const void* value, int8_t* key_cache, int8_t* value_cache,
                               float* scale_cache, const int32_t* slots, const float* pi_signs,
                               const void* tables, uint32_t strips, uint32_t H, uint32_t D,
                               uint32_t S, uint32_t P, float inv_sqrt_len);

hipError_t launch_scatter_writer(hipStream_t stream, uint32_t grid, const uint16_t* key,
                                 const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                                 float* scale_cache, const int32_t* slots, const float* pi_signs,
                                 const int32_t* cu_seqlens, int32_t* probe, uint32_t num_requests,
                                 uint32_t H, uint32_t D, uint32_t S, uint32_t P,
                                 uint32_t item_begin, uint32_t item_count, float inv_sqrt_len);

// Everything the decode kernels read; filled and validated by the ABI layer.
struct DecodeParams {
    const uint16_t* q;
    const int8_t* key_cache;
    const int8_t* value_cache;
    const float* scale_cache;
    const int32_t* block_tables;
    const int32_t* context_lens;
    const float* pi_signs;
    const float* gate;
    float* records;       // [B][Hq][K][D+4] partial records (may be null when K == 1 fused)
    uint32_t* counters;   // [B][Hkv] split tickets (fused only)
    uint32_t* queue;      // work-queue counter of the persistent fused kernel (or null)
    uint32_t* timeouts;   // fused: combined rows whose poll gave up (sticky count, or null)
    uint16_t* out;        // [B][Hq][D] bf16 (fused / combine)
    uint32_t B, Hq, Hkv, G, D, S, P, max_blocks, K;
    float scale, inv_sqrt_len;
    uint32_t output_stage, flags;
    uint32_t poll_limit;  // bound of a combiner's record polls
    uint32_t withhold;    // test hook: the first-ticket split of a group withholds its record
};

// mode 0: partials only; mode 1: fused (partials + last-workgroup combine).
hipError_t launch_decode(hipStream_t stream, const DecodeParams& p, int mode);
hipError_t launch_combine(hipStream_t stream, const DecodeParams& p);
// Partial records in the reference's FP32 operation order (tq4_precise.hip).
hipError_t launch_decode_precise(hipStream_t stream, const DecodeParams& p);
hipError_t launch_fill_zero(hipStream_t stream, void* ptr, size_t bytes);

// Codebook leaves (count = elements, a multiple of 8).
hipError_t launch_icdf_quantize(hipStream_t stream, int in_bf16, const uint16_t* in, uint8_t* out,
                                uint64_t count);
hipError_t launch_codebook_quantize(hipStream_t stream, uint32_t book, uint32_t bits,
                                    const float* src, float* recon, uint8_t* codes,
                                    uint64_t count);
hipError_t launch_codebook_dequantize(hipStream_t stream, uint32_t bits, const uint8_t* codes,
                                      float* recon, uint64_t count);

// The vllm-ascend RMS + threshold codec (tq4_rms.hip): the baseline writer
// over tokens [0, tokens), and the centroid decode of `bytes` packed bytes.
hipError_t launch_rms_writer(hipStream_t stream, int in_bf16, const uint16_t* key,
                             const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                             float* scale_cache, const int32_t* slots, const float* pi_signs,
                             uint32_t tokens, uint32_t H, uint32_t D, uint64_t slot_count,
                             float inv_sqrt_len);
hipError_t launch_rms_dequantize(hipStream_t stream, const int8_t* packed, float* out,
                                 uint64_t bytes);

// KV4/FP8 NZ-tiled decode (kv4fp8_decode.hip); filled by the ABI layer.
struct Kv4Params {
    const float* query;          // rotated FP32 [T][Hq][256] (pre-rotated entry)
    const uint16_t* raw_query;   // element bits [T][Hq][256] (raw-query entry) or null
    float* query_out;            // raw-query entry: the rotated query written back (or null)
    const uint8_t* key;
    const uint8_t* value;
    const float* scales;
    const int32_t* block_table;
    const int32_t* context_lens;
    const float* pi_signs;
    const uint16_t* gate;
    float* records;              // [T][Hq][parts][260], zero between calls
    uint32_t* counters;          // [T][H][chunks] part tickets, zero between calls
    uint32_t* timeouts;          // combined rows whose poll gave up (sticky count)
    uint32_t poll_limit;         // bound of a combiner's record polls
    uint32_t withhold;           // test hook: the first-ticket part withholds its records
    uint16_t* out;
    uint32_t T, Hq, H, G, chunks, block_shift, max_blocks, num_blocks, parts, nt;
    float score_scale, inv_gain, inv_sqrt_len;
    uint32_t stage, element;
    uint32_t combiners;          // set by launch_kv4_decode
};
hipError_t launch_kv4_decode(hipStream_t stream, const Kv4Params& p);
hipError_t launch_fp8_probe(hipStream_t stream, const float* in, uint16_t* out, uint32_t n);

// Byte offset of the counter region inside a workspace of K splits.
size_t decode_records_bytes(uint32_t B, uint32_t Hq, uint32_t D, uint32_t K);

// Words between consecutive split tickets (one 128-byte line each), and
// between the persistent kernel's work-queue counters (up to kSubQueues).
constexpr uint32_t kTicketStride = 32;
constexpr uint32_t kSubQueues = 4;

// The no-allocation decode's static scratch (tq4_decode.hip): its size, and
// its device address on the current device (looked up at the first call on
// each device; the array is zero at load).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
hipError_t noalloc_scratch(void** ptr);

}  // namespace tq4
