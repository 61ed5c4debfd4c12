// kv4fp8_abi.cpp -- the C ABI of the KV4/FP8 NZ-tiled decode (include/tq4_kv4fp8.h).
//
// Validation follows the reference's launchers: valid_launch
// (include/turboquant_fused_decode_opt.hpp:66-96) without its NPU grid <= 32
// bound, and the raw-query launcher's extra guards
// (vllm_integration_layer/op_kernel/turboquant_fused_decode.cpp:1240-1255:
// the prologue share covers every query vector, the Cube chunk is 0 or 16,
// the stage names a real stage), plus ascend_type_of's element check. A
// refusal returns a TQ4_ERR_* status and launches nothing.
#include <hip/hip_runtime.h>

#include "../../include/tq4.h"
#include "../../include/tq4_kv4fp8.h"
#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace {

constexpr uint32_t kTile = 64;
constexpr uint32_t kWaves = 4;
constexpr uint32_t kRecFloats = 260;
constexpr uint64_t kTargetWorkgroups = 512;  // two workgroups (eight waves) per CU
constexpr uint32_t kMaxWindowPages = 8192;

struct Plan {
    uint32_t chunks, parts, nt;
};

uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// The partition: parts of 4 * nt tiles (one nt per wave), enough of them to
// give about kTargetWorkgroups workgroups over the block tables' capacity.
Plan plan_of(const tq4_kv4fp8_launch* L)
{
    Plan p;
    const uint32_t group = L->heads / L->kv_heads;
    p.chunks = ceil_div(group, 16);
    const uint32_t tiles_cap = ceil_div((uint64_t)L->max_blocks * L->block_size, kTile);
    const uint64_t unit = (uint64_t)L->tokens * L->kv_heads * p.chunks;
    uint64_t parts = (kTargetWorkgroups + unit - 1) / unit;
    const uint64_t max_parts = ceil_div(tiles_cap, kWaves);
    if (parts > max_parts) parts = max_parts;
    if (parts < 1) parts = 1;
    p.nt = ceil_div(tiles_cap, kWaves * parts);
    const uint32_t nt_cap = kMaxWindowPages * (L->block_size / kTile) / kWaves;
    if (p.nt > nt_cap) p.nt = nt_cap;
    p.parts = ceil_div(tiles_cap, (uint64_t)kWaves * p.nt);
    return p;
}

bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

// valid_launch, less the grid bound; 0 or a status.
int geometry(const tq4_kv4fp8_launch* L)
{
    if (!L) return TQ4_ERR_NULL_POINTER;
    if (L->head_size != 256) return TQ4_ERR_HEAD_SIZE;
    if (!L->tokens || !L->kv_heads || L->kv_heads > 4 || !L->heads || L->heads % L->kv_heads ||
        !L->block_size || L->block_size % kTile || !pow2(L->block_size) || !L->max_blocks ||
        !L->heads_per_task || L->heads_per_task > 16 || !L->grid || !L->tasks_per_block ||
        !L->reduce_tasks_per_block || !L->num_blocks)
        return TQ4_ERR_GEOMETRY;
    if (!L->splits || L->splits > 8) return TQ4_ERR_SPLITS;
    const uint64_t group = L->heads / L->kv_heads;
    const uint64_t chunk = L->heads_per_task < group ? L->heads_per_task : group;
    const uint64_t tasks = (uint64_t)L->tokens * L->kv_heads * L->splits * ((group + chunk - 1) / chunk);
    const uint64_t rows = (uint64_t)L->tokens * L->heads;
    if (tasks > UINT32_MAX || (uint64_t)L->grid * L->tasks_per_block < tasks ||
        rows > UINT32_MAX || (uint64_t)L->grid * L->tasks_per_block > UINT32_MAX ||
        (uint64_t)L->grid * L->reduce_tasks_per_block > UINT32_MAX ||
        (uint64_t)L->grid * L->reduce_tasks_per_block < rows)
        return TQ4_ERR_GEOMETRY;
    if (L->element_type > 1) return TQ4_ERR_GEOMETRY;
    // tile rows are 32-bit in the kernels
    if ((uint64_t)L->max_blocks * L->block_size >= (1ull << 31)) return TQ4_ERR_RANGE;
    return TQ4_OK;
}

uint64_t round256(uint64_t b) { return (b + 255) & ~(uint64_t)255; }

// Workspace: the part ticket counter of every (token, kv head, chunk), then
// the partial records of every (token, q head, part); both all-zero between
// calls.
uint64_t counters_bytes(const tq4_kv4fp8_launch* L, const Plan& p)
{
    return round256((uint64_t)L->tokens * L->kv_heads * p.chunks * sizeof(uint32_t));
}

uint64_t records_bytes(const tq4_kv4fp8_launch* L, const Plan& p)
{
    return counters_bytes(L, p) +
           round256((uint64_t)L->tokens * L->heads * p.parts * kRecFloats * sizeof(float));
}

// ... then one 256-byte status block: word 0 the sticky poll-timeout count.
constexpr uint64_t kStatusBytes = 256;
uint64_t workspace_need(const tq4_kv4fp8_launch* L, const Plan& p)
{
    return records_bytes(L, p) + kStatusBytes;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int common_checks(const tq4_kv4fp8_launch* L, const tq4_kv4fp8_buffers* b, const Plan& plan)
{
    if (!b->key || !b->value || !b->scales || !b->block_table || !b->context_lengths ||
        !b->workspace || !b->output)
        return TQ4_ERR_NULL_POINTER;
    if (!aligned16(b->key) || !aligned16(b->value) || !aligned16(b->scales))
        return TQ4_ERR_GEOMETRY;
    if (!aligned16(b->workspace) || L->workspace_bytes < workspace_need(L, plan))
        return TQ4_ERR_WORKSPACE;
    // a group's tickets count in 16 bits of its counter word (at most
    // max_blocks / 8192 + 1024 parts arise; checked all the same)
    if (plan.parts > 0xFFFFu) return TQ4_ERR_GEOMETRY;
    if (L->test_flags & ~(uint32_t)(TQ4_KV4FP8_TEST_POLL_BOUND | TQ4_KV4FP8_TEST_WITHHOLD))
        return TQ4_ERR_FLAGS;
    if ((L->test_flags & TQ4_KV4FP8_TEST_WITHHOLD) && !(L->test_flags & TQ4_KV4FP8_TEST_POLL_BOUND))
        return TQ4_ERR_FLAGS;
    return TQ4_OK;
}

tq4::Kv4Params params_of(const tq4_kv4fp8_launch* L, const tq4_kv4fp8_buffers* b,
                         const Plan& plan)
{
    tq4::Kv4Params p{};
    p.query = (const float*)b->query;
    p.key = (const uint8_t*)b->key;
    p.value = (const uint8_t*)b->value;
    p.scales = (const float*)b->scales;
    p.block_table = (const int32_t*)b->block_table;
    p.context_lens = (const int32_t*)b->context_lengths;
    p.counters = (uint32_t*)b->workspace;
    p.records = (float*)((char*)b->workspace + counters_bytes(L, plan));
    p.timeouts = (uint32_t*)((char*)b->workspace + records_bytes(L, plan));
    p.poll_limit = (L->test_flags & TQ4_KV4FP8_TEST_POLL_BOUND) ? tq4::kPollLimitTest
                                                                 : tq4::kPollLimit;
    p.withhold = (L->test_flags & TQ4_KV4FP8_TEST_WITHHOLD) ? 1u : 0u;
    p.out = (uint16_t*)b->output;
    p.T = L->tokens;
    p.Hq = L->heads;
    p.H = L->kv_heads;
    p.G = L->heads / L->kv_heads;
    p.chunks = plan.chunks;
    p.block_shift = (uint32_t)__builtin_ctz(L->block_size);
    p.max_blocks = L->max_blocks;
    p.num_blocks = L->num_blocks;
    p.parts = plan.parts;
    p.nt = plan.nt;
    // scoreScale_ = scale / kGain, invGain_ = 1 / kGain (turboquant_vector_service.h:773-774)
    const float gain = 2.9832882881f;
    p.score_scale = L->scale / gain;
    p.inv_gain = 1.0f / gain;
    p.inv_sqrt_len = L->inv_sqrt_len;
    p.stage = 0;
    p.element = L->element_type;
    return p;
}

}  // namespace

extern "C" {

uint64_t tq4_kv4fp8_workspace_bytes(const tq4_kv4fp8_launch* launch)
{
    if (geometry(launch) != TQ4_OK) return 0;
    return workspace_need(launch, plan_of(launch));
}

int tq4_kv4fp8_poll_timeouts(void* stream, const tq4_kv4fp8_launch* launch,
                             const void* workspace, uint32_t* count)
{
    const int st = geometry(launch);
    if (st != TQ4_OK) return st;
    if (!workspace || !count) return TQ4_ERR_NULL_POINTER;
    const Plan plan = plan_of(launch);
    if (!aligned16(workspace) || launch->workspace_bytes < workspace_need(launch, plan))
        return TQ4_ERR_WORKSPACE;
    const char* word = (const char*)workspace + records_bytes(launch, plan);
    return hipMemcpyAsync(count, word, sizeof(uint32_t), hipMemcpyDefault,
                          (hipStream_t)stream) == hipSuccess
               ? TQ4_OK
               : TQ4_ERR_LAUNCH;
}

int tq4_kv4fp8_workspace_init(void* stream, void* workspace, uint64_t workspace_bytes)
{
    if (!workspace) return TQ4_ERR_NULL_POINTER;
    if (!aligned16(workspace)) return TQ4_ERR_WORKSPACE;
    return tq4::launch_fill_zero((hipStream_t)stream, workspace, workspace_bytes) == hipSuccess
               ? TQ4_OK
               : TQ4_ERR_LAUNCH;
}

int tq4_kv4fp8_decode(void* stream, const tq4_kv4fp8_launch* launch,
                      const tq4_kv4fp8_buffers* buffers)
{
    int st = geometry(launch);
    if (st != TQ4_OK) return st;
    if (!buffers || !buffers->query) return TQ4_ERR_NULL_POINTER;
    const Plan plan = plan_of(launch);
    if ((st = common_checks(launch, buffers, plan)) != TQ4_OK) return st;
    const tq4::Kv4Params p = params_of(launch, buffers, plan);
    return tq4::launch_kv4_decode((hipStream_t)stream, p) == hipSuccess ? TQ4_OK : TQ4_ERR_LAUNCH;
}

int tq4_kv4fp8_decode_raw_query(void* stream, const tq4_kv4fp8_launch* launch,
                                const tq4_kv4fp8_raw_query_buffers* buffers)
{
    int st = geometry(launch);
    if (st != TQ4_OK) return st;
    if (!buffers || !buffers->raw_query || !buffers->pi_signs) return TQ4_ERR_NULL_POINTER;
    if (launch->output_stage > 2 || (launch->output_stage == 2 && !buffers->gate))
        return TQ4_ERR_OUTPUT_STAGE;
    if ((launch->prologue_cube_chunk_vectors != 0 && launch->prologue_cube_chunk_vectors != 16) ||
        (uint64_t)launch->grid * launch->prologue_vectors_per_block <
            (uint64_t)launch->tokens * launch->heads)
        return TQ4_ERR_GEOMETRY;
    const Plan plan = plan_of(launch);
    if ((st = common_checks(launch, &buffers->decode, plan)) != TQ4_OK) return st;
    tq4::Kv4Params p = params_of(launch, &buffers->decode, plan);
    p.query = nullptr;
    p.raw_query = (const uint16_t*)buffers->raw_query;
    p.query_out = (float*)buffers->decode.query;
    p.pi_signs = (const float*)buffers->pi_signs;
    p.gate = (const uint16_t*)buffers->gate;
    p.stage = launch->output_stage;
    return tq4::launch_kv4_decode((hipStream_t)stream, p) == hipSuccess ? TQ4_OK : TQ4_ERR_LAUNCH;
}

int tq4_fp8_e4m3_round(void* stream, const float* in, uint16_t* out_f16, uint64_t n)
{
    if (!in || !out_f16) return TQ4_ERR_NULL_POINTER;
    if (n % 2 || n >= (1ull << 32)) return TQ4_ERR_RANGE;
    return tq4::launch_fp8_probe((hipStream_t)stream, in, out_f16, (uint32_t)n) == hipSuccess
               ? TQ4_OK
               : TQ4_ERR_LAUNCH;
}

}  // extern "C"
