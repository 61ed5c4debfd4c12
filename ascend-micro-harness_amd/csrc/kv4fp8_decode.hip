// kv4fp8_decode.hip -- decode over the KV4/FP8 64-token NZ-tiled cache
// (include/tq4_kv4fp8.h) for gfx950.
//
// Reference: the "fused decode opt" operator,
// kernels/ops/turboquant/vllm_integration_layer/op_kernel/ (opk/ below):
// turboquant_fused_decode.cpp:479-568 (tasks), vector/turboquant_vector_service.h
// (query operand 1033-1058, tile softmax 594-679, partials 1181-1201, split
// reduce 253-320, normalise/cast 144-185), vector/routine_vector_cube_softmax.hpp
// (the batched tile recurrence), common/turboquant_codec_mx.h:289-359 (levels,
// FP8 operand cast), cube/turboquant_query_basis.h:181-208 (output stages).
//
// Work split. One workgroup = (token, kv head, 16-head chunk, part); part
// covers 4*nt consecutive 64-row tiles, wave w the w-th nt of them. Each wave
// runs the reference's tile recurrence over its tiles; the four waves merge
// in LDS. The parts holding the last four tickets of their (token, kv head,
// chunk) then merge the group's partial records (m, l, acc), a quarter of
// the rows each, in the same launch, and run the egress; the other parts
// only export records. A combiner waits only for parts that hold a ticket:
// an early combiner (not the last ticket) merges only if every ticket had
// been taken when it registered (every part has then started), else it hands
// its rows to the last ticket holder -- so no part ever waits on one that
// has not started, whatever the number of workgroups in flight. Tiles are the reference's tiles (64 aligned rows of
// the sequence), so the per-tile FP8 operands are the same; only the
// summation order of the merges differs.
//
// Operands on the f16 MFMA (16x16x32). Every FP8 e4m3 value and every level
// n + 0.5 is exact in f16, and their products are exact in FP32, so the f16
// MFMA computes the reference's FP8 products exactly:
//   scores  S[token][head] = K[token][k] . Q8[k][head]: A = key row (lane =
//           token, its 32-byte chunk of column group g), B = the query operand
//           in the same k order (lane = head);
//   context ctx^T[channel][head] = V^T[channel][k] . P8[k][head]: A = value
//           (lane = channel, 8 rows paired by v_perm), B = the lane's own
//           probabilities -- the k order is chosen as the score layout's row
//           order, so P needs no transpose.
// A level is fed as w = 1 + (n ^ 8)/64 (one v_bitop3 per pair, as the TQ4
// decode does), i.e. n + 0.5 = 64 (w - 1.1171875): scores start from
// -1.1171875 * sum(Q8) and are scaled by 64 with the key scale; the context's
// offset is tracked per head (B below) and removed at the end.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {
namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 64;
constexpr int kD = 256;
constexpr uint32_t kNib = 0x00F000F0u;       // a level at f16 mantissa bits [7:4], both halves
constexpr uint32_t kCodeBase = 0x3C803C80u;  // f16 1.0 outside kNib; the nibble sign bit inside
constexpr float kLevelOffset = 1.1171875f;   // w = 1.1171875 + (n + 0.5) / 64
constexpr float kLevelUnit = 64.0f;
constexpr float kOperandMax = 448.0f;        // OperandMax<KV4_FP8> (e4m3)
constexpr float kEps = 1e-20f;               // TurboQuantCodec4::kEps
constexpr float kNegInf = -3.4028235e38f;    // kVectorNegInf
constexpr float kGateFloor = -80.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr uint32_t kRecFloats = 260;         // acc[256], m, l, pad, pad
// LDS rows of 256 floats (q rows, merge rows) are kRow apart: the pad of one
// float4 puts eight consecutive rows' same columns on eight different bank
// quads, so the row-strided float4 accesses below are conflict-free (at kD
// apart they all hit one quad: the q prologue and the merge took 2.4 and
// 2.8 us at the reference shape, 1.9 and 1.4 us padded).
constexpr int kRow = kD + 4;
constexpr int kMergeFloats = kWaves * 16 * kRow;
constexpr int kScaleFloats = kWaves * 3 * kTile;
constexpr int kQopFloats = 8 * 64 * 4;  // 8 k-steps x 64 lanes x 8 f16

// Eight levels of one dword as f16 pairs, halves in nibble order 0,4,1,5,2,6,3,7:
// each pair is kNib ? (bits ^ kCodeBase) : kCodeBase (v_bitop3 0x6A).
__device__ __forceinline__ u4_t codes8(uint32_t w)
{
    return u4_t{(uint32_t)__builtin_amdgcn_bitop3_b32(w << 4, kNib, kCodeBase, 0x6A),
                (uint32_t)__builtin_amdgcn_bitop3_b32(w, kNib, kCodeBase, 0x6A),
                (uint32_t)__builtin_amdgcn_bitop3_b32(w >> 4, kNib, kCodeBase, 0x6A),
                (uint32_t)__builtin_amdgcn_bitop3_b32(w >> 8, kNib, kCodeBase, 0x6A)};
}

__device__ __forceinline__ f4_t mfma(u4_t a, h8_t b, f4_t c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), b, c, 0, 0, 0);
}

// Reductions over the four lanes l, l^16, l^32, l^48 (one head's lane column).
__device__ __forceinline__ float col_max(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t w = __float_as_uint(v);
    const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float col_sum(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const uint32_t w = __float_as_uint(v);
    const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Two FP32 values on the FP8 e4m3 grid (v_cvt_pk_fp8_f32: OCP e4m3, round to
// nearest even, subnormals kept), back to FP32 (v_cvt_pk_f32_fp8) and packed
// as f16 (exact: every e4m3 value is an f16 value, so the truncating pack
// does not round).
// Only the low word of the conversion is read, so its other word may come
// from any register: a's bits, rather than a zero to materialise.
__device__ __forceinline__ h2_t fp8_pair(float a, float b)
{
    const uint32_t w =
        (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
    const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(f[0], f[1]));
}

// The same, also handing back the two values in FP32 (equal to the f16
// halves).
__device__ __forceinline__ h2_t fp8_pair_f(float a, float b, float& fa, float& fb)
{
    const uint32_t w =
        (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
    const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    fa = f[0];
    fb = f[1];
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(f[0], f[1]));
}

__device__ __forceinline__ float elem_to_f32(uint16_t bits, uint32_t element)
{
    if (element) return __uint_as_float((uint32_t)bits << 16);
    return (float)__builtin_bit_cast(_Float16, bits);
}

__device__ __forceinline__ uint16_t f32_to_elem(float x, uint32_t element)
{
    if (element) {
        const uint32_t u = __float_as_uint(x);
        if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
        return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
    return __builtin_bit_cast(uint16_t, (_Float16)x);  // v_cvt_f16_f32: round to nearest even
}

// One stride of the Walsh-Hadamard butterfly across lanes (lane bit `m`):
// the lower lane keeps a + b, the upper b' = a - b (a = lower, b = upper).
__device__ __forceinline__ float wht_lanes(float v, int m, int lane)
{
    const float o = __shfl_xor(v, m, 64);
    return (lane & m) ? o - v : v + o;
}

// ApplyPi over one 256-channel row held four consecutive channels per lane.
__device__ __forceinline__ void apply_pi(float (&x)[4], const float (&s)[4], float inv_sqrt_len,
                                         int lane)
{
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = x[j] * s[j];
    {
        const float a0 = x[0] + x[1], a1 = x[0] - x[1], a2 = x[2] + x[3], a3 = x[2] - x[3];
        x[0] = a0 + a2;
        x[1] = a1 + a3;
        x[2] = a0 - a2;
        x[3] = a1 - a3;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = wht_lanes(x[j], m, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = x[j] * inv_sqrt_len;
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = x[j] * s[j];
}

// One tile's operands in registers.
struct Tile {
    u4_t k[8];        // key: token block tb's 32-byte chunk of column group g (k[2tb], k[2tb+1])
    uint2 v[16];      // value: rows 16tb + 4g + i (v[4tb + i]), packed columns 8m..8m+7
    float ks, vs;     // scales of row `lane`
    int ok;
};

// One part record (m, l, acc) into a row's running merge: the split reduce's
// recurrence, records taken in part order.
__device__ __forceinline__ void merge_record(float& run_max, float& run_sum, float (&x)[4],
                                             float m, float l, const float (&a)[4])
{
    const float new_max = fmaxf(run_max, m);
    const float alpha = fexp(run_max - new_max);
    const float beta = fexp(m - new_max);
    run_sum = run_sum * alpha;
    const float ps = l * beta;
    run_sum = run_sum + ps;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float u = x[i] * alpha;
        const float v = a[i] * beta;
        x[i] = u + v;
    }
    run_max = new_max;
}

// One wave, one (token, q head) row, lane = channels 4 lane .. 4 lane + 3:
// normalise the merged row, output stage, cast, store.
__device__ __forceinline__ void finish_row(const Kv4Params& p, uint32_t row, float (&x)[4],
                                           float run_sum, int lane)
{
    run_sum = run_sum + kEps;
    const float inv = 1.0f / run_sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = x[j] * inv;
    if (p.stage >= 1) {
        const float4 sg = *(const float4*)(p.pi_signs + 4 * lane);
        const float s[4] = {sg.x, sg.y, sg.z, sg.w};
        apply_pi(x, s, p.inv_sqrt_len, lane);
        if (p.stage == 2) {
            const uint2 gw = *(const uint2*)(p.gate + (size_t)row * kD + 4 * lane);
            const uint16_t gb[4] = {(uint16_t)gw.x, (uint16_t)(gw.x >> 16), (uint16_t)gw.y,
                                    (uint16_t)(gw.y >> 16)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float gv = elem_to_f32(gb[j], p.element);
                gv = fmaxf(gv, kGateFloor);
                float den = gv * -1.0f;
                den = fexp(den);
                den = den + 1.0f;
                x[j] = x[j] / den;
            }
        }
    }
    uint2 o;
    o.x = (uint32_t)f32_to_elem(x[0], p.element) | ((uint32_t)f32_to_elem(x[1], p.element) << 16);
    o.y = (uint32_t)f32_to_elem(x[2], p.element) | ((uint32_t)f32_to_elem(x[3], p.element) << 16);
    *(uint2*)(p.out + (size_t)row * kD + 4 * lane) = o;
}


constexpr uint32_t kRecBytes = kRecFloats * 4;
constexpr int kPollBatch = 16;  // records polled together (one round trip)
constexpr uint32_t kTicketMask = 0xFFFFu;  // counter word: tickets taken
constexpr uint32_t kRegShift = 16;         // counter word: early combiners registered

// The combiner's merge of one row: the records of parts 0 .. live-1 in part
// order, its own part's (`own`) from LDS and the others' polled from the
// workspace. A batch of records is reloaded until none of its words is zero
// (at most p.poll_limit times; a batch still incomplete then adds one to
// *p.timeouts), then zeroed for the next call.
__device__ __forceinline__ void combine_polled(const Kv4Params& p, uint32_t row, uint32_t live,
                                               uint32_t own, const float* own_acc,
                                               const float* own_ml, int lane, float (&x)[4],
                                               float& run_sum)
{
    const __amdgpu_buffer_rsrc_t rs =
        records_rsrc(p.records + (size_t)row * p.parts * kRecFloats);
    const float4 oa = *(const float4*)(own_acc + 4 * lane);
    const float2 om = *(const float2*)own_ml;
    float run_max = kNegInf;
    run_sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = 0.0f;
    // zero a batch's records for the next call
    auto zero_batch = [&](uint32_t k0) {
#pragma unroll
        for (int j = 0; j < kPollBatch; ++j) {
            const uint32_t k = k0 + j;
            if (k < live && k != own) {
                __builtin_amdgcn_raw_buffer_store_b128(rec_u4_t{0u, 0u, 0u, 0u}, rs,
                                                       k * kRecBytes + 16u * lane, 0,
                                                       kCachePolicySc1);
                if (lane == 0)
                    __builtin_amdgcn_raw_buffer_store_b64(rec_u2_t{0u, 0u}, rs,
                                                          k * kRecBytes + 4u * kD, 0,
                                                          kCachePolicySc1);
            }
        }
    };
    for (uint32_t k0 = 0; k0 < live; k0 += kPollBatch) {
        uint32_t aw[kPollBatch][4], hw[kPollBatch][2];
        for (uint32_t it = 0;; ++it) {
            asm volatile("" ::: "memory");  // every poll reloads
            // Every slot loads (past `live` the last record again, the own
            // slot its never-written words), so the loads carry no branches;
            // the check skips those slots.
#pragma unroll
            for (int j = 0; j < kPollBatch; ++j) {
                const uint32_t k = min(k0 + j, live - 1);
                rec_load<4, true>(rs, k * kRecBytes + 16u * lane, aw[j]);
                rec_load<2, true>(rs, k * kRecBytes + 4u * kD, hw[j]);
            }
            uint32_t mn = 0xffffffffu;
#pragma unroll
            for (int j = 0; j < kPollBatch; ++j) {
                const uint32_t k = k0 + j;
                const uint32_t w = min(min(hw[j][0], hw[j][1]),
                                       min(min(aw[j][0], aw[j][1]), min(aw[j][2], aw[j][3])));
                mn = k < live && k != own ? min(mn, w) : mn;
            }
            if (!__any(mn == 0u)) break;
            if (it + 1 >= p.poll_limit) {  // gave up: merged from what arrived
                if (lane == 0) count_timeout(p.timeouts);
                break;
            }
        }
        // the last batch is zeroed at once, earlier ones after the loop (a
        // later batch's poll would wait for their write acknowledgements)
        if (k0 + kPollBatch >= live) zero_batch(k0);
        // merge_record over the batch in part order, four slots at a time
        // and branch-free inside: the running maxima first, then each
        // record's weights and sums (the same operations on the same values
        // as record by record; slots past the live records select the running
        // values through), so the compiler interleaves the records'
        // independent work
        const uint32_t nb = min((uint32_t)kPollBatch, live - k0);
        float nm[kPollBatch];
        float prev = run_max;
#pragma unroll
        for (int j = 0; j < kPollBatch; ++j) {
            const float m = k0 + j == own ? om.x : __uint_as_float(hw[j][0] ^ kRecMagic);
            nm[j] = (uint32_t)j < nb ? fmaxf(prev, m) : prev;
            prev = nm[j];
        }
        float pm = run_max;
#pragma unroll
        for (int j4 = 0; j4 < kPollBatch; j4 += 4) {
            if ((uint32_t)j4 >= nb) break;
#pragma unroll
            for (int j = j4; j < j4 + 4; ++j) {
                const bool mine = k0 + j == own;
                const float m = mine ? om.x : __uint_as_float(hw[j][0] ^ kRecMagic);
                const float l = mine ? om.y : __uint_as_float(hw[j][1] ^ kRecMagic);
                float a[4];
                a[0] = mine ? oa.x : __uint_as_float(aw[j][0] ^ kRecMagic);
                a[1] = mine ? oa.y : __uint_as_float(aw[j][1] ^ kRecMagic);
                a[2] = mine ? oa.z : __uint_as_float(aw[j][2] ^ kRecMagic);
                a[3] = mine ? oa.w : __uint_as_float(aw[j][3] ^ kRecMagic);
                const float alpha = fexp(pm - nm[j]), beta = fexp(m - nm[j]);
                float rs = run_sum * alpha;
                const float ps = l * beta;
                rs = rs + ps;
                const bool in = (uint32_t)j < nb;
                run_sum = in ? rs : run_sum;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float u = x[i] * alpha;
                    const float v = a[i] * beta;
                    x[i] = in ? u + v : x[i];
                }
                pm = nm[j];
            }
        }
        run_max = prev;
    }
    for (uint32_t k0 = 0; k0 + kPollBatch < live; k0 += kPollBatch) zero_batch(k0);
}

// Two waves per SIMD (248 registers): one wave's VALU and MFMA work overlaps
// the other's; a three-deep ring at one wave per SIMD was 15 % slower.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void kv4_decode_kernel(Kv4Params p)
{
    extern __shared__ __align__(16) float lds[];
    float* merge = lds;                                  // [4][16][kRow] (q rows first)
    float* q_lds = lds;                                  // [16][kRow]
    float* ml = lds + kMergeFloats;                      // [4][16][2]
    int* role_lds = (int*)(ml + kWaves * 32);            // [4] this part's combine role
    float* mlo = ml + kWaves * 32 + 4;                   // [16][2] merged (m, l) per head
    h8_t* qop_lds = (h8_t*)(mlo + 32);                   // [8 k-steps][64 lanes] query operand
    float* sc_all = mlo + 32 + kQopFloats;               // [4][3][64]
    int32_t* win = (int32_t*)(sc_all + kScaleFloats);    // the part's block-table window

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    const uint32_t part = blockIdx.x;
    const uint32_t kvh = blockIdx.y / p.chunks, chunk = blockIdx.y % p.chunks;
    const uint32_t token = blockIdx.z;
    const uint32_t S = 1u << p.block_shift;

    int32_t ctx_raw = p.context_lens[token];
    uint32_t ctx = ctx_raw > 0 ? (uint32_t)ctx_raw : 0u;
    const uint64_t cap = (uint64_t)p.max_blocks << p.block_shift;
    if (ctx > cap) ctx = (uint32_t)cap;
    const uint32_t tiles = (ctx + kTile - 1) / kTile;
    const uint32_t t0 = part * kWaves * p.nt;
    const bool live = t0 < tiles;
    const uint32_t live_parts = (tiles + kWaves * p.nt - 1) / (kWaves * p.nt);
    // a part with no live tile leaves no record (every part counts the live
    // parts from ctx); part 0 still writes the rotated query back (raw-query
    // launch) and, when no part is live, the rows' zero context
    if (!live && part != 0) return;
    const uint32_t t1 = live ? min(t0 + kWaves * p.nt, tiles) : t0;
    const uint32_t head0 = chunk * 16;
    const uint32_t gc = min(16u, p.G - head0);  // live heads of this chunk

    // ---- phase 0: the block-table window and the chunk's query rows.
    const uint32_t page0 = (t0 * kTile) >> p.block_shift;
    const uint32_t npages = live ? (((t1 * kTile - 1) >> p.block_shift) - page0) + 1 : 0u;
    for (uint32_t i = tid; i < npages; i += kThreads)
        win[i] = p.block_table[(size_t)token * p.max_blocks + page0 + i];
    for (uint32_t h = wave; h < 16; h += kWaves) {
        float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const size_t row = (size_t)token * p.Hq + p.G * kvh + head0 + h;
        if (h < gc) {
            if (p.raw_query) {
                const uint2 w = *(const uint2*)(p.raw_query + row * kD + 4 * lane);
                x[0] = elem_to_f32((uint16_t)w.x, p.element);
                x[1] = elem_to_f32((uint16_t)(w.x >> 16), p.element);
                x[2] = elem_to_f32((uint16_t)w.y, p.element);
                x[3] = elem_to_f32((uint16_t)(w.y >> 16), p.element);
                const float4 sg = *(const float4*)(p.pi_signs + 4 * lane);
                const float s[4] = {sg.x, sg.y, sg.z, sg.w};
                apply_pi(x, s, p.inv_sqrt_len, lane);
                if (p.query_out && part == 0)
                    *(float4*)(p.query_out + row * kD + 4 * lane) = make_float4(x[0], x[1], x[2], x[3]);
            } else {
                const float4 v = *(const float4*)(p.query + row * kD + 4 * lane);
                x[0] = v.x;
                x[1] = v.y;
                x[2] = v.z;
                x[3] = v.w;
            }
        }
        *(float4*)(q_lds + h * kRow + 4 * lane) = make_float4(x[0], x[1], x[2], x[3]);
    }
    __syncthreads();
    const size_t row0 = (size_t)token * p.Hq + p.G * kvh + head0;  // the chunk's first row
    if (!live) {
        if (live_parts == 0) {  // part 0: no live tile, so every row's context is zero
            for (uint32_t h = wave; h < gc; h += kWaves) {
                float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                finish_row(p, row0 + h, x, 0.0f, lane);
            }
        }
        return;
    }

    // ---- this wave's tiles
    const uint32_t w0 = min(t0 + wave * p.nt, t1), w1 = min(w0 + p.nt, t1);
    float* sc = sc_all + wave * 3 * kTile;
    const uint32_t H = p.H;
    const uint32_t m8 = 8 * n16;  // this lane's packed value columns 8m..8m+7

    // Every fetch issues the same loads (an unmapped page reads page 0 and its
    // tile is masked), so the count of loads in flight behind a tile is fixed
    // and the compiler waits for exactly that tile's operands.
    auto fetch = [&](Tile& r, uint32_t t) {
        const uint32_t row_abs = t * kTile;
        int32_t e = win[(row_abs >> p.block_shift) - page0];
        r.ok = e >= 0 && (uint32_t)e < p.num_blocks;
        e = r.ok ? e : 0;
        const uint32_t rip = row_abs & (S - 1);
        const size_t base = ((size_t)(uint32_t)e * S + rip) * H * 128 + (size_t)kvh * (kTile * 128);
        const int8_t* kb = (const int8_t*)p.key + base;
        const int8_t* vb = (const int8_t*)p.value + base;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const u4_t* src = (const u4_t*)(kb + (g * kTile + 16 * tb + n16) * 32);
            r.k[2 * tb] = src[0];
            r.k[2 * tb + 1] = src[1];
        }
        const int8_t* vcol = vb + ((m8 >> 5) * kTile) * 32 + (m8 & 31);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i) r.v[4 * tb + i] = *(const uint2*)(vcol + (16 * tb + 4 * g + i) * 32);
        const float* srow = p.scales + ((size_t)(uint32_t)e * S + rip + lane) * 8;
        r.ks = srow[kvh];
        r.vs = srow[H + kvh];
    };

    // the first tile's loads go out before the query prologue
    Tile R0, R1;
    if (w0 < w1) fetch(R0, w0);
    // This part's ticket of its (token, kv head, chunk): the last R ticket
    // holders combine. Its round trip overlaps the tile loads; the value is
    // first needed at the merge.
    // The group's counter word: tickets count in its low 16 bits; an early
    // combiner (role r < R - 1) registers by adding 1 << (16 + r). The word
    // ends each call at `full`, and the atomic that makes it so resets it.
    uint32_t* counter = p.counters + ((size_t)token * p.H + kvh) * p.chunks + chunk;
    const uint32_t R = live_parts > 1 ? min(p.combiners, live_parts) : 1u;
    const uint32_t full = live_parts | (((1u << (R - 1)) - 1u) << kRegShift);
    uint32_t ticket_word = 0;
    if (live_parts > 1 && tid == 0)
        ticket_word =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- the query operand of head n16 for k group g: k-step ks covers the
    // dword d = 8g + ks of a key row, channels 4d + {0, 2, 128, 130, 1, 3, 129, 131}.
    float qv[8][8];
    float amax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        const int c0 = 4 * (8 * g + ks);
        const float* qr = q_lds + n16 * kRow;
        const float4 lo = *(const float4*)(qr + c0);
        const float4 hi = *(const float4*)(qr + 128 + c0);
        qv[ks][0] = lo.x; qv[ks][1] = lo.z; qv[ks][2] = hi.x; qv[ks][3] = hi.z;
        qv[ks][4] = lo.y; qv[ks][5] = lo.w; qv[ks][6] = hi.y; qv[ks][7] = hi.w;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(qv[ks][j]));
    }
    amax = col_max(amax);
    amax = amax + kEps;
    const float q_scale = kOperandMax / amax;
    const float q_inv = 1.0f / q_scale;
    h8_t qop[8];
    float q1 = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            float f0, f1;
            const h2_t h = fp8_pair_f(qv[ks][j] * q_scale, qv[ks][j + 1] * q_scale, f0, f1);
            qop[ks][j] = h[0];
            qop[ks][j + 1] = h[1];
            q1 += f0 + f1;  // (float)h[i] == f_i: every e4m3 value is an f16 value
        }
    }
    q1 = col_sum(q1);
    const float sbias = -kLevelOffset * q1;
    // one copy of the query operand for the four waves (identical in each)
    if (wave == 0) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qop_lds[ks * 64 + lane] = qop[ks];
    }
    __syncthreads();

    float run_max = kNegInf, run_sum = 0.0f, bsum = 0.0f, inv_prev = 1.0f;
    f4_t acc[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) acc[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const u4_t ones = u4_t{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};  // f16 1.0
    auto process = [&](const Tile& r, uint32_t t) {
        // rows of the tile that count; 0 for an unmapped page (the tile adds nothing)
        const uint32_t valid = r.ok ? min((uint32_t)kTile, ctx - t * kTile) : 0u;
        // per-row operands through the wave's LDS slot (row `lane` in, rows
        // 16tb + 4g .. out): key and value scales, and the row mask as an
        // additive bias -- 0 (x + 0 = x) or -inf, as the reference's Min with
        // its -2.5e36 mask leaves an exp of 0 -- with the dead rows' scales
        // zeroed so that no poisoned slot reaches the sums
        const bool live_row = (uint32_t)lane < valid;
        sc[lane] = live_row ? (r.ks * p.score_scale) * kLevelUnit : 0.0f;
        sc[kTile + lane] = live_row ? r.vs * p.inv_gain : 0.0f;
        sc[2 * kTile + lane] = live_row ? 0.0f : -INFINITY;
        // scores
        f4_t s4[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            f4_t c = f4_t{sbias, sbias, sbias, sbias};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const uint32_t w = ks < 4 ? r.k[2 * tb][ks] : r.k[2 * tb + 1][ks - 4];
                c = mfma(codes8(w), qop_lds[ks * 64 + lane], c);
            }
            s4[tb] = c;
        }
        float s[16], vsc[16];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const f4_t k4 = *(const f4_t*)(sc + 16 * tb + 4 * g);
            const f4_t v4 = *(const f4_t*)(sc + kTile + 16 * tb + 4 * g);
            const f4_t m4 = *(const f4_t*)(sc + 2 * kTile + 16 * tb + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = s4[tb][i] * k4[i];
                x = x * q_inv;
                s[4 * tb + i] = x + m4[i];
                vsc[4 * tb + i] = v4[i];
            }
        }
        float tmax = s[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) tmax = fmaxf(tmax, s[j]);
        tmax = col_max(tmax);  // -inf when no row counts: new_max stays run_max
        const float new_max = fmaxf(run_max, tmax);
        const float alpha = fexp(run_max - new_max);
        float part_sum = 0.0f, pmax = 0.0f;
        float pv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float e = fexp(s[j] - new_max);
            part_sum += e;
            pv[j] = e * vsc[j];
            pmax = fmaxf(pmax, pv[j]);
        }
        part_sum = col_sum(part_sum);
        run_sum = run_sum * alpha;
        run_sum = run_sum + part_sum;
        pmax = col_max(pmax);
        pmax = pmax + kEps;
        const float prob_scale = kOperandMax / pmax;
        h8_t pop[2];
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            const h2_t h = fp8_pair(pv[j] * prob_scale, pv[j + 1] * prob_scale);
            pop[j >> 3][j & 7] = h[0];
            pop[j >> 3][(j & 7) + 1] = h[1];
        }
        // acc holds acc_ref * prob_scale (this tile's units): rescale, then add
        // P8 . V. A tile that adds nothing keeps the previous units.
        const float rho = valid ? alpha * (prob_scale * inv_prev) : 1.0f;
#pragma unroll
        for (int b = 0; b < 16; ++b) acc[b] = acc[b] * rho;
        // sum(P8) per head on the matrix unit (an all-ones operand): the
        // context's level offset
        f4_t p1 = mfma(ones, pop[0], f4_t{0.0f, 0.0f, 0.0f, 0.0f});
        p1 = mfma(ones, pop[1], p1);
        bsum = bsum * rho;
        bsum = bsum + p1[0];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // row pairs (tb, i01), (tb, i23), (tb+1, i01), (tb+1, i23) of k-step ks;
            // columns (2q, 2q+1) of them feed blocks 2q, 2q + 1 (low nibbles:
            // channel 8m + b) and 8 + 2q, 9 + 2q (high: 128 + 8m + b - 8)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u4_t cv[4];
#pragma unroll
                for (int rp = 0; rp < 4; ++rp) {
                    const uint2 ra = r.v[4 * (2 * ks + (rp >> 1)) + 2 * (rp & 1)];
                    const uint2 rb = r.v[4 * (2 * ks + (rp >> 1)) + 2 * (rp & 1) + 1];
                    const uint32_t x = q < 2 ? ra.x : ra.y, y = q < 2 ? rb.x : rb.y;
                    cv[rp] = codes8(__builtin_amdgcn_perm(y, x, (q & 1) ? 0x07060302u : 0x05040100u));
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int b = (e & 1) * 8 + 2 * q + (e >> 1);
                    const u4_t a = u4_t{cv[0][e], cv[1][e], cv[2][e], cv[3][e]};
                    acc[b] = mfma(a, pop[ks], acc[b]);
                }
            }
        }
        inv_prev = valid ? 1.0f / prob_scale : inv_prev;
        run_max = new_max;
    };

    // The register ring: tile t+1 is in flight while t is processed (the
    // index is clamped, so the tail re-reads the last tile).
    if (w0 < w1) {
        const uint32_t last = w1 - 1;
        for (uint32_t t = w0;; t += 2) {
            fetch(R1, min(t + 1, last));
            process(R0, t);
            if (t + 1 > last) break;
            fetch(R0, min(t + 2, last));
            process(R1, t + 1);
            if (t + 2 > last) break;
        }
    }

    // An early combiner (tickets live - R .. live - 2) registers now; the
    // reply, read at the end of the merge, says whether every ticket had
    // been taken, i.e. every part of the group had started. The merge's
    // barriers are LDS-only, so the atomic stays in flight under it.
    const uint32_t ticket = ticket_word & kTicketMask;
    uint32_t reg_old = 0;
    if (R > 1 && tid == 0 && ticket >= live_parts - R && ticket < live_parts - 1) {
        const uint32_t reg = 1u << (kRegShift + ticket - (live_parts - R));
        reg_old = __hip_atomic_fetch_add(counter, reg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (reg_old + reg == full)
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- this wave's (m, l, acc): acc = (64 acc' - 71.5 B) / prob_scale_last
    const float off = bsum * (kLevelUnit * kLevelOffset);
    lds_barrier();  // every wave is past its q_lds reads
    float* mw = merge + wave * 16 * kRow + n16 * kRow;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float x = acc[4 * qd + j][i] * kLevelUnit;
                o[j] = (x - off) * inv_prev;
            }
            const int c = (qd < 2 ? 0 : 128) + 32 * g + 8 * i + 4 * (qd & 1);
            *(float4*)(mw + c) = make_float4(o[0], o[1], o[2], o[3]);
        }
    if (g == 0) {
        ml[(wave * 16 + n16) * 2] = run_max;
        ml[(wave * 16 + n16) * 2 + 1] = run_sum;
    }
    // Roles: the parts holding the last R tickets are combiners 0 .. R-1,
    // combiner r owning the rows h = r (mod R). The last ticket (role R-1)
    // also takes the rows of every early combiner whose registration came
    // before it (the registrations its own ticket's reply holds).
    if (tid == 0) {
        int role = live_parts > 1 ? -1 : 0;
        uint32_t mine = live_parts > 1 ? 0u : 1u;  // role classes this part combines
        if (live_parts > 1) {
            if (ticket >= live_parts - R) role = (int)(ticket - (live_parts - R));
            if (ticket_word + 1u == full)  // this ticket completes the word
                __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ticket == live_parts - 1)
                mine = (1u << (R - 1)) | ((ticket_word >> kRegShift) & ((1u << (R - 1)) - 1u));
        }
        role_lds[0] = role;
        role_lds[2] = (int)mine;
        // test hook: the first ticket's part withholds the records the other
        // combiners wait for
        role_lds[1] = p.withhold && live_parts > 1 && ticket == 0;
    }
    lds_barrier();

    // ---- merge the four waves: thread -> head tid / 16, channels 4 (tid % 16)
    // + 64 q4 (consecutive lanes on consecutive float4s). The merged row
    // replaces the wave-0 slice (each thread reads and writes only its own
    // channels of it); (M, L) go to mlo.
    const uint32_t h = tid >> 4, c0 = (tid & 15) * 4;
    if (h < gc) {
        float mwv[kWaves], M = kNegInf;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mwv[w] = ml[(w * 16 + h) * 2];
            M = fmaxf(M, mwv[w]);
        }
        float f[kWaves], L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            f[w] = fexp(mwv[w] - M);
            L += ml[(w * 16 + h) * 2 + 1] * f[w];
        }
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float4 x = *(const float4*)(merge + (w * 16 + h) * kRow + c0 + 64 * q4);
                o.x += x.x * f[w];
                o.y += x.y * f[w];
                o.z += x.z * f[w];
                o.w += x.w * f[w];
            }
            *(float4*)(merge + h * kRow + c0 + 64 * q4) = o;
        }
        if ((tid & 15) == 0) *(float2*)(mlo + 2 * h) = make_float2(M, L);
    }
    lds_barrier();
    const int role = *role_lds;

    // ---- one live part: its rows finish from LDS (the merge of one record)
    if (live_parts == 1) {
        for (uint32_t hh = wave; hh < gc; hh += kWaves) {
            const float4 a4 = *(const float4*)(merge + hh * kRow + 4 * lane);
            const float2 m2 = *(const float2*)(mlo + 2 * hh);
            const float a[4] = {a4.x, a4.y, a4.z, a4.w};
            float x[4] = {0.0f, 0.0f, 0.0f, 0.0f}, run_max = kNegInf, run_sum = 0.0f;
            merge_record(run_max, run_sum, x, m2.x, m2.y, a);
            finish_row(p, row0 + hh, x, run_sum, lane);
        }
        return;
    }

    // An early combiner merges its rows only if every ticket had been taken
    // when it registered; else it exports them too and leaves them to the
    // last ticket holder. Decided before the exports: the registration's
    // reply then waits behind no store.
    uint32_t mine = (uint32_t)role_lds[2];
    if (role >= 0 && role < (int)R - 1) {
        if (tid == 0) role_lds[3] = (reg_old & kTicketMask) == live_parts ? (int)(1u << role) : 0;
        lds_barrier();
        mine = (uint32_t)role_lds[3];
    }

    // ---- export the records of the rows other parts combine: encoded
    // (bits ^ kRecMagic, never 0) with device-coherent stores. Not exported:
    // the rows this part combines (a record it stored for a row it combines
    // would never be consumed and cleared).
    const bool withheld = role_lds[1] != 0;
    for (uint32_t hh = wave; hh < gc && !withheld; hh += kWaves) {
        if ((mine >> (hh % R)) & 1u) continue;
        const __amdgpu_buffer_rsrc_t rs =
            records_rsrc(p.records + (row0 + hh) * p.parts * kRecFloats);
        rec_store<4, true>(rs, part * kRecBytes + 16u * lane, merge + hh * kRow + 4 * lane);
        if (lane == 0) rec_store<2, true>(rs, part * kRecBytes + 4u * kD, mlo + 2 * hh);
    }
    if (mine == 0) return;

    // ---- the rows of the role classes in `mine` (class c: rows c, c + R,
    // ...), listed class by class; wave w takes rows w, w + 4, ... of the list
    for (uint32_t k = wave;; k += kWaves) {
        uint32_t hh = gc, rem = k;
        for (uint32_t c = 0; c < R; ++c) {
            if (!((mine >> c) & 1u)) continue;
            const uint32_t cnt = c < gc ? (gc - c + R - 1) / R : 0u;
            if (rem < cnt) {
                hh = c + R * rem;
                break;
            }
            rem -= cnt;
        }
        if (hh >= gc) break;
        float x[4], run_sum;
        combine_polled(p, row0 + hh, live_parts, part, merge + hh * kRow, mlo + 2 * hh, lane, x,
                       run_sum);
        finish_row(p, row0 + hh, x, run_sum, lane);
    }
}

// The FP8 e4m3 conversion pair the decode uses, exposed for the conversion test.
__global__ void fp8_probe_kernel(const float* in, uint16_t* out, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * i + 1 >= n) return;
    const h2_t h = fp8_pair(in[2 * i], in[2 * i + 1]);
    *(uint32_t*)(out + 2 * i) = __builtin_bit_cast(uint32_t, h);
}

}  // namespace

size_t kv4_lds_bytes(uint32_t npages)
{
    return (size_t)(kMergeFloats + kWaves * 32 + 4 + 32 + kQopFloats + kScaleFloats) *
               sizeof(float) +
           (size_t)npages * sizeof(int32_t);
}

hipError_t launch_kv4_decode(hipStream_t stream, const Kv4Params& p)
{
    const uint32_t npages = ((kWaves * p.nt * kTile - 1) >> p.block_shift) + 2;
    const dim3 grid(p.parts, p.H * p.chunks, p.T);
    const size_t lds = kv4_lds_bytes(npages);
    // Four combiners per group on any grid: a combiner waits only for parts
    // that hold a ticket (see the kernel's roles).
    Kv4Params q = p;
    q.combiners = 4;
    hipLaunchKernelGGL(kv4_decode_kernel, grid, dim3(kThreads), lds, stream, q);
    return hipGetLastError();
}

hipError_t launch_fp8_probe(hipStream_t stream, const float* in, uint16_t* out, uint32_t n)
{
    const uint32_t pairs = n / 2;
    if (pairs == 0) return hipSuccess;
    hipLaunchKernelGGL(fp8_probe_kernel, dim3((pairs + 255) / 256), dim3(256), 0, stream, in, out, n);
    return hipGetLastError();
}

}  // namespace tq4
