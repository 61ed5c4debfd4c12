// tq4_writer.hip -- reshape_and_cache for the TQ4 cache on gfx950.
//
// Two kernels:
//   strip_writer     aligned 16-token strips (the reference's A8/BF16 prefill
//                    writers, turboquant_reshape_and_cache_{a8,bf16}.cpp)
//   scatter_writer   arbitrary slots per (request, kv_head) item, nibble-exact
//                    read-modify-write of the value strip
//                    (turboquant_reshape_scatter_aiv.cpp:598-731)
//
// Work decomposition (MI355X): one 256-lane workgroup owns one strip of one
// head, both planes: two panels of 16 rows x d channels, one row of each per
// 16-lane group (two independent row jobs per lane). A row lives on 16
// lanes with CPL = d/16 consecutive channels per lane, so the 16-point
// Hadamard stages below CPL are in-register and the rest are lane exchanges
// inside the row; a strip's 16 rows are the workgroup's 16 row groups.
// Activations load as one contiguous vector per lane (coalesced: a strip of
// a head is 16 rows of d elements, row stride H*d). Key rows store as one
// contiguous word per lane (token-major); the value strip is transposed
// through LDS and stored as d*8 contiguous bytes (channel-major).
//
// Bit-exactness: the rotation is adds and subtracts in the fixed stage order
// of the reference's Ingress cascade (rotate_butterfly_oracle.hpp:44-48), the
// scale is a power of two taken from the exponent field, y * 2^(2-e) is exact
// (ldexp), and the one rounding is v_rndne. This translation unit is built
// with -ffp-contract=off.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {
namespace {

constexpr int kWriterThreads = 256;  // 16 rows x 16 lanes

// Input element loads: CPL consecutive channels of one row.
template <int CPL>
__device__ __forceinline__ void load_row(const int8_t* src, float (&x)[CPL])
{
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = (float)src[j];
}

template <int CPL>
__device__ __forceinline__ void load_row(const uint16_t* src, float (&x)[CPL])
{
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = bf16_to_f32(src[j]);
}

// Signs for the lane's CPL channels: pi_signs when given (CPL consecutive
// floats, vector loads), else the first column of the reference's rotation
// tables (T[0][g][c0][0] = sign[g*32+c0]). The source is chosen once per
// launch (a uniform branch), never per channel.
template <int CPL>
__device__ __forceinline__ void load_signs(const float* pi_signs, const void* tables,
                                           int tables_bf16, int c0, float (&sign)[CPL])
{
    if (pi_signs != nullptr) {
        const float* src = pi_signs + c0;
        if constexpr (CPL % 4 == 0) {
#pragma unroll
            for (int j = 0; j < CPL; j += 4) {
                const float4 v = *(const float4*)(src + j);
                sign[j] = v.x;
                sign[j + 1] = v.y;
                sign[j + 2] = v.z;
                sign[j + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) sign[j] = src[j];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = c0 + j;
        if (tables_bf16) {
            const uint16_t raw = ((const uint16_t*)tables)[(size_t)c * 32];
            sign[j] = (raw & 0x8000u) ? -1.0f : 1.0f;
        } else {
            const int8_t raw = ((const int8_t*)tables)[(size_t)c * 32];
            sign[j] = raw < 0 ? -1.0f : 1.0f;
        }
    }
}

// Rotate one row, find its absmax over the 16 lanes of the row, quantise.
// q receives the INT4 codes, the return value is the stored scale.
template <int D, int CPL>
__device__ __forceinline__ float rotate_quantise(float (&v)[CPL], const float (&sign)[CPL],
                                                 int lane_in_row, float inv_sqrt_len, int policy,
                                                 int (&q)[CPL])
{
    rotate_ingress<D, CPL>(v, sign, lane_in_row);
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) a = fmaxf(a, fabsf(v[j]));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) a = fmaxf(a, xor_lanes(a, m));
    if (policy == kPolicyPrefill) {
        a = fmaxf(a, 1.0f);
    } else if (a == 0.0f) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) q[j] = 0;
        return 1.0f;
    }
    const int e = exponent_of(a);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        float r = rintf(ldexpf(v[j], 2 - e));
        r = fminf(r, 7.0f);
        q[j] = (int)r;
    }
    return ldexpf(1.0f, e - 2) * inv_sqrt_len;
}

// Pack CPL codes (low nibble first) into CPL/2 bytes and store them.
template <int CPL>
__device__ __forceinline__ void store_key_codes(int8_t* dst, const int (&q)[CPL])
{
    if constexpr (CPL == 16) {
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j / 8] |= ((uint32_t)q[j] & 0xfu) << (4 * (j % 8));
        *(uint2*)dst = make_uint2(w[0], w[1]);
    } else if constexpr (CPL == 8) {
        uint32_t w = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) w |= ((uint32_t)q[j] & 0xfu) << (4 * j);
        *(uint32_t*)dst = w;
    } else {
        static_assert(CPL == 4, "head_size 64, 128 or 256");
        uint32_t w = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) w |= ((uint32_t)q[j] & 0xfu) << (4 * j);
        *(uint16_t*)dst = (uint16_t)w;
    }
}

// ------------------------------------------------------------ strip writer
// grid.x = strips * (H / NH); a workgroup owns one strip of NH heads, both
// planes: every lane runs 2*NH independent row jobs (plane fastest), all of
// whose loads go out before the first rotation, and the launch has 2*NH
// times fewer waves to dispatch than one workgroup per (strip, head, plane).
template <int D, typename In, int NH>
__global__ __launch_bounds__(kWriterThreads) void strip_writer(
    const In* __restrict__ key, const In* __restrict__ value, int8_t* __restrict__ key_cache,
    int8_t* __restrict__ value_cache, float* __restrict__ scale_cache,
    const int32_t* __restrict__ slots, const float* __restrict__ pi_signs,
    const void* __restrict__ tables, int tables_bf16, uint32_t H, uint32_t S, uint32_t P,
    float inv_sqrt_len)
{
    constexpr int CPL = D / 16;
    constexpr int NJ = 2 * NH;
    constexpr int TS = 20;       // token stride of the transpose buffer, in words
    // per value job: [channel / 8][token, padded to TS] words of 8 channel
    // codes; 20-word rows put the 64 lanes of a wave (16 lanes x 4 tokens)
    // on distinct banks
    __shared__ __align__(16) uint32_t lds_t[NH][D / 8][TS];
    __shared__ __align__(16) int ok_w[kWriterThreads / 64];  // per-wave slot checks

    const uint32_t groups = H / NH;
    const uint32_t head0 = (blockIdx.x % groups) * NH;
    const uint32_t strip = blockIdx.x / groups;
    const int tid = threadIdx.x;
    const int row = tid >> 4;        // token within the strip
    const int lane_in_row = tid & 15;

    // The rows and the signs do not depend on the slots: their loads go out
    // together with the slot loads (one round trip, not two).
    float v[NJ][CPL], sign[CPL];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const In* src = ((j & 1) == 0 ? key : value) +
                        ((size_t)((size_t)strip * kStrip + row) * H + head0 + j / 2) * D +
                        lane_in_row * CPL;
        load_row<CPL>(src, v[j]);
    }
    load_signs<CPL>(pi_signs, tables, tables_bf16, lane_in_row * CPL, sign);

    // Slot contract for this strip: consecutive, strip-aligned, in range.
    const int32_t slot0 = slots[(size_t)strip * kStrip];
    const int32_t mine = slots[(size_t)strip * kStrip + row];
    const bool ok = slot0 >= 0 && (slot0 % kStrip) == 0 && mine == slot0 + row &&
                    (uint32_t)slot0 / S < P;
    // One barrier: every wave writes its own vote, so nothing needs clearing.
    static_assert(kWriterThreads == 256, "four wave votes");
    {
        const int wv = __all(ok);
        if ((tid & 63) == 0) ok_w[tid >> 6] = wv;
        __syncthreads();
        const int4 w4 = *(const int4*)ok_w;
        if (!(w4.x & w4.y & w4.z & w4.w)) return;
    }
    const uint32_t page = (uint32_t)slot0 / S;
    const uint32_t tip = (uint32_t)slot0 % S + (uint32_t)row;
    int q[NJ][CPL];
    float scale[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        scale[j] = rotate_quantise<D, CPL>(v[j], sign, lane_in_row, inv_sqrt_len, kPolicyPrefill,
                                           q[j]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t plane = j & 1, head = head0 + j / 2;
        const size_t head_base = ((size_t)page * H + head) * S;  // in tokens
        if (lane_in_row == 0) scale_cache[(((size_t)plane * P + page) * H + head) * S + tip] = scale[j];
        if (plane == 0) {
            store_key_codes<CPL>(key_cache + (head_base + tip) * (D / 2) + lane_in_row * (CPL / 2),
                                 q[j]);
        } else {
            // value plane: this token's codes of 8 channels per word, into
            // the transpose buffer (one 32-bit LDS store per word; at d = 64
            // two lanes share a word, a 16-bit store each)
            if constexpr (CPL >= 8) {
#pragma unroll
                for (int k = 0; k < CPL / 8; ++k) {
                    uint32_t w = 0;
#pragma unroll
                    for (int c = 0; c < 8; ++c) w |= ((uint32_t)q[j][8 * k + c] & 0xfu) << (4 * c);
                    lds_t[j / 2][lane_in_row * (CPL / 8) + k][row] = w;
                }
            } else {
                uint32_t w = 0;
#pragma unroll
                for (int c = 0; c < CPL; ++c) w |= ((uint32_t)q[j][c] & 0xfu) << (4 * c);
                ((uint16_t*)&lds_t[j / 2][lane_in_row >> 1][row])[lane_in_row & 1] = (uint16_t)w;
            }
        }
    }
    __syncthreads();
    // ... then each value strip leaves as d*8 contiguous bytes: output word
    // (channel, half) holds that channel's codes of tokens 8*half .. +7, one
    // nibble from each of 8 consecutive buffer words (two 16-byte reads)
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const size_t head_base = ((size_t)page * H + head0 + h) * S;
        uint32_t* strip_words =
            (uint32_t*)(value_cache + (head_base + (tip & ~(uint32_t)15)) * (D / 2));
        for (int w = tid; w < D * 2; w += kWriterThreads) {
            const int channel = w >> 1, half = w & 1;
            const uint32_t* src = &lds_t[h][channel >> 3][8 * half];
            const uint4 a = *(const uint4*)src;
            const uint4 b = *(const uint4*)(src + 4);
            const uint32_t t8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            const uint32_t sh = 4u * (uint32_t)(channel & 7);
            uint32_t out = 0;
#pragma unroll
            for (int t = 0; t < 8; ++t) out |= ((t8[t] >> sh) & 0xfu) << (4 * t);
            strip_words[w] = out;
        }
    }
}

// ----------------------------------------------------------- scatter writer
// One workgroup walks items item_begin + blockIdx.x, += gridDim.x. Inside an
// item the tokens are grouped into runs of consecutive slots inside one strip
// (at most 16), exactly the reference's transaction unit.
template <int D>
__global__ __launch_bounds__(kWriterThreads) void scatter_writer(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    int8_t* __restrict__ key_cache, int8_t* __restrict__ value_cache,
    float* __restrict__ scale_cache, const int32_t* __restrict__ slots,
    const float* __restrict__ pi_signs, const int32_t* __restrict__ cu_seqlens,
    int32_t* __restrict__ probe, uint32_t num_requests, uint32_t H, uint32_t S, uint32_t P,
    uint32_t item_begin, uint32_t item_count, float inv_sqrt_len)
{
    constexpr int CPL = D / 16;
    __shared__ uint32_t lds_codes[D * kStrip / 4];
    const int tid = threadIdx.x;
    const int row = tid >> 4;
    const int lane_in_row = tid & 15;

    if (probe != nullptr && blockIdx.x == 0 && tid < 32) {
        const int32_t fields[4] = {0, (int32_t)gridDim.x, 1, (int32_t)item_count};
        probe[tid] = fields[tid >> 3];
    }

    float sign[CPL];
    load_signs<CPL>(pi_signs, nullptr, 0, lane_in_row * CPL, sign);
    const uint64_t item_end = (uint64_t)item_begin + item_count;

    for (uint64_t item = (uint64_t)item_begin + blockIdx.x; item < item_end; item += gridDim.x) {
        const uint32_t request = (uint32_t)(item / H);
        const uint32_t head = (uint32_t)(item % H);
        if (request >= num_requests) continue;
        uint32_t token = cu_seqlens ? (uint32_t)cu_seqlens[request] : request;
        const uint32_t token_end = cu_seqlens ? (uint32_t)cu_seqlens[request + 1] : request + 1;

        while (token < token_end) {
            // Run discovery, computed identically by every lane (uniform).
            const int32_t slot0 = slots[token];
            if (slot0 < 0 || (uint32_t)slot0 / S >= P) {
                ++token;
                continue;
            }
            const uint32_t page = (uint32_t)slot0 / S;
            const uint32_t tip0 = (uint32_t)slot0 % S;
            const uint32_t strip_in_page = tip0 / kStrip;
            uint32_t run = 1;
            while (token + run < token_end && run < (uint32_t)kStrip) {
                const int32_t next = slots[token + run];
                if (next != slot0 + (int32_t)run) break;
                if ((uint32_t)next / S != page || ((uint32_t)next % S) / kStrip != strip_in_page) break;
                ++run;
            }
            const bool live = (uint32_t)row < run;
            const uint32_t tok = token + (live ? (uint32_t)row : 0u);
            const size_t head_base = ((size_t)page * H + head) * S;

            for (uint32_t plane = 0; plane < 2; ++plane) {
                const uint16_t* src = (plane == 0 ? key : value) +
                                      ((size_t)tok * H + head) * D + lane_in_row * CPL;
                float v[CPL];
                load_row<CPL>(src, v);
                int q[CPL];
                const float scale =
                    rotate_quantise<D, CPL>(v, sign, lane_in_row, inv_sqrt_len, kPolicyExact, q);
                const uint32_t tip = tip0 + (uint32_t)row;
                if (live && lane_in_row == 0)
                    scale_cache[(((size_t)plane * P + page) * H + head) * S + tip] = scale;
                if (plane == 0) {
                    if (live)
                        store_key_codes<CPL>(
                            key_cache + (head_base + tip) * (D / 2) + lane_in_row * (CPL / 2), q);
                    continue;
                }
                // Value plane: codes to LDS at their strip column, then merge
                // only the owned nibbles into the words they live in.
                uint8_t* lds = (uint8_t*)lds_codes;
                const uint32_t col = (tip0 % kStrip) + (uint32_t)row;
                if (live) {
#pragma unroll
                    for (int j = 0; j < CPL; ++j)
                        lds[(lane_in_row * CPL + j) * kStrip + col] = (uint8_t)(q[j] & 0xf);
                }
                __syncthreads();
                const uint32_t first = tip0 % kStrip, last = first + run;  // owned columns
                uint32_t* strip_words =
                    (uint32_t*)(value_cache + (head_base + strip_in_page * kStrip) * (D / 2));
                for (int w = tid; w < D * 2; w += kWriterThreads) {
                    const int channel = w >> 1, half = w & 1;
                    const uint32_t t0 = (uint32_t)half * 8u;
                    const uint32_t lo = first > t0 ? first : t0;
                    const uint32_t hi = last < t0 + 8u ? last : t0 + 8u;
                    if (lo >= hi) continue;
                    uint32_t mask = 0u, bits = 0u;
                    for (uint32_t t = lo; t < hi; ++t) {
                        const uint32_t sh = 4u * (t - t0);
                        mask |= 0xfu << sh;
                        bits |= (uint32_t)lds[channel * kStrip + t] << sh;
                    }
                    strip_words[w] = (strip_words[w] & ~mask) | bits;
                }
                __syncthreads();
            }
            token += run;
        }
    }
}

// One-token requests (cu_seqlens NULL: the decode step's writer). A 16-lane
// row group takes one (token, kv head) item, sixteen items per workgroup;
// each lane rotates and quantises its channels of both planes. The value
// strip's column is merged in registers: a lane reads the 2 CPL consecutive
// strip words of its channels (channel c's 16 tokens are words 2c and
// 2c + 1), replaces its nibble in each and writes the words back. A strip
// has one owner per launch (the writer's contract), so writing back the
// words read is safe. The rows' loads go out with the slot's; the strip's
// load follows the slot.
template <int D>
__global__ __launch_bounds__(kWriterThreads) void scatter_token_writer(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    int8_t* __restrict__ key_cache, int8_t* __restrict__ value_cache,
    float* __restrict__ scale_cache, const int32_t* __restrict__ slots,
    const float* __restrict__ pi_signs, int32_t* __restrict__ probe, uint32_t probe_grid,
    uint32_t num_requests, uint32_t H, uint32_t S, uint32_t P, uint32_t item_begin,
    uint32_t item_count, float inv_sqrt_len)
{
    constexpr int CPL = D / 16;
    constexpr int NW = 2 * CPL;  // strip words of a lane's channels
    const int tid = threadIdx.x;
    const int grp = tid >> 4;
    const int lane_in_row = tid & 15;

    if (probe != nullptr && blockIdx.x == 0 && tid < 32) {
        const int32_t fields[4] = {0, (int32_t)probe_grid, 1, (int32_t)item_count};
        probe[tid] = fields[tid >> 3];
    }

    float sign[CPL];
    load_signs<CPL>(pi_signs, nullptr, 0, lane_in_row * CPL, sign);
    const uint64_t item_end = (uint64_t)item_begin + item_count;
    for (uint64_t item = (uint64_t)item_begin + (uint64_t)blockIdx.x * 16u + (uint32_t)grp;
         item < item_end; item += (uint64_t)gridDim.x * 16u) {
        const uint32_t request = (uint32_t)(item / H);
        const uint32_t head = (uint32_t)(item % H);
        if (request >= num_requests) continue;
        // The rows do not depend on the slot: their loads go out with its
        // load. A pad or out-of-pool slot reads page 0's strip and stores
        // nothing (so no load waits behind a branch).
        const size_t src_off = ((size_t)request * H + head) * D + lane_in_row * CPL;
        const int32_t slot = slots[request];
        float kx[CPL], vx[CPL];
        load_row<CPL>(key + src_off, kx);
        load_row<CPL>(value + src_off, vx);
        const bool ok = slot >= 0 && (uint32_t)slot / S < P;
        const uint32_t page = ok ? (uint32_t)slot / S : 0u;
        const uint32_t tip = ok ? (uint32_t)slot % S : 0u;
        const uint32_t col = tip % kStrip;
        const size_t head_base = ((size_t)page * H + head) * S;
        uint4* strip = (uint4*)(value_cache + (head_base + (tip - col)) * (D / 2)) +
                       lane_in_row * (NW / 4);
        uint32_t w[NW];
#pragma unroll
        for (int i = 0; i < NW / 4; ++i) {
            const uint4 u = strip[i];
            w[4 * i] = u.x;
            w[4 * i + 1] = u.y;
            w[4 * i + 2] = u.z;
            w[4 * i + 3] = u.w;
        }
        int qk[CPL], qv[CPL];
        const float sk = rotate_quantise<D, CPL>(kx, sign, lane_in_row, inv_sqrt_len,
                                                 kPolicyExact, qk);
        const float sv = rotate_quantise<D, CPL>(vx, sign, lane_in_row, inv_sqrt_len,
                                                 kPolicyExact, qv);
        if (!ok) continue;
        if (lane_in_row == 0) {
            scale_cache[((size_t)page * H + head) * S + tip] = sk;
            scale_cache[(((size_t)P + page) * H + head) * S + tip] = sv;
        }
        store_key_codes<CPL>(key_cache + (head_base + tip) * (D / 2) + lane_in_row * (CPL / 2),
                             qk);
        const uint32_t sh = 4u * (col & 7u), half = col >> 3;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            uint32_t& x = w[2 * j + half];
            x = (x & ~(0xfu << sh)) | (((uint32_t)qv[j] & 0xfu) << sh);
        }
#pragma unroll
        for (int i = 0; i < NW / 4; ++i)
            strip[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    }
}

}  // namespace

// ------------------------------------------------------------- launchers
template <int D, typename In>
static hipError_t launch_strip_writer_t(hipStream_t stream, const In* key, const In* value,
                                        int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                                        const int32_t* slots, const float* pi_signs,
                                        const void* tables, int tables_bf16, uint32_t strips,
                                        uint32_t H, uint32_t S, uint32_t P, float inv_sqrt_len)
{
    // One head per workgroup (two row jobs per lane) measured faster than
    // two (four jobs): with one wave per SIMD nothing hides the rotation's
    // dependent lane exchanges.
    const uint64_t blocks = (uint64_t)strips * H;
    hipLaunchKernelGGL((strip_writer<D, In, 1>), dim3((uint32_t)blocks), dim3(kWriterThreads), 0,
                       stream, key, value, key_cache, value_cache, scale_cache, slots, pi_signs,
                       tables, tables_bf16, H, S, P, inv_sqrt_len);
    return hipGetLastError();
}

hipError_t launch_strip_writer(hipStream_t stream, int in_bf16, const void* key,
                               const void* value, int8_t* key_cache, int8_t* value_cache,
                               float* scale_cache, const int32_t* slots, const float* pi_signs,
                               const void* tables, uint32_t strips, uint32_t H, uint32_t D,
                               uint32_t S, uint32_t P, float inv_sqrt_len)
{
#define TQ4_STRIP_CASE(DD)                                                                        \
    if (D == DD) {                                                                                \
        if (in_bf16)                                                                              \
            return launch_strip_writer_t<DD, uint16_t>(                                           \
                stream, (const uint16_t*)key, (const uint16_t*)value, key_cache, value_cache,     \
                scale_cache, slots, pi_signs, tables, 1, strips, H, S, P, inv_sqrt_len);          \
        return launch_strip_writer_t<DD, int8_t>(stream, (const int8_t*)key, (const int8_t*)value, \
                                                 key_cache, value_cache, scale_cache, slots,      \
                                                 pi_signs, tables, 0, strips, H, S, P,            \
                                                 inv_sqrt_len);                                   \
    }
    TQ4_STRIP_CASE(64)
    TQ4_STRIP_CASE(128)
    TQ4_STRIP_CASE(256)
#undef TQ4_STRIP_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_scatter_writer(hipStream_t stream, uint32_t grid, const uint16_t* key,
                                 const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                                 float* scale_cache, const int32_t* slots, const float* pi_signs,
                                 const int32_t* cu_seqlens, int32_t* probe, uint32_t num_requests,
                                 uint32_t H, uint32_t D, uint32_t S, uint32_t P,
                                 uint32_t item_begin, uint32_t item_count, float inv_sqrt_len)
{
    // one-token requests: sixteen items per workgroup, a grid covering them
    // (at most 4096 workgroups, striding beyond); `grid` is still what the
    // launch probe reports
    const uint64_t groups = ((uint64_t)item_count + 15) / 16;
    const uint32_t tgrid = (uint32_t)(groups < 4096 ? groups : 4096);
#define TQ4_SCATTER_CASE(DD)                                                                      \
    if (D == DD) {                                                                                \
        if (cu_seqlens == nullptr)                                                                \
            hipLaunchKernelGGL((scatter_token_writer<DD>), dim3(tgrid), dim3(kWriterThreads), 0, \
                               stream, key, value, key_cache, value_cache, scale_cache, slots,    \
                               pi_signs, probe, grid, num_requests, H, S, P, item_begin,          \
                               item_count, inv_sqrt_len);                                         \
        else                                                                                      \
            hipLaunchKernelGGL((scatter_writer<DD>), dim3(grid), dim3(kWriterThreads), 0, stream, \
                               key, value, key_cache, value_cache, scale_cache, slots, pi_signs,  \
                               cu_seqlens, probe, num_requests, H, S, P, item_begin, item_count,  \
                               inv_sqrt_len);                                                     \
        return hipGetLastError();                                                                 \
    }
    TQ4_SCATTER_CASE(64)
    TQ4_SCATTER_CASE(128)
    TQ4_SCATTER_CASE(256)
#undef TQ4_SCATTER_CASE
    return hipErrorInvalidValue;
}

}  // namespace tq4
