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
// The strip writer's row order and arithmetic, tuned for the VALU issue rate
// (with two waves per SIMD the writer's rotation, quantisation and packing
// are issue-bound, four cycles per wave64 instruction):
//
// * Lane order and butterflies: the row lane order of tq4_device.hpp
//   (row_lane), where every cross-lane stride is one DPP pattern, and the
//   sign-tracked butterfly (row_fmac_stage): one DPP-fed v_fmac_f32 per
//   element and stage.
// * Quantiser. t = fma(y, 2^(2-e), kQMagic) with kQMagic = 1.5 * 2^23 + 8:
//   y * 2^(2-e) is exact and |y * 2^(2-e)| < 8, so the one rounding of the
//   sum is the round-to-nearest-even of y * 2^(2-e) (kQMagic is even: ties
//   keep their parity), and t = kQMagic + n exactly; min(t, kQMagic + 7) is
//   the clamp at 7. Bits 0..3 of t then hold n + 8 and bits 4..7 are zero,
//   so codes pack with one shift-or per pair and byte permutes, and the
//   packed word is XORed with 0x8...8 to give the two's-complement nibbles.
//   Non-finite inputs saturate: +inf and NaN give 7, -inf gives -8.
// * One barrier: the slot vote and the value-strip transpose share it. The
//   slot loads go out first, ahead of the rows they do not depend on, so
//   their round trip is the rows' round trip.

constexpr float kQMagic = 12582920.0f;     // 1.5 * 2^23 + 8
constexpr float kQMagicTop = 12582927.0f;  // kQMagic + 7

// One butterfly stage over the writer's two rows (key, value), l being this
// lane's logical lane: in registers below CPL, else row_fmac_stage on the
// sign-tracked values.
template <int CPL>
__device__ __forceinline__ void writer_butterfly(float (&v)[2][CPL], int stride, int l)
{
    if (stride < CPL) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (j & stride) continue;
                const float a = v[r][j];
                const float b = v[r][j + stride];
                v[r][j] = b + a;
                v[r][j + stride] = a - b;
            }
        }
    } else {
        const int k = __builtin_ctz(stride / CPL);
        const float c = ((l >> k) & 1) ? -1.0f : 1.0f;
        row_fmac_stage<CPL>(v[0], c, k);
        row_fmac_stage<CPL>(v[1], c, k);
    }
}

// Rotate both rows (strides 1..16, the sign diagonal, 32..D/2). The results
// are held as sigma * v with sigma = (-1)^popcount(l) (row_sigma).
template <int D, int CPL>
__device__ __forceinline__ void writer_rotate(float (&v)[2][CPL], const float (&sign)[CPL], int l)
{
#pragma unroll
    for (int s = 1; s < 32 && s < D; s <<= 1) writer_butterfly<CPL>(v, s, l);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[r][j] *= sign[j];
    }
#pragma unroll
    for (int s = 32; s < D; s <<= 1) writer_butterfly<CPL>(v, s, l);
}

// Each row's absmax over its 16 lanes, starting from `floor` (1.0 for the
// prefill policy, 0 for the exact one).
template <int CPL>
__device__ __forceinline__ void writer_absmax(const float (&v)[2][CPL], float floor, float (&a)[2])
{
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        a[r] = floor;
#pragma unroll
        for (int j = 0; j < CPL; ++j) a[r] = fmaxf(a[r], fabsf(v[r][j]));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) row_max2(a[0], a[1], k);
}

// Rotate both rows, take each row's absmax (prefill policy: floored at 1.0)
// and quantise: t[r][j] receives kQMagic + code as bits; scale[r] is the
// row's stored scale.
template <int D, int CPL>
__device__ __forceinline__ void writer_rotate_quantise(float (&v)[2][CPL], const float (&sign)[CPL],
                                                       int l, float inv_sqrt_len,
                                                       uint32_t (&t)[2][CPL], float (&scale)[2])
{
    writer_rotate<D, CPL>(v, sign, l);
    float a[2];
    writer_absmax<CPL>(v, 1.0f, a);
    // the stored values are sigma * v: the quantiser's exact power of two
    // carries sigma
    const float sigma = row_sigma(l);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        // a >= 1 (the prefill floor; NaN never wins fmaxf): the exponent
        // field alone, 0 .. 128 (128: infinity); 2^(2-e) is a normal float
        const int e = (int)(__float_as_uint(a[r]) >> 23) - 127;
        const float p2 = sigma * ldexpf(1.0f, 2 - e);
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            t[r][j] = __float_as_uint(fminf(__builtin_fmaf(v[r][j], p2, kQMagic), kQMagicTop));
        scale[r] = ldexpf(1.0f, e - 2) * inv_sqrt_len;
    }
}

// Eight codes (t[k] bits 0..3 = code + 8, bits 4..7 zero) as one word of
// signed nibbles, code k at bits 4k.
__device__ __forceinline__ uint32_t pack8(const uint32_t* t)
{
    const uint32_t p01 = (t[1] << 4) | t[0];
    const uint32_t p23 = (t[3] << 4) | t[2];
    const uint32_t p45 = (t[5] << 4) | t[4];
    const uint32_t p67 = (t[7] << 4) | t[6];
    const uint32_t lo = __builtin_amdgcn_perm(p23, p01, 0x0C0C0400u);  // p01.b0, p23.b0
    const uint32_t hi = __builtin_amdgcn_perm(p67, p45, 0x0C0C0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u) ^ 0x88888888u;
}

// Four codes as 16 bits of signed nibbles.
__device__ __forceinline__ uint32_t pack4(const uint32_t* t)
{
    const uint32_t p01 = (t[1] << 4) | t[0];
    const uint32_t p23 = (t[3] << 4) | t[2];
    return (__builtin_amdgcn_perm(p23, p01, 0x0C0C0400u) ^ 0x8888u) & 0xffffu;
}

// grid = (strips, H): a workgroup owns one strip of one head, both planes;
// every lane runs two row jobs (key, value), whose loads go out together
// with the slot loads before the first rotation.
template <int D, typename In>
__global__ __launch_bounds__(kWriterThreads) void strip_writer(
    const In* __restrict__ key, const In* __restrict__ value, int8_t* __restrict__ key_cache,
    int8_t* __restrict__ value_cache, float* __restrict__ scale_cache,
    const int32_t* __restrict__ slots, const float* __restrict__ pi_signs,
    const void* __restrict__ tables, int tables_bf16, uint32_t H, uint32_t S, uint32_t P,
    float inv_sqrt_len)
{
    constexpr int CPL = D / 16;
    constexpr int TS = 20;  // token stride of the transpose buffer, in words
    // [channel / 8][token, padded to TS] words of 8 channel codes; 20-word
    // rows put the 64 lanes of a wave (16 lanes x 4 tokens) on distinct banks
    __shared__ __align__(16) uint32_t lds_t[D / 8][TS];
    __shared__ __align__(16) int ok_w[kWriterThreads / 64];  // per-wave slot checks

    const uint32_t strip = blockIdx.x, head = blockIdx.y;
    const int tid = threadIdx.x;
    const int row = tid >> 4;                 // token within the strip
    const int l = row_lane(tid & 15);      // logical lane: channels l*CPL ..

    // slots first, then the rows and the signs: one round trip for all
    const int32_t slot0 = slots[(size_t)strip * kStrip];
    const int32_t mine = slots[(size_t)strip * kStrip + row];
    float v[2][CPL], sign[CPL];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const In* src = (j == 0 ? key : value) +
                        ((size_t)((size_t)strip * kStrip + row) * H + head) * D + l * CPL;
        load_row<CPL>(src, v[j]);
    }
    load_signs<CPL>(pi_signs, tables, tables_bf16, l * CPL, sign);

    uint32_t t[2][CPL];
    float scale[2];
    writer_rotate_quantise<D, CPL>(v, sign, l, inv_sqrt_len, t, scale);

    // Slot contract for this strip: consecutive, strip-aligned, in range.
    // Each wave votes; the vote is read behind the transpose's barrier.
    const bool ok = slot0 >= 0 && (slot0 % kStrip) == 0 && mine == slot0 + row &&
                    (uint32_t)slot0 / S < P;
    static_assert(kWriterThreads == 256, "four wave votes");
    const int wv = __all(ok);
    if ((tid & 63) == 0) ok_w[tid >> 6] = wv;
    // value codes into the transpose buffer: one word of 8 channels per store
    // (at d = 64 two lanes share a word, 16 bits each)
    if constexpr (CPL >= 8) {
#pragma unroll
        for (int k = 0; k < CPL / 8; ++k) lds_t[l * (CPL / 8) + k][row] = pack8(&t[1][8 * k]);
    } else {
        ((uint16_t*)&lds_t[l >> 1][row])[l & 1] = (uint16_t)pack4(t[1]);
    }
    lds_barrier();
    {
        const int4 w4 = *(const int4*)ok_w;
        if (!(w4.x & w4.y & w4.z & w4.w)) return;
    }
    const uint32_t page = (uint32_t)slot0 / S;
    const uint32_t tip = (uint32_t)slot0 % S + (uint32_t)row;
    const size_t head_base = ((size_t)page * H + head) * S;  // in tokens
    if ((tid & 15) == 0) {
        scale_cache[((size_t)page * H + head) * S + tip] = scale[0];
        scale_cache[(((size_t)P + page) * H + head) * S + tip] = scale[1];
    }
    int8_t* kdst = key_cache + (head_base + tip) * (D / 2) + l * (CPL / 2);
    if constexpr (CPL == 16)
        *(uint2*)kdst = make_uint2(pack8(t[0]), pack8(&t[0][8]));
    else if constexpr (CPL == 8)
        *(uint32_t*)kdst = pack8(t[0]);
    else
        *(uint16_t*)kdst = (uint16_t)pack4(t[0]);
    // the value strip leaves as d*8 contiguous bytes: output word (channel,
    // half) holds that channel's codes of tokens 8*half .. +7, one nibble
    // from each of 8 consecutive buffer words (two 16-byte reads)
    uint32_t* strip_words =
        (uint32_t*)(value_cache + (head_base + (tip & ~(uint32_t)15)) * (D / 2));
    for (int w = tid; w < D * 2; w += kWriterThreads) {
        const int channel = w >> 1, half = w & 1;
        const uint32_t* src = &lds_t[channel >> 3][8 * half];
        const uint4 a = *(const uint4*)src;
        const uint4 b = *(const uint4*)(src + 4);
        const uint32_t sh = 4u * (uint32_t)(channel & 7);
        const uint32_t n[8] = {__builtin_amdgcn_ubfe(a.x, sh, 4), __builtin_amdgcn_ubfe(a.y, sh, 4),
                               __builtin_amdgcn_ubfe(a.z, sh, 4), __builtin_amdgcn_ubfe(a.w, sh, 4),
                               __builtin_amdgcn_ubfe(b.x, sh, 4), __builtin_amdgcn_ubfe(b.y, sh, 4),
                               __builtin_amdgcn_ubfe(b.z, sh, 4), __builtin_amdgcn_ubfe(b.w, sh, 4)};
        const uint32_t p01 = (n[1] << 4) | n[0];
        const uint32_t p23 = (n[3] << 4) | n[2];
        const uint32_t p45 = (n[5] << 4) | n[4];
        const uint32_t p67 = (n[7] << 4) | n[6];
        const uint32_t lo = __builtin_amdgcn_perm(p23, p01, 0x0C0C0400u);
        const uint32_t hi = __builtin_amdgcn_perm(p67, p45, 0x0C0C0400u);
        strip_words[w] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
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
    const int l = row_lane(tid & 15);  // logical lane: channels l*CPL ..

    if (probe != nullptr && blockIdx.x == 0 && tid < 32) {
        const int32_t fields[4] = {0, (int32_t)probe_grid, 1, (int32_t)item_count};
        probe[tid] = fields[tid >> 3];
    }

    float sign[CPL];
    load_signs<CPL>(pi_signs, nullptr, 0, l * CPL, sign);
    const float sigma = row_sigma(l);
    auto one = [&](uint32_t request, uint32_t head) {
        if (request >= num_requests) return;
        // The rows do not depend on the slot: their loads go out with its
        // load. A pad or out-of-pool slot reads page 0's strip and stores
        // nothing (so no load waits behind a branch).
        const size_t src_off = ((size_t)request * H + head) * D + l * CPL;
        const int32_t slot = slots[request];
        float v[2][CPL];
        load_row<CPL>(key + src_off, v[0]);
        load_row<CPL>(value + src_off, v[1]);
        const uint32_t page_raw = (uint32_t)slot / S;
        const bool ok = slot >= 0 && page_raw < P;
        const uint32_t page = ok ? page_raw : 0u;
        const uint32_t tip = ok ? (uint32_t)slot - page_raw * S : 0u;
        const uint32_t col = tip % kStrip;
        const size_t head_base = ((size_t)page * H + head) * S;
        uint4* strip = (uint4*)(value_cache + (head_base + (tip - col)) * (D / 2)) + l * (NW / 4);
        uint32_t w[NW];
#pragma unroll
        for (int i = 0; i < NW / 4; ++i) {
            const uint4 u = strip[i];
            w[4 * i] = u.x;
            w[4 * i + 1] = u.y;
            w[4 * i + 2] = u.z;
            w[4 * i + 3] = u.w;
        }
        // exact policy: absmax as is; a zero row (every element +-0 or
        // NaN) stores codes 0 and scale 1.0
        writer_rotate<D, CPL>(v, sign, l);
        float a[2];
        writer_absmax<CPL>(v, 0.0f, a);
        int e[2];
        float sc[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            e[r] = a[r] == 0.0f ? 2 : exponent_of(a[r]);
            sc[r] = a[r] == 0.0f ? 1.0f : ldexpf(1.0f, e[r] - 2) * inv_sqrt_len;
        }
        // y = v * 2^(2-e) by ldexp (e may be as low as -149), then the
        // magic-number rounding with sigma folded into the multiplier: keys
        // with kQMagic (code + 8 in bits 0..3, packed), values with
        // kQMagic - 8 (the two's-complement nibble in bits 0..3, spliced)
        uint32_t tk[CPL], tv[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float yk = a[0] == 0.0f ? 0.0f : ldexpf(v[0][j], 2 - e[0]);
            const float yv = a[1] == 0.0f ? 0.0f : ldexpf(v[1][j], 2 - e[1]);
            tk[j] = __float_as_uint(fminf(__builtin_fmaf(yk, sigma, kQMagic), kQMagicTop));
            tv[j] = __float_as_uint(
                fminf(__builtin_fmaf(yv, sigma, kQMagic - 8.0f), kQMagicTop - 8.0f));
        }
        if (!ok) return;
        if ((tid & 15) == 0) {
            scale_cache[((size_t)page * H + head) * S + tip] = sc[0];
            scale_cache[(((size_t)P + page) * H + head) * S + tip] = sc[1];
        }
        int8_t* kdst = key_cache + (head_base + tip) * (D / 2) + l * (CPL / 2);
        if constexpr (CPL == 16)
            *(uint2*)kdst = make_uint2(pack8(tk), pack8(&tk[8]));
        else if constexpr (CPL == 8)
            *(uint32_t*)kdst = pack8(tk);
        else
            *(uint16_t*)kdst = (uint16_t)pack4(tk);
        // the column's nibble in word 2j (tokens 0..7) or 2j + 1 (8..15):
        // both words take a bit-field insert, one under an empty mask (no
        // register array indexed by a lane value)
        const uint32_t sh = 4u * (col & 7u);
        const uint32_t m1 = (col >> 3) ? 0xfu << sh : 0u, m0 = (0xfu << sh) ^ m1;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t y = tv[j] << sh;
            w[2 * j] = (w[2 * j] & ~m0) | (y & m0);
            w[2 * j + 1] = (w[2 * j + 1] & ~m1) | (y & m1);
        }
#pragma unroll
        for (int i = 0; i < NW / 4; ++i)
            strip[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    };
    const uint64_t item_end = (uint64_t)item_begin + item_count;
    const uint32_t stride = gridDim.x * 16u;  // at most 4096 * 16
    if (item_end + stride <= 0xffffffffull) {
        // 32-bit item arithmetic: no item, nor the step past the last one,
        // reaches 2^32
        for (uint32_t item = item_begin + blockIdx.x * 16u + (uint32_t)grp;
             item < (uint32_t)item_end; item += stride)
            one(item / H, item % H);
    } else {
        for (uint64_t item = (uint64_t)item_begin + (uint64_t)blockIdx.x * 16u + (uint32_t)grp;
             item < item_end; item += (uint64_t)gridDim.x * 16u)
            one((uint32_t)(item / H), (uint32_t)(item % H));
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
    if (strips == 0 || H == 0) return hipSuccess;
    if (H > 65535u) return hipErrorInvalidValue;
    hipLaunchKernelGGL((strip_writer<D, In>), dim3(strips, H), dim3(kWriterThreads), 0, stream,
                       key, value, key_cache, value_cache, scale_cache, slots, pi_signs, tables,
                       tables_bf16, H, S, P, inv_sqrt_len);
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
