// tq4_rms.hip -- the vllm-ascend RMS + threshold codec (TurboQuantCodec<4>)
// and the baseline writer that applies it, on gfx950.
//
// Reference semantics (paths relative to the reference checkout):
//   codec      kernels/ops/turboquant/baseline/common/turboquant_codec_950.h
//                ApplyPi = signs, FWHT (strides 1..n/2, a+b | a-b), x inv_sqrt_len, signs  :115-151
//                scale = sqrt(sum y^2) * inv_sqrt_len + 1e-20                               :186-197
//                level = #{i : y * (-1/scale) + t_i has its sign bit set}                    :199-231
//                byte = (even level + 16 * odd level) - 128 as int8                         :234-248
//                dequantize: byte + 128 -> even / odd level -> centroid                     :251-285
//   writer     kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:98-246
//                (per token: every (plane, kv head) vector; rows at slot*H*(d/2) + h*(d/2);
//                 the slot's scale record [K scales, V scales, zeros to a multiple of 8];
//                 tokens with a slot outside [0, num_blocks * block_size) write nothing)
//   thresholds / centroids: codec_950.h:43-51,
//                tests/npu/bench/bench_turboquant_reshape_and_cache.cpp:55-61
//
// MI355X design: a vector is spread over 16 lanes of one wave row, d/16
// consecutive channels per lane (one 16-byte load of BF16 at d = 128), 16
// vectors per 256-lane workgroup, in the row lane order of the TQ4 writers
// (row_lane). The FWHT runs in registers below d/16 and as DPP-fed fused
// butterflies above (row_fmac_stage, same a+b / a-b bits); the sum of
// squares is a sequential per-lane sum and a 4-step tree over logical lanes. The level needs no table walk: since t_{14-i} = -t_i and
// t_7 = 0, a positive z counts 8 + #{t_8..t_14 < z} and a negative one
// 7 - #{t_8..t_14 <= -z}, each a 3-step binary search over seven constants.
// A row's d/2 packed bytes leave as one coalesced run (d/32 bytes per lane).
// Built with -ffp-contract=off: every FP32 operation is the one written, so the
// bits are those of the C oracle's restatement.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {
namespace {

constexpr int kRmsThreads = 256;
constexpr int kRowLanes = 16;
constexpr float kRmsEps = 1e-20f;

// The positive thresholds t_8 .. t_14 (codec_950.h:45-49); t_7 = 0 and
// t_{14-i} = -t_i.
constexpr float kPos[7] = {0.2582216646707196f, 0.5224037090113789f, 0.7995497875097155f,
                           1.0992858269170722f, 1.4371387916845330f, 1.8435318062766393f,
                           2.4008033987632817f};
// The 16 centroids, level order (bench_turboquant_reshape_and_cache.cpp:55-61).
constexpr float kCentroids[16] = {
    -2.7325895709951710f, -2.0690172265313920f, -1.6180463860218863f, -1.2562311973471796f,
    -0.9423404564869651f, -0.6567591185324659f, -0.3880482994902919f, -0.1283950298511473f,
    0.1283950298511473f,  0.3880482994902919f,  0.6567591185324659f,  0.9423404564869651f,
    1.2562311973471796f,  1.6180463860218863f,  2.0690172265313920f,  2.7325895709951710f};

// sqrt(x) rounded to nearest even for x >= 0: v_sqrt_f32 is faithful (within
// one ulp), so the neighbour whose residual sign says the root lies beyond
// the midpoint replaces it; x below 2^-96 is scaled by 2^32 first (and the
// root back by 2^-16) so the residuals stay normal.
__device__ __forceinline__ float sqrt_rn(float x)
{
    const bool tiny = x < 0x1.0p-96f;
    const float xs = tiny ? x * 0x1.0p+32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);
    const float dn = __uint_as_float(__float_as_uint(s) - 1u);
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    const float r_dn = __builtin_fmaf(-dn, s, xs);
    const float r_up = __builtin_fmaf(-up, s, xs);
    s = r_dn <= 0.0f ? dn : s;
    s = r_up > 0.0f ? up : s;
    // zero and +inf pass through unchanged (their neighbours are not roots)
    s = (xs == 0.0f || xs == __builtin_inff()) ? __builtin_amdgcn_sqrtf(xs) : s;
    return tiny ? s * 0x1.0p-16f : s;
}

// The level search by bins of |z| a quarter wide: bin b < 10 is [b/4,
// (b+1)/4), bin 10 is [2.5, inf]. The positive thresholds lie more than a
// quarter apart and none on a multiple of a quarter, so a bin holds at most
// one of them: #{k : kPos[k] < a} = below + (inside < a) of a's bin, `below`
// counting the thresholds under the bin and `inside` its own (+inf when it
// has none). 4a and its truncation are exact, so the count is.
struct LevelBin {
    float inside;
    uint32_t below;
};
constexpr int kLevelBins = 11;
constexpr LevelBin kBins[kLevelBins] = {
    {__builtin_inff(), 0}, {kPos[0], 0}, {kPos[1], 1}, {kPos[2], 2}, {kPos[3], 3},
    {kPos[4], 4},          {__builtin_inff(), 5}, {kPos[5], 5}, {__builtin_inff(), 6},
    {kPos[6], 6},          {__builtin_inff(), 7}};
static_assert((int)(kPos[0] * 4) == 1 && (int)(kPos[1] * 4) == 2 && (int)(kPos[2] * 4) == 3 &&
                  (int)(kPos[3] * 4) == 4 && (int)(kPos[4] * 4) == 5 &&
                  (int)(kPos[5] * 4) == 7 && (int)(kPos[6] * 4) == 9,
              "each threshold sits in the bin the table gives it");
static_assert(kPos[0] * 4 != 1 && kPos[1] * 4 != 2 && kPos[2] * 4 != 3 && kPos[3] * 4 != 4 &&
                  kPos[4] * 4 != 5 && kPos[5] * 4 != 7 && kPos[6] * 4 != 9,
              "no threshold on a bin boundary");

// The codec's level of z = y * (1/scale): #{i : t_i < z} (NaN -> 0). lut:
// kBins staged in LDS.
__device__ __forceinline__ uint32_t level_of(float z, const LevelBin* lut)
{
    const float a = fabsf(z);
    // for z < 0 the count is 7 - #{t_k <= |z|} = 7 - #{t_k < nextup(|z|)}
    const float up = __uint_as_float(min(__float_as_uint(a) + 1u, 0x7F800000u));
    const bool neg = z < 0.0f;
    const float b = neg ? up : a;
    // truncation: a NaN gives bin 0, +inf saturates to the last bin
    const uint32_t bin = min(__float2uint_rz(b * 4.0f), (uint32_t)(kLevelBins - 1));
    const LevelBin e = lut[bin];
    const uint32_t c = e.below + (e.inside < b ? 1u : 0u);
    return z > 0.0f ? 8u + c : neg ? 7u - c : (z == 0.0f ? 7u : 0u);
}

template <int D, int IN_BF16>
__global__ __launch_bounds__(kRmsThreads) void rms_writer(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    int8_t* __restrict__ key_cache, int8_t* __restrict__ value_cache,
    float* __restrict__ scale_cache, const int32_t* __restrict__ slots,
    const float* __restrict__ pi_signs, uint32_t tokens, uint32_t H, uint64_t slot_count,
    float inv_sqrt_len)
{
    constexpr int CPL = D / kRowLanes;
    const int lane = threadIdx.x & (kRowLanes - 1);
    const int l = row_lane(lane);  // logical lane: channels l*CPL ..
    // the level search's bins, staged before any lane leaves
    __shared__ LevelBin lut[kLevelBins];
    if (threadIdx.x == 0) {
#pragma unroll
        for (int b = 0; b < kLevelBins; ++b) lut[b] = kBins[b];
    }
    __syncthreads();
    const uint64_t row = (uint64_t)blockIdx.x * (kRmsThreads / kRowLanes) + threadIdx.x / kRowLanes;
    const uint32_t planes = 2 * H;
    const uint64_t rows = (uint64_t)tokens * planes;
    if (row >= rows) return;
    // 32-bit division when every row index fits (a uniform branch)
    const uint32_t t = rows <= 0xffffffffull ? (uint32_t)row / planes : (uint32_t)(row / planes);
    const uint32_t plane = (uint32_t)row - t * planes;
    const uint32_t h = plane < H ? plane : plane - H;
    const int32_t slot = slots[t];
    // the row's channels lane*CPL .. +CPL: one vector load, and the signs
    const uint16_t* src = (plane < H ? key : value) + ((uint64_t)t * H + h) * D + l * CPL;
    uint16_t raw[CPL];
    if constexpr (CPL == 4) {
        const uint2 w = *(const uint2*)src;
        raw[0] = w.x & 0xffff; raw[1] = w.x >> 16; raw[2] = w.y & 0xffff; raw[3] = w.y >> 16;
    } else {
#pragma unroll
        for (int q = 0; q < CPL / 8; ++q) {
            const uint4 w = *(const uint4*)(src + 8 * q);
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                raw[8 * q + 2 * k] = u[k] & 0xffff;
                raw[8 * q + 2 * k + 1] = u[k] >> 16;
            }
        }
    }
    float sg[CPL], v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        sg[j] = pi_signs[l * CPL + j];
        v[j] = IN_BF16 ? bf16_to_f32(raw[j]) : (float)__builtin_bit_cast(_Float16, raw[j]);
    }
    if (slot < 0 || (uint64_t)slot >= slot_count) return;  // a pad token or a slot past the pool

    // ApplyPi: signs, FWHT at strides 1 .. D/2, x inv_sqrt_len, signs. The
    // FWHT's cross-lane stages run on sign-tracked values (row_fmac_stage):
    // v holds sigma * y afterwards, sigma = row_sigma(l)
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] = v[j] * sg[j];
#pragma unroll
    for (int s = 1; s < D; s <<= 1) {
        if (s < CPL) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (j & s) continue;
                const float a = v[j];
                const float b = v[j + s];
                v[j] = b + a;
                v[j + s] = a - b;
            }
        } else {
            const int k = __builtin_ctz(s / CPL);
            row_fmac_stage<CPL>(v, ((l >> k) & 1) ? -1.0f : 1.0f, k);
        }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] = (v[j] * inv_sqrt_len) * sg[j];

    // scale = sqrt(sum y^2) * inv_sqrt_len + eps: per-lane sequential sum,
    // then the tree over logical lanes l ^ 1, l ^ 2, l ^ 4, l ^ 8 ((sigma y)^2
    // is y^2 exactly)
    float ss = v[0] * v[0];
#pragma unroll
    for (int j = 1; j < CPL; ++j) ss = ss + v[j] * v[j];
#pragma unroll
    for (int k = 0; k < 4; ++k) row_add1(ss, k);
    const float scale = sqrt_rn(ss) * inv_sqrt_len + kRmsEps;
    // sigma rides on the reciprocal: (sigma y) * (sigma r) rounds as y * r
    const float rcp = row_sigma(l) * __fdiv_rn(1.0f, scale);

    // levels, packed (even | odd << 4) ^ 0x80 -- the -128 bias of the int8 byte
    uint32_t pk[CPL / 8 > 0 ? CPL / 8 : 1] = {};
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t q = level_of(v[j] * rcp, lut);
        pk[j / 8] |= q << (4 * (j % 8));
    }
    int8_t* dst = (plane < H ? key_cache : value_cache) + ((uint64_t)slot * H + h) * (D / 2) +
                  l * (CPL / 2);
    if constexpr (CPL == 4) {
        *(uint16_t*)dst = (uint16_t)(pk[0] ^ 0x8080u);
    } else if constexpr (CPL == 8) {
        *(uint32_t*)dst = pk[0] ^ 0x80808080u;
    } else {
        *(uint2*)dst = make_uint2(pk[0] ^ 0x80808080u, pk[1] ^ 0x80808080u);
    }
    // the slot's scale record: this plane's scale, and its share of the zero padding
    const uint32_t ssf = (planes + 7u) / 8u * 8u;
    float* rec = scale_cache + (uint64_t)slot * ssf;
    if (lane == 0) {
        rec[plane] = scale;
    } else {
        const uint32_t pad = planes + plane * (kRowLanes - 1) + (lane - 1);
        if (pad < ssf) rec[pad] = 0.0f;
    }
}

// Dequantize4Bit: four packed bytes -> eight centroids per lane, grid-stride.
__global__ __launch_bounds__(kRmsThreads) void rms_dequant(const uint32_t* __restrict__ packed,
                                                           float4* __restrict__ out,
                                                           uint64_t words)
{
    __shared__ float cent[16];
    if (threadIdx.x < 16) cent[threadIdx.x] = kCentroids[threadIdx.x];
    __syncthreads();
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t w = packed[i] ^ 0x80808080u;
        float f[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] = cent[(w >> (4 * k)) & 15u];
        out[2 * i] = make_float4(f[0], f[1], f[2], f[3]);
        out[2 * i + 1] = make_float4(f[4], f[5], f[6], f[7]);
    }
}

__global__ void rms_dequant_tail(const uint8_t* __restrict__ packed, float* __restrict__ out,
                                 uint64_t first, uint64_t bytes)
{
    const uint64_t j = first + threadIdx.x;
    if (j >= bytes) return;
    const uint32_t v = packed[j] ^ 0x80u;
    out[2 * j] = kCentroids[v & 15u];
    out[2 * j + 1] = kCentroids[v >> 4];
}

template <int D>
hipError_t launch_rms_writer_t(hipStream_t stream, int in_bf16, const uint16_t* key,
                               const uint16_t* value, int8_t* kc, int8_t* vc, float* sc,
                               const int32_t* slots, const float* signs, uint32_t tokens,
                               uint32_t H, uint64_t slot_count, float isl)
{
    const uint64_t rows = (uint64_t)tokens * 2 * H;
    const uint32_t blocks = (uint32_t)((rows + kRmsThreads / kRowLanes - 1) / (kRmsThreads / kRowLanes));
    if (in_bf16)
        hipLaunchKernelGGL((rms_writer<D, 1>), dim3(blocks), dim3(kRmsThreads), 0, stream, key,
                           value, kc, vc, sc, slots, signs, tokens, H, slot_count, isl);
    else
        hipLaunchKernelGGL((rms_writer<D, 0>), dim3(blocks), dim3(kRmsThreads), 0, stream, key,
                           value, kc, vc, sc, slots, signs, tokens, H, slot_count, isl);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rms_writer(hipStream_t stream, int in_bf16, const uint16_t* key,
                             const uint16_t* value, int8_t* key_cache, int8_t* value_cache,
                             float* scale_cache, const int32_t* slots, const float* pi_signs,
                             uint32_t tokens, uint32_t H, uint32_t D, uint64_t slot_count,
                             float inv_sqrt_len)
{
    if (tokens == 0) return hipSuccess;
    switch (D) {
        case 64: return launch_rms_writer_t<64>(stream, in_bf16, key, value, key_cache, value_cache,
                                                scale_cache, slots, pi_signs, tokens, H, slot_count,
                                                inv_sqrt_len);
        case 128: return launch_rms_writer_t<128>(stream, in_bf16, key, value, key_cache,
                                                  value_cache, scale_cache, slots, pi_signs, tokens,
                                                  H, slot_count, inv_sqrt_len);
        case 256: return launch_rms_writer_t<256>(stream, in_bf16, key, value, key_cache,
                                                  value_cache, scale_cache, slots, pi_signs, tokens,
                                                  H, slot_count, inv_sqrt_len);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rms_dequantize(hipStream_t stream, const int8_t* packed, float* out,
                                 uint64_t bytes)
{
    const uint64_t words = bytes / 4;
    if (words) {
        uint64_t blocks = (words + kRmsThreads - 1) / kRmsThreads;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(rms_dequant, dim3((uint32_t)blocks), dim3(kRmsThreads), 0, stream,
                           (const uint32_t*)packed, (float4*)out, words);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (bytes % 4) {
        hipLaunchKernelGGL(rms_dequant_tail, dim3(1), dim3(4), 0, stream, (const uint8_t*)packed,
                           out, words * 4, bytes);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace tq4
