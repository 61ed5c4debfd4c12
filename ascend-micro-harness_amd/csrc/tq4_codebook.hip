// tq4_codebook.hip -- the codebook quantiser leaves on gfx950.
//
// Reference semantics (paths relative to the reference checkout):
//   ICDF leaf        routines/routine_vector_icdf_quantize.hpp:10-30 (transform, packing),
//                    oracle tests/cpu/icdf_fixture.hpp:122-142,222-232
//   Lloyd-Max        include/routines/routine_vector_lloydmax_quantize.hpp:8-37 (codebooks,
//                    code = #thresholds <= x), :223-255 (packed decode)
//   Gaussian-CDF     tests/common/lloydmax_oracle.hpp:19-28 (compander),
//                    include/routines/routine_vector_gaussian_cdf_quantize.hpp:6-19 (centroids)
//   packing          tests/common/lloydmax_oracle.hpp:58-62 (code i at bit (i*bits) % 8 of
//                    byte i*bits/8)
//
// Every kernel is an elementwise HBM stream in which each load and store
// instruction of a wave covers one contiguous span. ICDF: a lane owns eight
// consecutive FP16/BF16 elements (one 16-byte load, a wave 1 KiB) and stores
// their codes as one 32-bit word. FP32 Lloyd-Max / Gaussian-CDF: a lane owns
// two quads of four elements, T lanes apart (a float4 each, a wave 1 KiB per
// instruction, both loads in flight), and stores each quad's codes as one
// 16-bit (4-bit codes) or 8-bit (2-bit codes) word; this measured 12 % faster
// than eight consecutive elements per lane (two float4 loads 32 bytes apart
// across the lanes). Grid-stride loops over a grid sized to the device (a few
// waves per SIMD), so any length runs.
//
// Lloyd-Max codes without a table walk: the 4-bit thresholds are symmetric
// about 0 (t[14-i] = -t[i], t[7] = 0), so the code is the sign plus a 3-step
// binary search of |x| over t[8..14] (>= for x >= 0, > for x < 0: ties go to
// the upper bin on both sides), and the centroid is sign * c[8 + search] by a
// select tree -- about twenty VALU per element, no LDS and no gather.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq4_internal.hpp"

namespace tq4 {
namespace {

constexpr int kCbThreads = 256;

// Lloyd-Max codebooks (include/routines/routine_vector_lloydmax_quantize.hpp:14-28):
// the positive half of the 4-bit centroids / thresholds, and the 2-bit ones.
constexpr float kLm4C[8] = {0.128395030f, 0.388048299f, 0.656759119f, 0.942340456f,
                            1.256231197f, 1.618046386f, 2.069017227f, 2.732589571f};
constexpr float kLm4T[7] = {0.258221665f, 0.522403709f, 0.799549788f, 1.099285827f,
                            1.437138792f, 1.843531806f, 2.400803399f};
constexpr float kLm2C[2] = {0.452794f, 1.510418f};
constexpr float kLm2T = 0.981606f;
// Gaussian-CDF centroids (include/routines/routine_vector_gaussian_cdf_quantize.hpp:9-18)
constexpr float kCdf4C[16] = {-1.8627318674f, -1.3180108973f, -1.0099901692f, -0.7764217611f,
                              -0.5791321623f, -0.4022500653f, -0.2372021093f, -0.0784124127f,
                              0.0784124127f,  0.2372021093f,  0.4022500653f,  0.5791321623f,
                              0.7764217611f,  1.0099901692f,  1.3180108973f,  1.8627318674f};
constexpr float kCdf2C[4] = {-1.1503493804f, -0.318639364f, 0.318639364f, 1.1503493804f};

// code (0..15) and centroid of one value, Lloyd-Max 4-bit
__device__ __forceinline__ uint32_t lm4(float x, float& recon)
{
    const bool neg = x < 0.0f;  // -0 counts as positive: -0 >= t[7] = 0
    const float a = fabsf(x);
    // binary search of |x| over t[8..14]: k = #{t <= a} (x >= 0) or #{t < a} (x < 0)
    auto over = [&](float t) { return neg ? a > t : a >= t; };
    const bool b2 = over(kLm4T[3]);
    const bool b1 = over(b2 ? kLm4T[5] : kLm4T[1]);
    const float t0 = b2 ? (b1 ? kLm4T[6] : kLm4T[4]) : (b1 ? kLm4T[2] : kLm4T[0]);
    const bool b0 = over(t0);
    const uint32_t k = (uint32_t)b2 * 4u + (uint32_t)b1 * 2u + (uint32_t)b0;
    const float m = b2 ? (b1 ? (b0 ? kLm4C[7] : kLm4C[6]) : (b0 ? kLm4C[5] : kLm4C[4]))
                       : (b1 ? (b0 ? kLm4C[3] : kLm4C[2]) : (b0 ? kLm4C[1] : kLm4C[0]));
    const bool nan = x != x;  // every comparison false: code 0
    recon = nan ? -kLm4C[7] : (neg ? -m : m);
    return nan ? 0u : (neg ? 7u - k : 8u + k);
}

__device__ __forceinline__ uint32_t lm2(float x, float& recon)
{
    const bool neg = x < 0.0f;
    const float a = fabsf(x);
    const bool far = neg ? a > kLm2T : a >= kLm2T;
    const float m = far ? kLm2C[1] : kLm2C[0];
    const bool nan = x != x;
    recon = nan ? -kLm2C[1] : (neg ? -m : m);
    return nan ? 0u : (neg ? (far ? 0u : 1u) : (far ? 3u : 2u));
}

// Gaussian-CDF compander in the reference oracle's FP32 operation order
// (this unit is built with -ffp-contract=off): floor(2^b / (1 + exp(-z))),
// z = (0.070565 x^2 + 1.5976) x, clamped to [0, 2^b - 1]; NaN gives 0.
template <int BITS>
__device__ __forceinline__ uint32_t cdf_code(float x)
{
    const float xx = x * x;
    const float cubic = 0.070565f * xx;
    const float slope = cubic + 1.5976f;
    const float z = slope * x;
    const float e = expf(-z);
    const float d = e + 1.0f;
    const float v = (float)(1 << BITS) / d;
    const float f = floorf(v);
    const float lo = f > 0.0f ? f : 0.0f;
    const uint32_t u = (uint32_t)lo;
    constexpr uint32_t top = (1u << BITS) - 1u;
    return u < top ? u : top;
}

template <int BITS>
__device__ __forceinline__ float cdf_centroid(uint32_t q)
{
    if constexpr (BITS == 2) {
        return q & 2u ? (q & 1u ? kCdf2C[3] : kCdf2C[2]) : (q & 1u ? kCdf2C[1] : kCdf2C[0]);
    } else {
        // symmetric: c[15 - i] = -c[i]
        const bool hi = q >= 8u;
        const uint32_t k = hi ? q - 8u : 7u - q;  // index into the positive half
        const float m = k & 4u ? (k & 2u ? (k & 1u ? kCdf4C[15] : kCdf4C[14])
                                         : (k & 1u ? kCdf4C[13] : kCdf4C[12]))
                               : (k & 2u ? (k & 1u ? kCdf4C[11] : kCdf4C[10])
                                         : (k & 1u ? kCdf4C[9] : kCdf4C[8]));
        return hi ? m : -m;
    }
}

template <int BITS>
__device__ __forceinline__ float lm_centroid(uint32_t q)
{
    if constexpr (BITS == 2) {
        return q & 2u ? (q & 1u ? kLm2C[1] : kLm2C[0]) : (q & 1u ? -kLm2C[0] : -kLm2C[1]);
    } else {
        const bool hi = q >= 8u;
        const uint32_t k = hi ? q - 8u : 7u - q;
        const float m = k & 4u ? (k & 2u ? (k & 1u ? kLm4C[7] : kLm4C[6])
                                         : (k & 1u ? kLm4C[5] : kLm4C[4]))
                               : (k & 2u ? (k & 1u ? kLm4C[3] : kLm4C[2])
                                         : (k & 1u ? kLm4C[1] : kLm4C[0]));
        return hi ? m : -m;
    }
}

// ---------------------------------------------------------------- kernels
// book 0 Lloyd-Max, 1 Gaussian-CDF: FP32 -> codes (+ centroids when recon)
template <int BITS, int BOOK>
__global__ __launch_bounds__(kCbThreads) void quantize_kernel(const float* __restrict__ src,
                                                              float* __restrict__ recon,
                                                              uint8_t* __restrict__ codes,
                                                              uint64_t groups)
{
    // quads of 4 values, lane-contiguous: quads u and u + T per iteration
    const uint64_t nq = 2 * groups, T = (uint64_t)gridDim.x * kCbThreads;
    for (uint64_t u = (uint64_t)blockIdx.x * kCbThreads + threadIdx.x; u < nq; u += 2 * T) {
        const bool two = u + T < nq;
        const float4 a = *(const float4*)(src + 4 * u);
        float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
        if (two) b = *(const float4*)(src + 4 * (u + T));
        float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}, y[8];
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (BOOK == 0) {
                q[i] = BITS == 4 ? lm4(x[i], y[i]) : lm2(x[i], y[i]);
            } else {
                q[i] = cdf_code<BITS>(x[i]);
                y[i] = cdf_centroid<BITS>(q[i]);
            }
        }
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= q[i] << (BITS * i);
            w1 |= q[4 + i] << (BITS * i);
        }
        if constexpr (BITS == 4) {
            ((uint16_t*)codes)[u] = (uint16_t)w0;
            if (two) ((uint16_t*)codes)[u + T] = (uint16_t)w1;
        } else {
            codes[u] = (uint8_t)w0;
            if (two) codes[u + T] = (uint8_t)w1;
        }
        if (recon != nullptr) {
            *(float4*)(recon + 4 * u) = make_float4(y[0], y[1], y[2], y[3]);
            if (two) *(float4*)(recon + 4 * (u + T)) = make_float4(y[4], y[5], y[6], y[7]);
        }
    }
}

// packed Lloyd-Max codes -> centroids
template <int BITS>
__global__ __launch_bounds__(kCbThreads) void dequantize_kernel(const uint8_t* __restrict__ codes,
                                                                float* __restrict__ recon,
                                                                uint64_t groups)
{
    // quads of 4 values, lane-contiguous: quads u and u + T per iteration
    const uint64_t nq = 2 * groups, T = (uint64_t)gridDim.x * kCbThreads;
    for (uint64_t u = (uint64_t)blockIdx.x * kCbThreads + threadIdx.x; u < nq; u += 2 * T) {
        const bool two = u + T < nq;
        uint32_t w0, w1 = 0;
        if constexpr (BITS == 4) {
            w0 = ((const uint16_t*)codes)[u];
            if (two) w1 = ((const uint16_t*)codes)[u + T];
        } else {
            w0 = codes[u];
            if (two) w1 = codes[u + T];
        }
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            y[i] = lm_centroid<BITS>((w0 >> (BITS * i)) & ((1u << BITS) - 1u));
            y[4 + i] = lm_centroid<BITS>((w1 >> (BITS * i)) & ((1u << BITS) - 1u));
        }
        *(float4*)(recon + 4 * u) = make_float4(y[0], y[1], y[2], y[3]);
        if (two) *(float4*)(recon + 4 * (u + T)) = make_float4(y[4], y[5], y[6], y[7]);
    }
}

// ICDF: FP16/BF16 -> signed int4 of RNE(14 / (1 + exp(-x)) - 7), saturated
// to [-8, 7], element 2j in bits [3:0] of byte j. The FP32 evaluation is
// within a few 1e-6 of the exact value; no 16-bit input lies that close to a
// rounding boundary, so every one of the 65536 FP16 and the 65536 BF16 bit
// patterns gets the code of the double-precision evaluation (checked
// exhaustively against the C oracle on the GPU).
template <bool BF16>
__global__ __launch_bounds__(kCbThreads) void icdf_kernel(const uint16_t* __restrict__ in,
                                                          uint32_t* __restrict__ out,
                                                          uint64_t groups)
{
    for (uint64_t g = (uint64_t)blockIdx.x * kCbThreads + threadIdx.x; g < groups;
         g += (uint64_t)gridDim.x * kCbThreads) {
        const uint4 w = *(const uint4*)(in + 8 * g);
        const uint32_t h[4] = {w.x, w.y, w.z, w.w};
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t bits = (h[i >> 1] >> (16 * (i & 1))) & 0xffffu;
            float x;
            if constexpr (BF16)
                x = __uint_as_float(bits << 16);
            else
                x = (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
            const float e = __expf(-x);
            const float y = 14.0f * __builtin_amdgcn_rcpf(1.0f + e) - 7.0f;
            const float r = fminf(fmaxf(__builtin_rintf(y), -8.0f), 7.0f);
            const int32_t q = y == y ? (int32_t)r : 0;
            word |= ((uint32_t)q & 0xfu) << (4 * i);
        }
        out[g] = word;
    }
}

uint32_t grid_for(uint64_t groups)
{
    const uint64_t want = (groups + kCbThreads - 1) / kCbThreads;
    const uint64_t cap = 256ull * 8ull;  // 256 CUs x 8 workgroups
    return (uint32_t)(want < cap ? (want > 0 ? want : 1) : cap);
}

}  // namespace

hipError_t launch_icdf_quantize(hipStream_t stream, int in_bf16, const uint16_t* in, uint8_t* out,
                                uint64_t count)
{
    const uint64_t groups = count / 8;
    if (in_bf16)
        hipLaunchKernelGGL((icdf_kernel<true>), dim3(grid_for(groups)), dim3(kCbThreads), 0,
                           stream, in, (uint32_t*)out, groups);
    else
        hipLaunchKernelGGL((icdf_kernel<false>), dim3(grid_for(groups)), dim3(kCbThreads), 0,
                           stream, in, (uint32_t*)out, groups);
    return hipGetLastError();
}

hipError_t launch_codebook_quantize(hipStream_t stream, uint32_t book, uint32_t bits,
                                    const float* src, float* recon, uint8_t* codes,
                                    uint64_t count)
{
    const uint64_t groups = count / 8;
    const dim3 grid(grid_for(groups)), block(kCbThreads);
    if (book == 0 && bits == 4)
        hipLaunchKernelGGL((quantize_kernel<4, 0>), grid, block, 0, stream, src, recon, codes, groups);
    else if (book == 0)
        hipLaunchKernelGGL((quantize_kernel<2, 0>), grid, block, 0, stream, src, recon, codes, groups);
    else if (bits == 4)
        hipLaunchKernelGGL((quantize_kernel<4, 1>), grid, block, 0, stream, src, recon, codes, groups);
    else
        hipLaunchKernelGGL((quantize_kernel<2, 1>), grid, block, 0, stream, src, recon, codes, groups);
    return hipGetLastError();
}

hipError_t launch_codebook_dequantize(hipStream_t stream, uint32_t bits, const uint8_t* codes,
                                      float* recon, uint64_t count)
{
    const uint64_t groups = count / 8;
    if (bits == 4)
        hipLaunchKernelGGL((dequantize_kernel<4>), dim3(grid_for(groups)), dim3(kCbThreads), 0,
                           stream, codes, recon, groups);
    else
        hipLaunchKernelGGL((dequantize_kernel<2>), dim3(grid_for(groups)), dim3(kCbThreads), 0,
                           stream, codes, recon, groups);
    return hipGetLastError();
}

}  // namespace tq4
