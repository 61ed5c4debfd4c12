// tq4_device.hpp -- device helpers shared by the TQ4 kernels (gfx950, wave64).
//
// Cache contract and arithmetic restated from the reference (paths relative
// to the reference checkout):
//   layout        tests/common/turboquant_scatter_oracle.hpp:31-38,110-132
//   rotation      tests/common/rotate_butterfly_oracle.hpp:44-48,120-142
//   quantiser     tests/common/turboquant_oracle.hpp:412-448,
//                 tests/common/turboquant_scatter_oracle.hpp:185-217
//   tail masking  kernels/ops/turboquant/turboquant_decode_tail.hpp:56-118
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tq4 {

constexpr int kStrip = 16;            // tokens per strip (R)
constexpr float kMasked = -3.0e38f;   // score of a masked lane, also the neutral m
constexpr int kPolicyPrefill = 0;     // absmax floored at 1.0
constexpr int kPolicyExact = 1;       // exact absmax, zero row -> scale 1.0

__device__ __forceinline__ float bf16_to_f32(uint32_t raw16)
{
    return __uint_as_float(raw16 << 16);
}

// Round-to-nearest-even float -> bf16 bits; quiet NaN kept quiet.
__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x7fffffu)) return ((b >> 16) | 0x40u) & 0xffffu;
    return ((b + 0x7fffu + ((b >> 16) & 1u)) >> 16) & 0xffffu;
}

// Partner value `mask` lanes away inside the wave (mask a power of two < 64),
// with VALU lane moves only: DPP inside a 16-lane row, permlane swaps across
// rows. `mask` is a compile-time constant at every call site.
__device__ __forceinline__ float dpp_move(float v, int ctrl_tag)
{
    const int x = __float_as_int(v);
    int r;
    switch (ctrl_tag) {
        case 1: r = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, true); break;   // quad_perm 1,0,3,2
        case 2: r = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, true); break;   // quad_perm 2,3,0,1
        case 4: {
            const int h = __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, true);    // row_half_mirror
            r = __builtin_amdgcn_update_dpp(h, h, 0x1B, 0xF, 0xF, true);             // quad_perm 3,2,1,0
            break;
        }
        default: r = __builtin_amdgcn_update_dpp(x, x, 0x128, 0xF, 0xF, true); break; // row_ror:8
    }
    return __int_as_float(r);
}

__device__ __forceinline__ float xor_lanes(float v, int mask)
{
    if (mask < 16) return dpp_move(v, mask);
    const uint32_t u = __float_as_uint(v);
    const uint32_t lane = __lane_id();
    if (mask == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((lane & 16u) ? p[0] : p[1]);
    }
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((lane & 32u) ? p[0] : p[1]);
}

// Row lane order for rows of 16 lanes (the writers): logical lane l
// (channels l*CPL ..) lives on physical lane p(l) = l ^ (l & 4 ? 3 : 0), a
// linear map that puts logical bits 1, 2, 4, 8 at physical xor masks 1, 2, 7,
// 8, so that each is one DPP pattern: quad_perm (xor 1, xor 2),
// row_half_mirror (xor 7 inside each 8-lane half) and row_ror:8 (xor 8).
// p is its own inverse.
__device__ __forceinline__ int row_lane(int p) { return p ^ ((p & 4) ? 3 : 0); }

// The value at logical lane l ^ (1 << k) of the row (k = 0..3).
__device__ __forceinline__ float row_partner(float v, int k)
{
    const int x = __float_as_int(v);
    int r;
    switch (k) {
        case 0: r = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, true); break;   // quad_perm 1,0,3,2
        case 1: r = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, true); break;   // quad_perm 2,3,0,1
        case 2: r = __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, true); break;  // row_half_mirror
        default: r = __builtin_amdgcn_update_dpp(x, x, 0x128, 0xF, 0xF, true); break; // row_ror:8
    }
    return __int_as_float(r);
}

// v = OP(v, v at logical lane l ^ (1 << k)) for two values (row_max2: max,
// row_add1: sum), the partner read through DPP by the operation itself: one
// instruction per value instead of a DPP move plus the operation (plus, for
// fmaxf, a canonicalisation of the moved value). Each block opens with the two
// wait states a DPP read of a VGPR written just before it needs; a max or a
// sum of two finite or infinite floats returns the same bits either way.
#define TQ4_DPP_OP(OP, I, CTRL) \
    "v_" OP "_f32_dpp %" #I ", %" #I ", %" #I " " CTRL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define TQ4_MAX_DPP2(CTRL) \
    asm volatile("s_nop 1\n\t" TQ4_DPP_OP("max", 0, CTRL) TQ4_DPP_OP("max", 1, CTRL) \
                 : "+v"(a0), "+v"(a1))
#define TQ4_ADD_DPP1(CTRL) asm volatile("s_nop 1\n\t" TQ4_DPP_OP("add", 0, CTRL) : "+v"(a0))

__device__ __forceinline__ void row_max2(float& a0, float& a1, int k)
{
    switch (k) {
        case 0: TQ4_MAX_DPP2("quad_perm:[1,0,3,2]"); break;
        case 1: TQ4_MAX_DPP2("quad_perm:[2,3,0,1]"); break;
        case 2: TQ4_MAX_DPP2("row_half_mirror"); break;
        default: TQ4_MAX_DPP2("row_ror:8"); break;
    }
}

__device__ __forceinline__ void row_add1(float& a0, int k)
{
    switch (k) {
        case 0: TQ4_ADD_DPP1("quad_perm:[1,0,3,2]"); break;
        case 1: TQ4_ADD_DPP1("quad_perm:[2,3,0,1]"); break;
        case 2: TQ4_ADD_DPP1("row_half_mirror"); break;
        default: TQ4_ADD_DPP1("row_ror:8"); break;
    }
}
#undef TQ4_ADD_DPP1
#undef TQ4_MAX_DPP2
#undef TQ4_DPP_OP

// w += c * w[logical lane l ^ (1 << k)] for 8 (or 4) values: v_fmac_f32 with
// its first source read through DPP. One asm block, so nothing is scheduled
// inside it; it opens with the two wait states that a DPP read of a VGPR
// written by the instruction just before it needs. (The compiler does not
// fold a DPP move into v_fmac_f32.)
#define TQ4_FMAC_DPP(I, C, CTRL) \
    "v_fmac_f32_dpp %" #I ", %" #I ", %" #C " " CTRL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define TQ4_FMAC_DPP8(CTRL)                                                                       \
    asm volatile("s_nop 1\n\t" TQ4_FMAC_DPP(0, 8, CTRL) TQ4_FMAC_DPP(1, 8, CTRL)                 \
                     TQ4_FMAC_DPP(2, 8, CTRL) TQ4_FMAC_DPP(3, 8, CTRL) TQ4_FMAC_DPP(4, 8, CTRL)  \
                         TQ4_FMAC_DPP(5, 8, CTRL) TQ4_FMAC_DPP(6, 8, CTRL) TQ4_FMAC_DPP(7, 8, CTRL) \
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),        \
                   "+v"(x[6]), "+v"(x[7])                                                         \
                 : "v"(c))
#define TQ4_FMAC_DPP4(CTRL)                                                                       \
    asm volatile("s_nop 1\n\t" TQ4_FMAC_DPP(0, 4, CTRL) TQ4_FMAC_DPP(1, 4, CTRL)                 \
                     TQ4_FMAC_DPP(2, 4, CTRL) TQ4_FMAC_DPP(3, 4, CTRL)                            \
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3])                                 \
                 : "v"(c))

__device__ __forceinline__ void fmac_partner8(float* x, float c, int k)
{
    switch (k) {
        case 0: TQ4_FMAC_DPP8("quad_perm:[1,0,3,2]"); break;
        case 1: TQ4_FMAC_DPP8("quad_perm:[2,3,0,1]"); break;
        case 2: TQ4_FMAC_DPP8("row_half_mirror"); break;
        default: TQ4_FMAC_DPP8("row_ror:8"); break;
    }
}

__device__ __forceinline__ void fmac_partner4(float* x, float c, int k)
{
    switch (k) {
        case 0: TQ4_FMAC_DPP4("quad_perm:[1,0,3,2]"); break;
        case 1: TQ4_FMAC_DPP4("quad_perm:[2,3,0,1]"); break;
        case 2: TQ4_FMAC_DPP4("row_half_mirror"); break;
        default: TQ4_FMAC_DPP4("row_ror:8"); break;
    }
}
#undef TQ4_FMAC_DPP4
#undef TQ4_FMAC_DPP8
#undef TQ4_FMAC_DPP

// One cross-lane butterfly stage of a row in the row lane order, on values
// held with a per-lane sign: a lane stores w = sigma * v, sigma = (-1)^(the
// number of logical lane bits below the stage's that are set). The stage's
// pair shares sigma, and the butterfly
//   out[i] = in[i ^ s] + ((i & s) ? -in[i] : in[i])
// is w' = w + c * w_partner with c = -1 on the upper lane (whose sigma then
// flips) and +1 on the lower: one fused multiply-add per element, exact in
// the product (c = +-1), so its one rounding is that of the add or subtract.
// In-register stages and sign diagonals commute with sigma; after the last
// stage sigma = (-1)^popcount(l) (row_sigma).
template <int CPL>
__device__ __forceinline__ void row_fmac_stage(float (&v)[CPL], float c, int k)
{
    if constexpr (CPL >= 8) {
#pragma unroll
        for (int j = 0; j < CPL; j += 8) fmac_partner8(&v[j], c, k);
    } else {
        static_assert(CPL == 4, "4, 8 or 16 channels per lane");
        fmac_partner4(v, c, k);
    }
}

__device__ __forceinline__ float row_sigma(int l) { return (__builtin_popcount(l) & 1) ? -1.0f : 1.0f; }

// One butterfly stage at `stride` over a row spread across lanes, CPL
// consecutive channels per lane (channel = lane_in_row * CPL + j):
//   out[i] = in[i ^ s] + ((i & s) ? -in[i] : in[i])
// In-register below CPL, a lane exchange (xor stride/CPL) at or above it.
template <int CPL>
__device__ __forceinline__ void butterfly(float (&v)[CPL], int stride, int lane_in_row)
{
    if (stride < CPL) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if (j & stride) continue;
            const float a = v[j];
            const float b = v[j + stride];
            v[j] = b + a;
            v[j + stride] = a - b;
        }
    } else {
        // p - v is p + (-v) exactly (IEEE subtraction is the addition of the
        // negation), so the upper lanes flip v's sign bit and every lane adds:
        // one XOR and one DPP-fed add instead of an add, a subtract and a select.
        const int m = stride / CPL;
        const uint32_t flip = (lane_in_row & m) != 0 ? 0x80000000u : 0u;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float p = xor_lanes(v[j], m);
            v[j] = p + __uint_as_float(__float_as_uint(v[j]) ^ flip);
        }
    }
}

// Ingress rotation y = M x: strides 1..16, the sign diagonal, then 32..D/2.
template <int D, int CPL>
__device__ __forceinline__ void rotate_ingress(float (&v)[CPL], const float (&sign)[CPL],
                                               int lane_in_row)
{
#pragma unroll
    for (int s = 1; s < 32 && s < D; s <<= 1) butterfly<CPL>(v, s, lane_in_row);
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] *= sign[j];
#pragma unroll
    for (int s = 32; s < D; s <<= 1) butterfly<CPL>(v, s, lane_in_row);
}

// Egress rotation y = M^T x: strides 32..D/2, the sign diagonal, then 1..16.
template <int D, int CPL>
__device__ __forceinline__ void rotate_egress(float (&v)[CPL], const float (&sign)[CPL],
                                              int lane_in_row)
{
#pragma unroll
    for (int s = 32; s < D; s <<= 1) butterfly<CPL>(v, s, lane_in_row);
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] *= sign[j];
#pragma unroll
    for (int s = 1; s < 32 && s < D; s <<= 1) butterfly<CPL>(v, s, lane_in_row);
}

// Exponent e with 2^e <= a < 2^(e+1), for finite a > 0 (ilogb).
__device__ __forceinline__ int exponent_of(float a)
{
    const uint32_t bits = __float_as_uint(a);
    const uint32_t field = (bits >> 23) & 0xffu;
    if (field != 0u) return (int)field - 127;
    const uint32_t m = bits & 0x7fffffu;
    return (31 - (int)__clz((int)m)) - 149;
}

// Live tokens of the strip starting at token_base, 0..16.
__device__ __forceinline__ uint32_t active_in_strip(uint64_t token_base, uint32_t seq_len)
{
    const uint64_t live = seq_len;
    if (token_base >= live) return 0u;
    return live - token_base >= (uint64_t)kStrip ? (uint32_t)kStrip : (uint32_t)(live - token_base);
}

// Partition of `pages` logical pages over `splits`
// (include/turboquant_splitk_contract.hpp:123-130).
__device__ __forceinline__ void partition(uint32_t pages, uint32_t splits, uint32_t split,
                                          uint32_t& begin, uint32_t& count)
{
    const uint32_t width = (pages + splits - 1u) / splits;
    begin = split * width;
    const uint32_t remaining = begin < pages ? pages - begin : 0u;
    count = remaining < width ? remaining : width;
}

// Workgroup barrier for LDS traffic only: it does not wait for outstanding
// global loads or for store acknowledgements (vmcnt), which __syncthreads()
// does, so prefetched loads stay in flight and earlier stores are not
// waited for.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Record traffic between workgroups of one launch: buffer stores and loads
// with the device-coherence bit (sc1 -- what agent-scope relaxed atomic
// stores and loads are on gfx950), plain accesses to the compiler, so they
// vectorise and a whole chunk of loads is in flight at once. No whole-L2
// write-back or invalidate is needed around the arrival counter.

constexpr int kCachePolicySc1 = 16;          // cache-policy operand bit of sc1
constexpr uint32_t kRecMagic = 0x7FBADBADu;  // fused records hold bits ^ kRecMagic; 0 = not written
constexpr uint32_t kPollLimit = 1u << 20;    // bound of a combiner's record polls
constexpr uint32_t kPollLimitTest = 16;      // the bound under the test hook (a few microseconds)

// A combiner whose bounded poll gave up adds one to a sticky count in the
// workspace (per combined row), which the host reads back; the row's output
// is then computed from incomplete records and must not be used.
__device__ __forceinline__ void count_timeout(uint32_t* timeouts)
{
    if (timeouts != nullptr)
        __hip_atomic_fetch_add(timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t records_rsrc(const float* base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7fffffff,
                                             0x00020000);
}

typedef uint32_t rec_u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t rec_u4_t __attribute__((ext_vector_type(4)));

// Stores and loads of N = 1, 2 or 4 consecutive record floats. ENC: the fused
// encoding (bits ^ kRecMagic) and the device-coherence bit.
template <int N, bool ENC>
__device__ __forceinline__ void rec_store(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                          const float* v)
{
    const uint32_t x = ENC ? kRecMagic : 0u;
    const int pol = ENC ? kCachePolicySc1 : 0;
    if constexpr (N == 4) {
        const rec_u4_t u = rec_u4_t{__float_as_uint(v[0]) ^ x, __float_as_uint(v[1]) ^ x,
                                    __float_as_uint(v[2]) ^ x, __float_as_uint(v[3]) ^ x};
        __builtin_amdgcn_raw_buffer_store_b128(u, r, byte_off, 0, pol);
    } else if constexpr (N == 2) {
        const rec_u2_t u = rec_u2_t{__float_as_uint(v[0]) ^ x, __float_as_uint(v[1]) ^ x};
        __builtin_amdgcn_raw_buffer_store_b64(u, r, byte_off, 0, pol);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]) ^ x, r, byte_off, 0, pol);
    }
}

// Raw words (still encoded when ENC).
template <int N, bool ENC>
__device__ __forceinline__ void rec_load(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                         uint32_t* w)
{
    const int pol = ENC ? kCachePolicySc1 : 0;
    if constexpr (N == 4) {
        const rec_u4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, pol);
        w[0] = u[0];
        w[1] = u[1];
        w[2] = u[2];
        w[3] = u[3];
    } else if constexpr (N == 2) {
        const rec_u2_t u = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, pol);
        w[0] = u[0];
        w[1] = u[1];
    } else {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, pol);
    }
}

}  // namespace tq4
