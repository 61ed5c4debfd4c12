// tq4_precise.hip -- the partial-record decode in the reference's FP32
// operation order (gfx950), for tq4_paged_decode_partials with
// TQ4_DECODE_PRECISE.
//
// Reference semantics (paths relative to the reference checkout):
//   q_rot, rounded to BF16 as the device's score operand
//                                      tests/common/paged_decode_oracle.hpp:486-514
//   score R . key scale, FP32          tests/common/paged_decode_oracle.hpp:516-540
//   recurrence (tile max, alpha, p, value scale folded into p, l, acc)
//                                      tests/common/single_token_decode_oracle.hpp:257-310
//   tail masking by overwrite          kernels/ops/turboquant/turboquant_decode_tail.hpp:56-118
//   partition, neutral record          include/turboquant_splitk_contract.hpp:119-130,
//                                      turboquant_paged_decode_attention.cpp:1630-1633
//
// The MFMA decode (tq4_decode.hip) feeds fp16 operands: its score operand
// carries a per-row offset that is cancelled in the FP32 accumulator, and
// its P.V operand is P * value scale in fp16, so its records agree with the
// reference's to about 2^-11. This kernel keeps every product and sum in
// FP32 on the vector ALU, so its records meet the reference rig's budgets
// (tests/npu/turboquant_splitk_rigs.hpp:144-158: m 2e-6, l 1e-4,
// acc 2e-4): the score is sum_c q_eff[c] * nibble[c] (exact products of a
// BF16 operand and a small integer), times the key scale; then per strip
// m' = max(m, tile max), alpha = exp(m - m'), p = exp(s - m'),
// l = l alpha + sum p, acc[c] = acc[c] alpha + sum_t (p vscale)[t] nib[c][t],
// in token order. Built with -ffp-contract=off: every multiply and add
// rounds where the oracle's does.
//
// One 256-lane workgroup per (seq, kv head, split); every wave walks all of
// the split's strips for its q rows g = wave, wave + 4, ... (up to 4 rows).
// Score lanes: token t = lane & 15 of the strip, channel quarter lane >> 4;
// value lanes: channels lane * d/64 ... The next strip's loads are issued
// before the current strip's arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tq4.h"
#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {
namespace {

constexpr int kWavesP = 4;
constexpr int kThreadsP = 64 * kWavesP;
constexpr int kRowsPerWave = 4;  // G <= 16

// Signed nibble k (0..7) of a 32-bit word: low nibble first.
__device__ __forceinline__ float nib(uint32_t w, int k)
{
    return (float)(((int32_t)(w << (28 - 4 * k))) >> 28);
}

template <int D>
struct StripData {
    uint32_t k[D / 32];  // key bytes: token lane & 15, channels (lane >> 4) * d/4 .. + d/4
    uint32_t v[D / 32];  // value bytes: channels lane * d/64 .., 8 bytes (16 tokens) each
    float ks, vs;        // key and value scale of token lane & 15
    uint32_t active;     // live tokens of the strip (0: skipped)
};

template <int D>
__device__ __forceinline__ void load_strip(const DecodeParams& p, uint32_t seq, uint32_t kvh,
                                           uint32_t ctx, uint32_t lp, uint32_t sip, int lane,
                                           StripData<D>& s)
{
    const int32_t phys_raw = p.block_tables[(size_t)seq * p.max_blocks + lp];
    const uint64_t tbase = (uint64_t)lp * p.S + (uint64_t)sip * kStrip;
    // a table entry that names no page contributes no token
    const bool valid = phys_raw >= 0 && (uint32_t)phys_raw < p.P;
    s.active = valid ? active_in_strip(tbase, ctx) : 0u;
    const uint32_t phys = valid ? (uint32_t)phys_raw : 0u;
    const uint32_t row0 = (phys * p.Hkv + kvh) * p.S + sip * kStrip;  // the strip's first row
    const int t = lane & 15, qd = lane >> 4;
    const uint8_t* kb = (const uint8_t*)p.key_cache + (size_t)(row0 + t) * (D / 2) + qd * (D / 8);
    const uint8_t* vb = (const uint8_t*)p.value_cache + (size_t)row0 * (D / 2) + lane * (D / 8);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        s.k[i] = ((const uint32_t*)kb)[i];
        s.v[i] = ((const uint32_t*)vb)[i];
    }
    const size_t plane = (size_t)p.P * p.Hkv * p.S;
    s.ks = p.scale_cache[row0 + t];
    s.vs = p.scale_cache[plane + row0 + t];
}

template <int D>
__global__ __launch_bounds__(kThreadsP) void decode_precise_kernel(DecodeParams p)
{
    constexpr int CPL = D / 64;   // value channels per lane
    constexpr int CQ = D / 4;     // score channels per lane
    __shared__ float q_eff[16][D];

    const uint32_t item = blockIdx.x;
    const uint32_t seq = item / (p.K * p.Hkv), kvh = (item / p.K) % p.Hkv, split = item % p.K;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = p.G;

    // ---- q_eff per row: (Pi q) rounded to BF16 (the reference's q_rot
    // image), or q as given when it is already rotated; times the softmax
    // scale (the oracle's fold: tq4o_rotate_query)
    const bool rotated = (p.flags & 1u) != 0;
    float sg[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) sg[j] = rotated ? 1.0f : p.pi_signs[lane * CPL + j];
    for (uint32_t g = wave; g < G; g += kWavesP) {
        const uint16_t* qr = p.q + ((size_t)seq * p.Hq + kvh * G + g) * D + lane * CPL;
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[j] = bf16_to_f32(qr[j]);
        if (!rotated) {
            rotate_ingress<D, CPL>(v, sg, lane);
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[j] = bf16_to_f32(f32_to_bf16(v[j] * p.inv_sqrt_len));
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) q_eff[g][lane * CPL + j] = v[j] * p.scale;
    }
    __syncthreads();

    uint32_t pb, pc;
    partition(p.max_blocks, p.K, split, pb, pc);
    const int32_t ctx_raw = p.context_lens[seq];
    uint32_t ctx = ctx_raw < 0 ? 0u : (uint32_t)ctx_raw;
    const uint64_t capacity = (uint64_t)p.max_blocks * p.S;
    if (ctx > capacity) ctx = (uint32_t)capacity;
    const uint32_t spp = p.S / kStrip;
    // strips of the window that may hold a live token
    uint32_t ns = 0;
    if (pc > 0 && ctx > (uint64_t)pb * p.S) {
        const uint64_t live = ctx - (uint64_t)pb * p.S;
        const uint64_t cap = (uint64_t)pc * p.S;
        ns = (uint32_t)(((live < cap ? live : cap) + kStrip - 1) / kStrip);
    }

    float m[kRowsPerWave], l[kRowsPerWave], acc[kRowsPerWave][CPL];
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
        m[i] = kMasked;
        l[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[i][j] = 0.0f;
    }
    const int t = lane & 15, qd = lane >> 4;
    StripData<D> cur, nxt;
    if (ns > 0) load_strip<D>(p, seq, kvh, ctx, pb, 0, lane, cur);
    for (uint32_t si = 0; si < ns; ++si) {
        if (si + 1 < ns) {
            const uint32_t sj = si + 1;
            load_strip<D>(p, seq, kvh, ctx, pb + sj / spp, sj % spp, lane, nxt);
        }
        const uint32_t active = __builtin_amdgcn_readfirstlane(cur.active);  // wave-uniform
        if (active > 0) {
#pragma unroll
            for (int i = 0; i < kRowsPerWave; ++i) {
                const uint32_t g = wave + kWavesP * i;
                if (g >= G) break;
                // score of token t: this lane's quarter of the channels in
                // channel order, then the quarters summed
                const float* qrow = &q_eff[g][qd * CQ];
                float dot = 0.0f;
#pragma unroll
                for (int w = 0; w < D / 32; ++w) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) dot = dot + qrow[8 * w + k] * nib(cur.k[w], k);
                }
                dot = dot + __shfl_xor(dot, 16, 64);
                dot = dot + __shfl_xor(dot, 32, 64);
                const bool live = (uint32_t)t < active;
                const float s = live ? dot * cur.ks : kMasked;  // overwrite, never multiply
                float tmax = s;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 64));
                const float m_new = m[i] > tmax ? m[i] : tmax;
                const float alpha = expf(m[i] - m_new);
                const float pt = live ? expf(s - m_new) : 0.0f;
                float psum = pt;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) psum = psum + __shfl_xor(psum, o, 64);
                const float ps = live ? pt * cur.vs : 0.0f;
                // acc[c] = acc[c] * alpha + sum over live tokens in token order
                float wsum[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) wsum[j] = 0.0f;
                // tokens 0..7 sit in word 2j of channel j, tokens 8..15 in 2j + 1
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t t1 = min(active, 8u * (half + 1));
                    for (uint32_t tt = 8u * half; tt < t1; ++tt) {
                        const float pst =
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ps), tt));
#pragma unroll
                        for (int j = 0; j < CPL; ++j)
                            wsum[j] = wsum[j] + pst * nib(cur.v[2 * j + half], (int)(tt & 7));
                    }
                }
#pragma unroll
                for (int j = 0; j < CPL; ++j) acc[i][j] = acc[i][j] * alpha + wsum[j];
                l[i] = l[i] * alpha + psum;
                m[i] = m_new;
            }
        }
        if (si + 1 < ns) cur = nxt;
    }

    // ---- export: [m, l, 0, 0, acc] per q row
    constexpr int RS = D + 4;
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
        const uint32_t g = wave + kWavesP * i;
        if (g >= G) break;
        float* rec = p.records + (((size_t)seq * p.Hq + kvh * G + g) * p.K + split) * RS;
        if (lane == 0) *(float4*)rec = make_float4(m[i], l[i], 0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < CPL; ++j) rec[4 + lane * CPL + j] = acc[i][j];
    }
}

template <int D>
hipError_t launch_precise_t(hipStream_t stream, const DecodeParams& p)
{
    const size_t blocks = (size_t)p.B * p.Hkv * p.K;
    hipLaunchKernelGGL((decode_precise_kernel<D>), dim3((uint32_t)blocks), dim3(kThreadsP), 0,
                       stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_precise(hipStream_t stream, const DecodeParams& p)
{
    switch (p.D) {
        case 64: return launch_precise_t<64>(stream, p);
        case 128: return launch_precise_t<128>(stream, p);
        case 256: return launch_precise_t<256>(stream, p);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace tq4
