// tq4_decode.hip -- paged split-K decode attention over the TQ4 cache (gfx950).
//
// Reference semantics (paths relative to the reference checkout):
//   partial per (request, kv head, split)  turboquant_paged_decode_attention.cpp:1570-1641
//   score / recurrence order               tests/common/single_token_decode_oracle.hpp:257-310
//   tail masking by overwrite              kernels/ops/turboquant/turboquant_decode_tail.hpp:56-118
//   neutral element of an empty split      turboquant_paged_decode_attention.cpp:1630-1633
//   LSE combine                            tests/common/l2_atomic_oracle.hpp:156-176
//   egress (Pi^T, 1/sqrt(d), gate)         tests/common/paged_decode_oracle.hpp:598-665
//
// MI355X design
// -------------
// One 256-lane workgroup per (seq, kv head, split); its four waves take the
// split's live strips round-robin and each streams its strips with
// register-double-buffered loads. Per strip and wave:
//   * S = K . Q^T on MFMA f32_16x16x16_f16: M = the strip's 16 tokens, N =
//     the GQA group (up to 16 q heads), K = head_size in head_size/16 steps.
//     A lane loads d/8 contiguous bytes of one token's key row (one 16-byte
//     load at d = 128; the whole 1 KiB strip is one coalesced wave load).
//     Nibbles become fp16 (1 + u/16), u = nibble ^ 8, by shift/and/or only;
//     the MFMA accumulator starts at -1.5 * sum(q), which removes the bias
//     exactly in real arithmetic, so the product is sum(q * nibble) / 16.
//   * The score tile lands in the C layout (lane = q head + 16 * token
//     quarter), which is exactly the A layout the P.V product needs, so the
//     online softmax runs in registers (exp2 domain, two lane exchanges for
//     the row max) and P never leaves the wave.
//   * O += P . V on the same MFMA, V nibbles as exact fp16 n/16, P scaled by
//     the value scale and a running power of two so it stays in [0, 2).
// The four waves' (m, l, acc) merge through LDS; the workgroup then exports
// one partial record, or, in the fused entry, the last workgroup of each
// (seq, kv head) to arrive (an agent-scope counter that resets itself)
// combines all splits, rotates back, gates and stores BF16. No spinlock: the
// reference's L2-line lock (turboquant_splitk_reduce.cpp:279-350) is replaced
// by disjoint records plus one counter increment per workgroup.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {
namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint32_t kMant = 0x03C003C0u;  // a nibble placed in fp16 mantissa bits [9:6]
constexpr uint32_t kOne = 0x3C003C00u;   // fp16 1.0 in both halves
constexpr uint32_t kFlagRotated = 1u;

__device__ __forceinline__ h4_t as_h4(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(h4_t, u2_t{a, b});
}

__device__ __forceinline__ f4_t mfma16(h4_t a, h4_t b, f4_t c)
{
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// fp16 pair (1 + u/16) with u = n + 8  ->  exact n/16.
__device__ __forceinline__ uint32_t signed_pair(uint32_t p)
{
    const h2_t v = __builtin_bit_cast(h2_t, p) - h2_t{(_Float16)1.5f, (_Float16)1.5f};
    return __builtin_bit_cast(uint32_t, v);
}

// One strip's operands for one lane (n = lane & 15, kg = lane >> 4).
template <int D>
struct StripRegs {
    uint32_t k[D / 32];  // key row of token n, bytes kg*d/8 .. +d/8
    uint32_t v[D / 16];  // value: tokens 4kg..4kg+3 of channel 16b + n (16 bits)
    f4_t ks;             // key scales of tokens 4kg..4kg+3
    f4_t vs;             // value scales of tokens 4kg..4kg+3
};

template <int D>
__device__ __forceinline__ void load_strip(StripRegs<D>& r, const int8_t* kb, const int8_t* vb,
                                           const float* ksp, const float* vsp, int n, int kg)
{
    const int8_t* kp = kb + n * (D / 2) + kg * (D / 8);
    if constexpr (D == 64) {
        const uint2 w = *(const uint2*)kp;
        r.k[0] = w.x;
        r.k[1] = w.y;
    } else {
#pragma unroll
        for (int i = 0; i < D / 128; ++i) {
            const uint4 w = *(const uint4*)(kp + 16 * i);
            r.k[4 * i + 0] = w.x;
            r.k[4 * i + 1] = w.y;
            r.k[4 * i + 2] = w.z;
            r.k[4 * i + 3] = w.w;
        }
    }
#pragma unroll
    for (int b = 0; b < D / 16; ++b) r.v[b] = *(const uint16_t*)(vb + (16 * b + n) * 8 + 2 * kg);
    r.ks = *(const f4_t*)(ksp + 4 * kg);
    r.vs = *(const f4_t*)(vsp + 4 * kg);
}

// LDS layout (floats): [0, 2*G*D) two exchange slots, aliased by the q
// staging area and by the in-LDS record of a single-split fused launch;
// then m[4][16], l[4][16], q exponents[16], one flag word.
__host__ __device__ constexpr size_t lds_floats(uint32_t G, uint32_t D)
{
    return 2ull * G * D + 2ull * kWaves * 16 + 16 + 4;
}

// LSE-combine K records of one (seq, q head) row (first record at `rec`,
// stride D+4 floats), normalise, optionally rotate back and gate, store BF16.
// One wave; lane holds CPL = D/64 consecutive channels.
template <int D>
__device__ void finish_row(const float* rec, uint32_t K, const float* pi_signs, const float* gate,
                           uint16_t* out, float inv_sqrt_len, uint32_t stage, int lane)
{
    constexpr int CPL = D / 64;
    constexpr int RS = D + 4;
    float M = kMasked;
    for (uint32_t k = 0; k < K; ++k) M = fmaxf(M, rec[(size_t)k * RS]);
    float L = 0.0f, acc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
        const float* r = rec + (size_t)k * RS;
        const float w = expf(r[0] - M);
        L += r[1] * w;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] += r[4 + lane * CPL + j] * w;
    }
    float v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] = L == 0.0f ? 0.0f : acc[j] / L;
    if (stage >= 1) {
        float sg[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) sg[j] = pi_signs[lane * CPL + j];
        rotate_egress<D, CPL>(v, sg, lane);
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[j] *= inv_sqrt_len;
        if (stage == 2) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[j] = v[j] / (1.0f + expf(-gate[lane * CPL + j]));
        }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) out[lane * CPL + j] = (uint16_t)f32_to_bf16(v[j]);
}

template <int D, int MODE>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams p)
{
    constexpr int CPL = D / 64;   // channels per lane in the row layout
    constexpr int NB = D / 16;    // MFMA steps of the score, blocks of the output
    constexpr int KDW = D / 32;   // key words per lane per strip
    constexpr int RS = D + 4;     // record stride in floats
    extern __shared__ float smem[];

    const uint32_t G = p.G, S = p.S;
    float* m_x = smem + 2 * (size_t)G * D;
    float* l_x = m_x + kWaves * 16;
    int* q_exp = (int*)(l_x + kWaves * 16);
    int* flag = q_exp + 16;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, kg = lane >> 4;
    const uint32_t item = blockIdx.x;
    const uint32_t split = item % p.K;
    const uint32_t kvh = (item / p.K) % p.Hkv;
    const uint32_t seq = item / (p.K * p.Hkv);

    int32_t ctx_raw = p.context_lens[seq];
    uint32_t ctx = ctx_raw < 0 ? 0u : (uint32_t)ctx_raw;
    const uint64_t capacity = (uint64_t)p.max_blocks * S;
    if (ctx > capacity) ctx = (uint32_t)capacity;
    const uint32_t pages = (ctx + S - 1) / S;
    uint32_t pb, pc;
    partition(pages, p.K, split, pb, pc);
    const uint32_t spp = S / kStrip;
    const uint64_t tok0 = (uint64_t)pb * S;
    uint32_t live = 0;
    if (pc > 0 && ctx > tok0) {
        const uint64_t need = (ctx - tok0 + kStrip - 1) / kStrip;
        live = need < (uint64_t)pc * spp ? (uint32_t)need : pc * spp;
    }

    // ---- q prologue: rotate (Pi = M * inv_sqrt_len), fold the softmax
    // scale, normalise each row by a power of two, stage in LDS.
    float* q_st = smem;
    for (uint32_t g = wave; g < G; g += kWaves) {
        const uint16_t* qr = p.q + ((size_t)seq * p.Hq + kvh * G + g) * D + lane * CPL;
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[j] = bf16_to_f32(qr[j]);
        if (!(p.flags & kFlagRotated)) {
            float sg[CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) sg[j] = p.pi_signs[lane * CPL + j];
            rotate_ingress<D, CPL>(v, sg, lane);
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[j] = (v[j] * p.inv_sqrt_len) * p.scale;
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[j] = v[j] * p.scale;
        }
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) a = fmaxf(a, fabsf(v[j]));
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) a = fmaxf(a, xor_lanes(a, m));
        const int kq = a > 0.0f ? exponent_of(a) : 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) q_st[g * D + lane * CPL + j] = ldexpf(v[j], -kq);
        if (lane == 0) q_exp[g] = kq;
    }
    __syncthreads();

    // ---- this lane's B operand (q head n, channel group kg) and constants.
    u2_t qop[NB];
    float bias = 0.0f, cf = 0.0f;
    if ((uint32_t)n < G) {
        const float* qrow = q_st + n * D;
#pragma unroll
        for (int dd = 0; dd < KDW; ++dd) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int base = kg * (D / 4) + 8 * dd + 2 * h;
                const _Float16 a0 = (_Float16)qrow[base], a1 = (_Float16)qrow[base + 4];
                const _Float16 a2 = (_Float16)qrow[base + 1], a3 = (_Float16)qrow[base + 5];
                bias += ((float)a0 + (float)a1) + ((float)a2 + (float)a3);
                qop[2 * dd + h] = __builtin_bit_cast(u2_t, h4_t{a0, a1, a2, a3});
            }
        }
        cf = ldexpf(16.0f * kLog2e, q_exp[n]);
    } else {
#pragma unroll
        for (int s = 0; s < NB; ++s) qop[s] = u2_t{0u, 0u};
    }
    bias += xor_lanes(bias, 16);
    bias += xor_lanes(bias, 32);
    bias *= -1.5f;
    __syncthreads();  // q staging is dead from here; its LDS is reused below

    // ---- stream the strips.
    f4_t acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m2 = kMasked, lpart = 0.0f;
    int E = 0;  // running max exponent field of the live value scales
    const int32_t* tbl = p.block_tables + (size_t)seq * p.max_blocks;
    const size_t plane_floats = (size_t)p.P * p.Hkv * S;

    auto strip_ptrs = [&](uint32_t idx, const int8_t*& kb, const int8_t*& vb, const float*& ksp,
                          const float*& vsp) -> bool {
        const uint32_t lp = pb + idx / spp, sip = idx % spp;
        const uint32_t phys = (uint32_t)tbl[lp];
        const size_t row = ((size_t)phys * p.Hkv + kvh) * S + (size_t)sip * kStrip;
        kb = p.key_cache + row * (D / 2);
        vb = p.value_cache + row * (D / 2);
        ksp = p.scale_cache + row;
        vsp = ksp + plane_floats;
        return phys < p.P;
    };

    StripRegs<D> cur, nxt;
    bool cur_ok = false;
    if ((uint32_t)wave < live) {
        const int8_t *kb, *vb;
        const float *ksp, *vsp;
        cur_ok = strip_ptrs(wave, kb, vb, ksp, vsp);
        if (cur_ok) load_strip<D>(cur, kb, vb, ksp, vsp, n, kg);
    }
    for (uint32_t idx = wave; idx < live; idx += kWaves) {
        bool nxt_ok = false;
        if (idx + kWaves < live) {
            const int8_t *kb, *vb;
            const float *ksp, *vsp;
            nxt_ok = strip_ptrs(idx + kWaves, kb, vb, ksp, vsp);
            if (nxt_ok) load_strip<D>(nxt, kb, vb, ksp, vsp, n, kg);
        }
        if (cur_ok) {
            // Scores: C[token][q] = sum_c (1 + u/16) q16 - 1.5 sum q16 = sum q16 n / 16.
            f4_t sc = f4_t{bias, bias, bias, bias};
#pragma unroll
            for (int dd = 0; dd < KDW; ++dd) {
                const uint32_t x = cur.k[dd] ^ 0x88888888u;
                const uint32_t p0 = ((x << 6) & kMant) | kOne;
                const uint32_t p1 = ((x << 2) & kMant) | kOne;
                const uint32_t p2 = ((x >> 2) & kMant) | kOne;
                const uint32_t p3 = ((x >> 6) & kMant) | kOne;
                sc = mfma16(as_h4(p0, p1), __builtin_bit_cast(h4_t, qop[2 * dd]), sc);
                sc = mfma16(as_h4(p2, p3), __builtin_bit_cast(h4_t, qop[2 * dd + 1]), sc);
            }
            const uint32_t act = active_in_strip(tok0 + (uint64_t)idx * kStrip, ctx);
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = (sc[i] * cf) * cur.ks[i];
                s[i] = (uint32_t)(4 * kg + i) < act ? v : kMasked;
            }
            float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mx = fmaxf(mx, xor_lanes(mx, 16));
            mx = fmaxf(mx, xor_lanes(mx, 32));
            const float mn = fmaxf(m2, mx);
            const float alpha = exp2f(m2 - mn);
            float pr[4], psum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[i] = exp2f(s[i] - mn);
                psum += pr[i];
            }
            lpart = lpart * alpha + psum;
            int e = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if ((uint32_t)(4 * kg + i) < act)
                    e = max(e, (int)((__float_as_uint(cur.vs[i]) >> 23) & 0xffu));
            e = max(e, __shfl_xor(e, 16, 64));
            e = max(e, __shfl_xor(e, 32, 64));
            const int En = max(E, e);
            const float av = ldexpf(alpha, E - En);
            _Float16 hp[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x =
                    (uint32_t)(4 * kg + i) < act ? ldexpf(pr[i] * cur.vs[i], 127 - En) : 0.0f;
                hp[i] = (_Float16)x;
            }
            const h4_t P = h4_t{hp[0], hp[1], hp[2], hp[3]};
            if (__any(av != 1.0f)) {
                float f[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) f[i] = __shfl(av, 4 * kg + i, 64);
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[b][i] *= f[i];
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint32_t x = cur.v[b] ^ 0x8888u;
                const uint32_t y = x | (x << 12);
                const uint32_t b0 = signed_pair(((y << 6) & kMant) | kOne);
                const uint32_t b1 = signed_pair(((y >> 2) & kMant) | kOne);
                acc[b] = mfma16(P, as_h4(b0, b1), acc[b]);
            }
            m2 = mn;
            E = En;
        }
        cur = nxt;
        cur_ok = nxt_ok;
    }

    // ---- merge the four waves.
    lpart += xor_lanes(lpart, 16);
    lpart += xor_lanes(lpart, 32);
    if (kg == 0) {
        m_x[wave * 16 + n] = m2;
        l_x[wave * 16 + n] = lpart;
    }
    __syncthreads();
    const float unit = ldexpf(16.0f, E - 127);
    float Mrow[4], Lrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 4 * kg + i;
        float M = m_x[r];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, m_x[w * 16 + r]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) L += exp2f(m_x[w * 16 + r] - M) * l_x[w * 16 + r];
        const float f = exp2f(m_x[wave * 16 + r] - M) * unit;
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b][i] *= f;
        Mrow[i] = M;
        Lrow[i] = L;
    }
    float* slot0 = smem;
    float* slot1 = smem + (size_t)G * D;
    auto put = [&](float* slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 4 * kg + i;
            if (r < G) {
#pragma unroll
                for (int b = 0; b < NB; ++b) slot[r * D + 16 * b + n] = acc[b][i];
            }
        }
    };
    auto add = [&](const float* slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 4 * kg + i;
            if (r < G) {
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[b][i] += slot[r * D + 16 * b + n];
            }
        }
    };
    if (wave >= 2) put(wave == 2 ? slot0 : slot1);
    __syncthreads();
    if (wave < 2) add(wave == 0 ? slot0 : slot1);
    __syncthreads();
    if (wave == 1) put(slot0);
    __syncthreads();

    // ---- wave 0 owns the workgroup's result: export one record per q head.
    const bool fused_local = (MODE == 1) && p.K == 1;
    float* rec_base = fused_local
                          ? smem
                          : p.records + (((size_t)seq * p.Hq + (size_t)kvh * G) * p.K + split) * RS;
    const size_t row_stride = fused_local ? (size_t)RS : (size_t)p.K * RS;
    if (wave == 0) {
        add(slot0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 4 * kg + i;
            if (r < G) {
                float* rec = rec_base + r * row_stride;
#pragma unroll
                for (int b = 0; b < NB; ++b) rec[4 + 16 * b + n] = acc[b][i];
                if (n == 0) {
                    rec[0] = Mrow[i] == kMasked ? kMasked : Mrow[i] * kLn2;
                    rec[1] = Lrow[i];
                    rec[2] = 0.0f;
                    rec[3] = 0.0f;
                }
            }
        }
    }
    if constexpr (MODE == 0) return;

    // ---- fused: the last workgroup of this (seq, kv head) combines.
    uint32_t K_rows = 1;
    if (!fused_local) {
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            uint32_t* ctr = p.counters + (size_t)seq * p.Hkv + kvh;
            const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == p.K - 1;
            if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last;
        }
        __syncthreads();
        if (!*flag) return;
        __threadfence();
        rec_base = p.records + ((size_t)seq * p.Hq + (size_t)kvh * G) * p.K * RS;
        K_rows = p.K;
    } else {
        __syncthreads();
    }
    for (uint32_t g = wave; g < G; g += kWaves) {
        const size_t qh = (size_t)seq * p.Hq + kvh * G + g;
        finish_row<D>(rec_base + g * row_stride, K_rows, p.pi_signs,
                      p.gate ? p.gate + qh * D : nullptr, p.out + qh * D, p.inv_sqrt_len,
                      p.output_stage, lane);
    }
}

template <int D>
__global__ __launch_bounds__(kThreads) void combine_kernel(DecodeParams p)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t row = (size_t)blockIdx.x * kWaves + wave;  // seq * Hq + q head
    if (row >= (size_t)p.B * p.Hq) return;
    finish_row<D>(p.records + row * p.K * (D + 4), p.K, p.pi_signs,
                  p.gate ? p.gate + row * D : nullptr, p.out + row * D, p.inv_sqrt_len,
                  p.output_stage, lane);
}

__global__ void fill_zero_kernel(uint32_t* ptr, size_t words)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (size_t)gridDim.x * blockDim.x)
        ptr[i] = 0u;
}

template <int D>
hipError_t launch_decode_t(hipStream_t stream, const DecodeParams& p, int mode)
{
    const size_t blocks = (size_t)p.B * p.Hkv * p.K;
    const size_t lds = lds_floats(p.G, D) * sizeof(float);
    if (mode == 0)
        hipLaunchKernelGGL((decode_kernel<D, 0>), dim3((uint32_t)blocks), dim3(kThreads), lds,
                           stream, p);
    else
        hipLaunchKernelGGL((decode_kernel<D, 1>), dim3((uint32_t)blocks), dim3(kThreads), lds,
                           stream, p);
    return hipGetLastError();
}

}  // namespace

size_t decode_records_bytes(uint32_t B, uint32_t Hq, uint32_t D, uint32_t K)
{
    const size_t bytes = (size_t)B * Hq * K * (D + 4) * sizeof(float);
    return (bytes + 255) & ~(size_t)255;
}

hipError_t launch_decode(hipStream_t stream, const DecodeParams& p, int mode)
{
    switch (p.D) {
        case 64: return launch_decode_t<64>(stream, p, mode);
        case 128: return launch_decode_t<128>(stream, p, mode);
        case 256: return launch_decode_t<256>(stream, p, mode);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_combine(hipStream_t stream, const DecodeParams& p)
{
    const size_t rows = (size_t)p.B * p.Hq;
    const uint32_t blocks = (uint32_t)((rows + kWaves - 1) / kWaves);
    switch (p.D) {
        case 64:
            hipLaunchKernelGGL((combine_kernel<64>), dim3(blocks), dim3(kThreads), 0, stream, p);
            break;
        case 128:
            hipLaunchKernelGGL((combine_kernel<128>), dim3(blocks), dim3(kThreads), 0, stream, p);
            break;
        case 256:
            hipLaunchKernelGGL((combine_kernel<256>), dim3(blocks), dim3(kThreads), 0, stream, p);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero(hipStream_t stream, void* ptr, size_t bytes)
{
    const size_t words = bytes / 4;
    if (words == 0) return hipSuccess;
    size_t blocks = (words + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                       (uint32_t*)ptr, words);
    return hipGetLastError();
}

}  // namespace tq4
