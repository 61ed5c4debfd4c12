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
// One 256-lane workgroup per (seq, kv head, split). The split's strips are
// walked in PAIRS (32 tokens); the four waves take pairs round-robin and each
// wave streams its pairs through a three-deep register ring (loads for pairs
// j+1 and j+2 in flight while pair j computes). Every load in the ring is
// unconditional (indices clamp to the wave's last pair), so the compiler's
// wait counts stay exact and nothing drains the prefetch.
//
// Per pair and wave, on MFMA f32_16x16x32_f16:
//   * scores, two MFMA chains (token sets T1, T2; M = 16 tokens, N = the GQA
//     group padded to 16, K = head_size): lane (m, g) loads d/8 contiguous
//     bytes of one key row, so the wave reads both 1 KiB key strips in one
//     coalesced pass. Row m of T1 is token 8*((m>>2)&1) + (m&3) of strip m>>3,
//     T2 the same token + 4 -- chosen so that the score tile leaves each lane
//     holding exactly the 8 consecutive tokens whose value nibbles form ONE
//     dword of the channel-major value strip.
//   * key nibbles decode to normal fp16 (1 + u/64 or 16 + u/64), u = nibble
//     ^ 8, one bitop3 per pair of codes (no conversion instruction); the
//     MFMA accumulator starts at -sum(q * offset), which removes the
//     offsets, so the product is sum(q * nibble) / 64.
//   * value nibbles decode to fp16 subnormals (u * 2^-24 or u * 2^-20, no
//     implicit 1), the same one bitop3 per pair of codes.
//   * the score tile IS the A operand of P.V (same lane, same token order),
//     so P never leaves the lane; O += P.V per 16-channel block, plus one
//     MFMA against a constant column that tracks the values' +8.
//   * softmax in the exp2 domain with a lazy maximum: the running maximum
//     moves only when a score exceeds it by more than 2^8 (or a value scale
//     outgrows the fp16 headroom), so the accumulator rescale -- the only
//     cross-lane step -- is off the common path.
// The four waves' (m, l, acc) merge through LDS; the workgroup then exports
// one partial record. In the fused entry every live split takes a ticket from
// an agent-scope counter right after its prologue (the round trip hides under
// the strip loads); the split holding the last ticket combines. Every other
// split of its (seq, kv head) has started by then, so waiting for them is
// safe: they only stream, merge and store. Their records travel with the
// device-coherence bit, XOR-encoded so that an all-zero word means "not yet
// written" (no arithmetic result has the encoded bit pattern). The combiner
// exports its own record like the others, then polls all of them with
// coherent loads -- no store acknowledgement, no second atomic; the combine
// runs in split order whichever split combines -- rotates back, gates, stores
// BF16 and zeroes the records it consumed for the next call. A sequence with
// one live split finalises from LDS. No spinlock: the reference's L2-line lock
// (turboquant_splitk_reduce.cpp:279-350) is replaced by disjoint records and
// one ticket per workgroup.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/tq4.h"
#include "tq4_device.hpp"
#include "tq4_internal.hpp"

namespace tq4 {

// Phase stamps of the measurement build (make stamps: libtq4_stamps.so,
// bench.py --phases): thread 0 of the workgroup running work item b <
// kStampBlocks (blockIdx.x in the one-launch and partials grids; the queue
// item in the persistent kernel, read from LDS, which the others avoid)
// writes the 100 MHz realtime counter to slot [b][i] at each phase boundary -- 0 start, 1 phase-0 loads retired, 2 first strip pairs
// issued, 3 q operands built, 4 wave 0's strip loop done, 5 waves merged, 6
// record exported (a split that does not combine), 7 first row combined
// (poll complete + merge), 8 egress done (the combiner); the persistent
// kernel adds 9 its workgroup, 10 the item's start (before its coordinates),
// 11 its end, 12 its sequence and 13 its split. Slots an item does not reach
// keep an earlier launch's value. The product library is built without them.
#ifdef TQ4_DECODE_STAMPS
constexpr int kStampBlocks = 4096;
constexpr int kStampSlots = 16;
__device__ uint64_t g_decode_stamps[kStampBlocks * kStampSlots];
__shared__ uint32_t g_stamp_item;  // the persistent kernel's current item
#define TQ4_STAMP_ITEM(w)                       \
    do {                                        \
        if (threadIdx.x == 0) g_stamp_item = w; \
    } while (0)
#define TQ4_STAMP_AT(b, i, v)                                                          \
    do {                                                                               \
        if (threadIdx.x == 0) {                                                        \
            const uint32_t b_ = (b);                                                   \
            if (b_ < kStampBlocks) g_decode_stamps[b_ * kStampSlots + (i)] = (v);      \
        }                                                                              \
    } while (0)
// inside decode_item / finish_item (OWN is false only in the persistent kernel)
#define TQ4_STAMP(i, v) TQ4_STAMP_AT(OWN ? blockIdx.x : g_stamp_item, i, v)
#define TQ4_STAMP_P(i, v) TQ4_STAMP_AT(g_stamp_item, i, v)
#else
#define TQ4_STAMP_ITEM(w) \
    do {                  \
    } while (0)
#define TQ4_STAMP(i, v) \
    do {                \
    } while (0)
#define TQ4_STAMP_P(i, v) \
    do {                  \
    } while (0)
#endif
#define TQ4_NOW __builtin_amdgcn_s_memrealtime()

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint32_t kNib = 0x00F000F0u;   // a code at fp16 mantissa bits [7:4], both halves
constexpr uint32_t kCodeBase = 0x3C803C80u;  // fp16 1.0 outside kNib; the nibble sign bit inside
constexpr float kCodeOffset = 1.125f;    // fp16 key code value is 1 + u/64 = 1.125 + n/64
constexpr uint32_t kNibLo = 0x000F000Fu;     // a code at fp16 mantissa bits [3:0], both halves
constexpr uint32_t kCodeBaseLo = 0x4C084C08u;  // fp16 16.0 outside kNibLo; the nibble sign bit inside
constexpr float kCodeOffsetLo = 16.125f;     // fp16 key code value is 16 + u/64 = 16.125 + n/64
constexpr float kKeyUnit = 64.0f;            // key codes step 1/64 (score units)
constexpr uint32_t kValBase = 0x00800080u;   // exponent 0: the nibble at [7:4] is u * 2^-20
constexpr uint32_t kValBaseLo = 0x00080008u; // exponent 0: the nibble at [3:0] is u * 2^-24
constexpr float kValueUnit = 16777216.0f;    // value codes step 2^-24 (product units)
constexpr float kTau = 8.0f;             // lazy-maximum headroom, log2 units
constexpr float kShiftLimit = 100.0f;    // bound of a row's product normalisation shift
constexpr float kXLimit = 32768.0f;      // a normalised product at or above this rescales (fp16 max 65504)
constexpr int kMassLimit = 100;          // log2 bound of a row's normalised mass after a rescale
constexpr uint32_t kBadStrip = 0xFFFFFFFFu;
constexpr uint32_t kFlagRotated = 1u;
constexpr int kHdrFloats = 544;          // m_x, l_x [16][4], q_exp[16], flags, wave flags[4], scale slots [4][64], 2^-sh [16][4], exact maxima [16][4]
constexpr uint32_t kPersistentMaxSeqs = 4096; // the persistent kernel stages two words per sequence
constexpr uint32_t kLptMaxSeqs = 1024;        // and a third (the last-split order) up to this many
constexpr int kStripSlots = TQ4_MAX_SPLIT_STRIPS + 4;  // staged window rows + padding

// The thread index through an empty asm statement: address arithmetic
// derived from it is computed where it is used rather than once per kernel
// and held in registers across the strip loop (the kernels run at 256
// registers per wave, and a spilled address reloaded between items would
// wait for every load in flight).
__device__ __forceinline__ int fresh_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Eight value codes of one dword as fp16 subnormals, u = nibble ^ 8 (the
// code plus 8); halves in nibble order 0,4,1,5,2,6,3,7 (every operand built
// against this table uses that order). Each pair is one v_bitop3:
// (bits & mask) ^ base, truth table 0x6A over S0 = bits, S1 = mask, S2 =
// base, the base flipping the nibble's sign bit under a zero exponent. Under
// a zero exponent there is no implicit leading 1, so the only offset is the
// code's +8: nibbles 1,5 and 3,7 sit at mantissa bits [7:4] and are u *
// 2^-20, nibbles 0,4 and 2,6 at bits [3:0] are u * 2^-24 -- the caller
// builds the odd nibbles' A operands with 2^-4 in their exponent, so every
// product is P'vs * u * 2^-24.
__device__ __forceinline__ h8_t value_codes8(uint32_t w)
{
    const uint32_t w8 = w >> 8;
    const uint32_t p04 = __builtin_amdgcn_bitop3_b32(w, kNibLo, kValBaseLo, 0x6A);
    const uint32_t p15 = __builtin_amdgcn_bitop3_b32(w, kNib, kValBase, 0x6A);
    const uint32_t p26 = __builtin_amdgcn_bitop3_b32(w8, kNibLo, kValBaseLo, 0x6A);
    const uint32_t p37 = __builtin_amdgcn_bitop3_b32(w8, kNib, kValBase, 0x6A);
    return __builtin_bit_cast(h8_t, u4_t{p04, p15, p26, p37});
}

// Eight key codes of one dword as normal fp16, in the same nibble order and
// with the same one shift: nibbles 1,5 and 3,7 at mantissa bits [7:4] under
// an fp16 1.0 are 1 + u/64, nibbles 0,4 and 2,6 at bits [3:0] under an fp16
// 16.0 are 16 + u/64 (the same step). The score's start value removes both
// offsets; they cancel inside each pair's score, so the larger one costs
// nothing that accumulates across the split.
__device__ __forceinline__ h8_t key_codes8(uint32_t w)
{
    const uint32_t w8 = w >> 8;
    const uint32_t p04 = __builtin_amdgcn_bitop3_b32(w, kNibLo, kCodeBaseLo, 0x6A);
    const uint32_t p15 = __builtin_amdgcn_bitop3_b32(w, kNib, kCodeBase, 0x6A);
    const uint32_t p26 = __builtin_amdgcn_bitop3_b32(w8, kNibLo, kCodeBaseLo, 0x6A);
    const uint32_t p37 = __builtin_amdgcn_bitop3_b32(w8, kNib, kCodeBase, 0x6A);
    return __builtin_bit_cast(h8_t, u4_t{p04, p15, p26, p37});
}

__device__ __forceinline__ f4_t mfma32(h8_t a, h8_t b, f4_t c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Reductions over the four lanes l, l^16, l^32, l^48 (one MFMA column).
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

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, xor_lanes(v, m));
    return v;
}

// One pair's operands for one lane (n = lane & 15, g = lane >> 4).
template <int D>
struct PairRegs {
    uint32_t k1[D / 32];  // T1 key row (token of row n), channels g*d/4 .. +d/4
    uint32_t k2[D / 32];  // T2 key row
    uint32_t v[D / 16];   // value strip g>>1: 16 B chunks, channels n*d/16 + 4q + 2*(g&1) + {0,1}
    float sc;             // one scale: plane g&1, strip g>>1, token n
};

template <int D>
__device__ __forceinline__ void load_row_chunk(uint32_t (&k)[D / 32], const int8_t* src)
{
    if constexpr (D == 64) {
        const uint2 w = *(const uint2*)src;
        k[0] = w.x;
        k[1] = w.y;
    } else {
#pragma unroll
        for (int i = 0; i < D / 128; ++i) {
            const uint4 w = *(const uint4*)(src + 16 * i);
            k[4 * i + 0] = w.x;
            k[4 * i + 1] = w.y;
            k[4 * i + 2] = w.z;
            k[4 * i + 3] = w.w;
        }
    }
}


// Combine layout of one wave over one (seq, q head) row: lane c = lane & 31
// owns channels c*CC .. c*CC+CC-1 (CC = d/32); ks = lane >> 5 takes the
// splits of parity ks of every round of 2*NS, so a round costs each lane NS
// (m, l) loads and NS CC-float loads, all in flight together (one memory
// round trip per round; NS = 16 covers 32 splits at once). Slots past K
// load split K-1 (in range, already required) and are selected out.
//
// LSE-combine the K partial records [m, l, 0, 0, acc[d]] at rr (stride d+4)
// in split order, leaving acc / L in v (0 when L == 0).
// (tests/common/l2_atomic_oracle.hpp:156-176; identity :100-108)
// FUSED: the records are encoded; a chunk is reloaded until none of its words
// is zero (at most poll_limit times; a chunk still incomplete then adds one
// to *timeouts), then zeroed for the next call.
// own_k < K: the calling split's own record is not in memory. Its encoded
// words come from own(h, a), in this lane's combine layout, called once after
// the first chunk's loads are issued (so it runs under their round trip);
// they replace that slot's loaded words, and the combine is the same as if
// the record had been stored and loaded.
template <int D, bool FUSED, int NS = 8, class Own>
__device__ void combine_records(const float* rr, uint32_t K, int lane, float (&v)[D / 32],
                                uint32_t own_k, Own&& own, uint32_t poll_limit = 1,
                                uint32_t* timeouts = nullptr)
{
    constexpr int CC = D / 32;
    constexpr int LD = CC >= 4 ? 4 : CC;  // floats per load
    constexpr int RS = D + 4;
    const __amdgpu_buffer_rsrc_t rsrc = records_rsrc(rr);
    const int c = lane & 31, ks = lane >> 5;
    const uint32_t x = FUSED ? kRecMagic : 0u;
    float M = -INFINITY, L = 0.0f, a[CC];
    uint32_t oh[2] = {0u, 0u}, oa[CC];
#pragma unroll
    for (int j = 0; j < CC; ++j) a[j] = 0.0f, oa[j] = 0u;
    // Zero a chunk's records, so the next call starts from "not written"
    // (slots past K zero split K-1 again).
    auto zero_chunk = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const uint32_t k = k0 + ks + 2 * i;
            const uint32_t off0 = (k < K ? k : K - 1) * RS * 4u;
            __builtin_amdgcn_raw_buffer_store_b64(rec_u2_t{0u, 0u}, rsrc, off0, 0,
                                                  kCachePolicySc1);
#pragma unroll
            for (int j = 0; j < CC; j += LD) {
                const uint32_t off = off0 + 4u * (4 + c * CC + j);
                if constexpr (LD == 4)
                    __builtin_amdgcn_raw_buffer_store_b128(rec_u4_t{0u, 0u, 0u, 0u}, rsrc, off,
                                                           0, kCachePolicySc1);
                else
                    __builtin_amdgcn_raw_buffer_store_b64(rec_u2_t{0u, 0u}, rsrc, off, 0,
                                                          kCachePolicySc1);
            }
        }
    };
    for (uint32_t k0 = 0; k0 < K; k0 += 2 * NS) {
        uint32_t roff[NS];
        bool vi[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const uint32_t k = k0 + ks + 2 * i;
            vi[i] = k < K;
            roff[i] = (vi[i] ? k : K - 1) * RS * 4u;
        }
        uint32_t hw[NS][2], aw[NS][CC];
        for (uint32_t it = 0;; ++it) {
            asm volatile("" ::: "memory");  // every poll reloads
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                rec_load<2, FUSED>(rsrc, roff[i], hw[i]);
#pragma unroll
                for (int j = 0; j < CC; j += LD)
                    rec_load<LD, FUSED>(rsrc, roff[i] + 4u * (4 + c * CC + j), &aw[i][j]);
            }
            if constexpr (!FUSED) break;
            if (k0 == 0 && it == 0) own(oh, oa);
            // the own slot (wave-uniform: slot i_own of lane parity p_own)
            if (own_k >= k0 && own_k < k0 + 2 * NS) {
                const uint32_t i_own = (own_k - k0) >> 1;
                const bool here = ks == (int)((own_k - k0) & 1);
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    if (i == (int)i_own) {
                        hw[i][0] = here ? oh[0] : hw[i][0];
                        hw[i][1] = here ? oh[1] : hw[i][1];
#pragma unroll
                        for (int j = 0; j < CC; ++j) aw[i][j] = here ? oa[j] : aw[i][j];
                    }
                }
            }
            // slots past K are not waited for (they may alias the own slot)
            uint32_t mn = 0xffffffffu;
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                uint32_t ms = min(hw[i][0], hw[i][1]);
#pragma unroll
                for (int j = 0; j < CC; ++j) ms = min(ms, aw[i][j]);
                mn = vi[i] ? min(mn, ms) : mn;
            }
            if (!__any(mn == 0u)) break;
            if (it + 1 >= poll_limit) {  // gave up: the row is combined from what arrived
                if (lane == 0) count_timeout(timeouts);
                break;
            }
        }
        // The last chunk's records are zeroed at once (the stores complete
        // under the arithmetic below); earlier chunks' after the loop, since
        // the next chunk's poll would otherwise wait for their write
        // acknowledgements (stores and loads share one counter).
        if constexpr (FUSED) {
            if (k0 + 2 * NS >= K) zero_chunk(k0);
        }
        float mk[NS], Mc = -INFINITY;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            mk[i] = __uint_as_float(hw[i][0] ^ x) * kLog2e;
            Mc = fmaxf(Mc, vi[i] ? mk[i] : -INFINITY);
        }
        Mc = fmaxf(Mc, xor_lanes(Mc, 32));  // the other parity
        const float Mn = fmaxf(M, Mc);
        const float sc = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        float lw = 0.0f;
#pragma unroll
        for (int j = 0; j < CC; ++j) a[j] *= sc;
        if (k0 + 2 * NS <= K) {
            // every slot of the chunk holds a split (wave-uniform): one
            // decode and one fma per word, no select
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const float w = __builtin_amdgcn_exp2f(mk[i] - Mn);
                lw = fmaf(__uint_as_float(hw[i][1] ^ x), w, lw);
#pragma unroll
                for (int j = 0; j < CC; ++j) a[j] = fmaf(__uint_as_float(aw[i][j] ^ x), w, a[j]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const float w = __builtin_amdgcn_exp2f(mk[i] - Mn);
                lw += vi[i] ? __uint_as_float(hw[i][1] ^ x) * w : 0.0f;
#pragma unroll
                for (int j = 0; j < CC; ++j)
                    a[j] += vi[i] ? __uint_as_float(aw[i][j] ^ x) * w : 0.0f;
            }
        }
        L = L * sc + (lw + xor_lanes(lw, 32));
        M = Mn;
    }
    if constexpr (FUSED) {
        for (uint32_t k0 = 0; k0 + 2 * NS < K; k0 += 2 * NS) zero_chunk(k0);
    }
    // the two split parities
#pragma unroll
    for (int j = 0; j < CC; ++j) a[j] += xor_lanes(a[j], 32);
    const float inv = L == 0.0f ? 0.0f : __builtin_amdgcn_rcpf(L);
#pragma unroll
    for (int j = 0; j < CC; ++j) v[j] = a[j] * inv;
}

// Egress of one normalised row in the combine layout (lane c = lane & 31
// owns channels c*CC ..; both halves hold the row): optionally Pi^T and
// 1/sqrt(d), optionally the gate, BF16 RNE; lanes 0..31 store.
template <int D>
__device__ void egress_row(float (&v)[D / 32], const float (&sg)[D / 32], const float (&gt)[D / 32],
                           uint16_t* out_row, float inv_sqrt_len, uint32_t stage, int lane)
{
    constexpr int CC = D / 32;
    const int c = lane & 31;
    if (stage >= 1) {
        rotate_egress<D, CC>(v, sg, c);
#pragma unroll
        for (int j = 0; j < CC; ++j) v[j] *= inv_sqrt_len;
        if (stage == 2) {
#pragma unroll
            for (int j = 0; j < CC; ++j) v[j] = v[j] / (1.0f + expf(-gt[j]));
        }
    }
    uint32_t pk[CC / 2];
#pragma unroll
    for (int j = 0; j < CC / 2; ++j)
        pk[j] = f32_to_bf16(v[2 * j]) | (f32_to_bf16(v[2 * j + 1]) << 16);
    if (lane < 32) {
        uint16_t* dst = out_row + c * CC;
        if constexpr (CC == 8)
            *(uint4*)dst = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        else if constexpr (CC == 4)
            *(uint2*)dst = make_uint2(pk[0], pk[1]);
        else
            *(uint32_t*)dst = pk[0];
    }
}

// The combine layout's signs and gate values of one lane.
template <int D>
__device__ __forceinline__ void load_lane_floats(const float* src, int lane, float (&x)[D / 32])
{
    constexpr int CC = D / 32;
    const float* p = src + (lane & 31) * CC;
    if constexpr (CC >= 4) {
#pragma unroll
        for (int j = 0; j < CC; j += 4) {
            const float4 f = *(const float4*)(p + j);
            x[j] = f.x;
            x[j + 1] = f.y;
            x[j + 2] = f.z;
            x[j + 3] = f.w;
        }
    } else {
        const float2 f = *(const float2*)p;
        x[0] = f.x;
        x[1] = f.y;
    }
}

__host__ __device__ constexpr size_t region_floats(uint32_t G, uint32_t D)
{
    // q staging [G][D + 4], then the four waves' rows [4][G][D], disjoint: a
    // wave without pairs parks its rows while the others may still be
    // reading q for their operands
    return (size_t)G * (D + 4) + 4ull * G * D;
}

// One wave's streaming state over the q rows of one item. Scores t = s - mo
// with s = score * log2(e) (log2 units), mo = m_used - sh (before a live
// row's first rescale mo = 0, so that t = s): P' = exp2(t) =
// P * 2^sh, and the MFMA operand is the product P' * vscale in fp16. The
// row's shift sh is set at each rescale so that the largest product of that
// pair lands in [1, 2): every product that matters for the row's sum then
// fits fp16 (one below 2^-24 of the largest is below 2^-24 of the sum),
// whatever the spread of the value scales; the accumulators are FP32.
template <int D>
struct RowState {
    f4_t acc[D / 16];
    f4_t cr;       // offset column: 8 * 2^-24 * sum P'vs per row
    float m_used;  // the row maximum in use (log2 units)
    float smax;    // partials only: this lane's exact maximum score (log2 units)
    float sh, mo, lpart, thr;
    float mo4;     // mo + 4: the odd tokens' exponent offset (value_codes8)
    bool virgin;   // no rescale yet in this stream (wave-uniform)

    __device__ __forceinline__ void reset(bool row_live)
    {
#pragma unroll
        for (int b = 0; b < D / 16; ++b) acc[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        cr = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        // A padded row stays silent (mo = +inf: every t is -inf). A live
        // row starts with a finite mo (t = s exactly) and thr = -inf, so its
        // first pair holding a live token always rescales.
        m_used = row_live ? -INFINITY : INFINITY;
        smax = -INFINITY;
        sh = 0.0f;
        mo = row_live ? 0.0f : INFINITY;
        mo4 = mo + 4.0f;
        lpart = 0.0f;
        thr = row_live ? -INFINITY : kTau;
        virgin = true;
    }
};

// This lane's B operands (q head n, channels g4*d/4 ..) in the key_codes8
// channel order, the MFMA start value that removes the code offsets, and the
// score factor 64 * log2(e) * 2^q_exp (1 for a padded row, whose scores the
// infinite mo silences: a factor of 0 would make 0 * -inf of a dead token).
template <int D>
struct QOps {
    h8_t qop[D / 32];
    f4_t bias4;
    float cf;
    bool row_live;
};

// One pair (two strips, 32 tokens) of one wave into its rows. masked: the
// pair holds dead tokens -- those at or past live_rel tokens from the pair's
// start, and every token of this lane's value strip when strip_ok is false;
// a dead token is overwritten (score -inf, value scale 0), never multiplied
// (its payload may be NaN). EXACT (the partials entry): also track the exact
// maximum score, which the exported record's m must be (the lazy maximum
// may sit up to kTau below it).
template <int D, bool EXACT = false>
__device__ __forceinline__ void process_pair(RowState<D>& st, const QOps<D>& qo,
                                             const PairRegs<D>& r, float* sc_wave, int lane,
                                             bool masked, uint32_t live_rel, bool strip_ok)
{
    constexpr int NJ = D / 32;
    constexpr int NB = D / 16;
    const int half = (lane >> 4) & 1, sp = lane >> 5;
    // the value codes' +8 in each slot's unit (value_codes8): 8 * 2^-24 for
    // nibbles 0,4,2,6, 8 * 2^-20 for the odd nibbles, whose P' carries 2^-4
    // -- so the column sums 8 * 2^-24 * P'vs over the row
    const _Float16 oe = (_Float16)0x1p-21f, oo = (_Float16)0x1p-17f;
    const h8_t offset_col = h8_t{oe, oe, oo, oo, oe, oe, oo, oo};
    f4_t c1 = qo.bias4, c2 = qo.bias4;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        c1 = mfma32(key_codes8(r.k1[j]), qo.qop[j], c1);
        c2 = mfma32(key_codes8(r.k2[j]), qo.qop[j], c2);
    }
    // scales through the wave's LDS slot: key scales of this lane's 8
    // tokens (strip sp, tokens 8*half..) at [32sp + 8half], values at +16
    sc_wave[lane] = r.sc;
    const f4_t ks1 = *(const f4_t*)(sc_wave + 32 * sp + 8 * half);
    const f4_t ks2 = *(const f4_t*)(sc_wave + 32 * sp + 8 * half + 4);
    const f4_t vs1 = *(const f4_t*)(sc_wave + 32 * sp + 16 + 8 * half);
    const f4_t vs2 = *(const f4_t*)(sc_wave + 32 * sp + 16 + 8 * half + 4);
    bool live[8];
    if (masked) {
        // token of value i from the pair's start: strip sp, 8*half + (i&3) + 4*(i>>2)
        const uint32_t tb = 16 * sp + 8 * half;
#pragma unroll
        for (int i = 0; i < 8; ++i) live[i] = strip_ok && tb + (i & 3) + 4 * (i >> 2) < live_rel;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) live[i] = true;
    }
    // raw scores (the row's factor cf > 0 turns them into log2 units inside
    // each exponent's FMA) and value scales; a dead token is overwritten
    float sr[8], vs[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sr[i] = live[i] ? c1[i] * ks1[i] : -INFINITY;
        sr[4 + i] = live[4 + i] ? c2[i] * ks2[i] : -INFINITY;
        vs[i] = live[i] ? vs1[i] : 0.0f;
        vs[4 + i] = live[4 + i] ? vs2[i] : 0.0f;
    }
    // Rescale when a score passes the lazy maximum by kTau, or when a
    // product could reach kXLimit: exp2(tmax) * vmax bounds every
    // product (one exp per lane; the products themselves are formed
    // after the branch, so nothing of them stays live across it). cf > 0,
    // so cf times the largest raw score is the largest score.
    float rmax = -INFINITY, vmax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        rmax = fmaxf(rmax, sr[i]);
        vmax = fmaxf(vmax, vs[i]);
    }
    if constexpr (EXACT) st.smax = fmaxf(st.smax, qo.cf * rmax);
    // a live row's mo is finite; a padded row's is +inf
    const float tmax = fmaf(qo.cf, rmax, -st.mo);
    if (__builtin_expect(
            __any(tmax > st.thr || __builtin_amdgcn_exp2f(tmax) * vmax >= kXLimit), 0)) {
        // Move the row maximum and re-normalise the row's products.
        float sc8[8];  // scores, log2 units
#pragma unroll
        for (int i = 0; i < 8; ++i) sc8[i] = qo.cf * sr[i];
        float smax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) smax = fmaxf(smax, sc8[i]);
        smax = col_max(smax);
        const float mn = qo.row_live ? fmaxf(st.m_used, smax) : st.m_used;
        // the pair's largest product under the new maximum, unnormalised
        float ymax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ymax = fmaxf(ymax, __builtin_amdgcn_exp2f(sc8[i] - mn) * vs[i]);
        ymax = col_max(ymax);
        if (st.virgin) {
            // The stream's first rescale: nothing is accumulated yet
            // (acc, cr and lpart are zero), so there is no mass to keep
            // and nothing to re-scale -- only the row's maximum and shift.
            float shn = st.sh;
            if (qo.row_live && ymax > 0.0f)
                shn = fminf(fmaxf(-(float)exponent_of(ymax), -kShiftLimit), kShiftLimit);
            st.m_used = mn;
            st.mo = mn - shn;
            st.mo4 = st.mo + 4.0f;
            st.sh = shn;
            st.thr = kTau + shn;
            st.virgin = false;
        } else {
            // (lane indices of this rare path are taken afresh: held across
            // the strip loop they would cost registers every pair)
            const int ln = fresh_tid() & 63;
            const int n = ln & 15, g4 = ln >> 4;
            // the row's mass so far (its offset-column sum, P.V layout row n)
            const int src = 16 * (n >> 2);
            const float r0 = __shfl(st.cr[0], src, 64), r1 = __shfl(st.cr[1], src, 64);
            const float r2 = __shfl(st.cr[2], src, 64), r3 = __shfl(st.cr[3], src, 64);
            const int k3 = n & 3;
            const float crow = k3 == 0 ? r0 : k3 == 1 ? r1 : k3 == 2 ? r2 : r3;
            float shn = st.sh;
            if (qo.row_live && ymax > 0.0f) {
                shn = fminf(fmaxf(-(float)exponent_of(ymax), -kShiftLimit), kShiftLimit);
                // keep the old mass, moved to the new units, inside FP32
                if (st.m_used != -INFINITY && crow > 0.0f) {
                    const float lm = (float)exponent_of(crow) + (shn - st.sh) + (st.m_used - mn);
                    if (lm > (float)kMassLimit) shn -= ceilf(lm - (float)kMassLimit);
                }
            }
            const float mon = mn - shn;
            float f = 1.0f;
            if (qo.row_live) f = __builtin_amdgcn_exp2f(st.mo - mon);
            st.lpart *= f;
            float fr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fr[i] = __shfl(f, 4 * g4 + i, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int b = 0; b < NB; ++b) st.acc[b][i] *= fr[i];
                st.cr[i] *= fr[i];
            }
            st.m_used = mn;
            st.mo = mon;
            st.mo4 = mon + 4.0f;
            st.sh = shn;
            st.thr = kTau + shn;
        }
    }
    // A dead token's t = s - mo is -inf, and so is every t of a padded row
    // (mo = +inf); a live row's mo is always finite, so no t is NaN.
    _Float16 x[8];
    float pr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // an odd token's code unit is 16 times an even one's
        // (value_codes8): its P' carries 2^-4, and counts 16 times in l
        pr[i] = __builtin_amdgcn_exp2f(fmaf(qo.cf, sr[i], (i & 1) ? -st.mo4 : -st.mo));
        x[i] = (_Float16)(pr[i] * vs[i]);
    }
    st.lpart += (fmaf(16.0f, pr[1], pr[0]) + fmaf(16.0f, pr[3], pr[2])) +
                (fmaf(16.0f, pr[5], pr[4]) + fmaf(16.0f, pr[7], pr[6]));
    // A operand in the value_codes8 token order: (T1[0], T2[0], T1[1], T2[1], ...)
    const h8_t P = h8_t{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
    // B operands: block b = 4q + 2hb + e is channel n*d/16 + b. The lane
    // pair (half 0, half 1) swaps so each holds its own 8-token half:
    // permlane16_swap(x, y) leaves the even row's x plus the odd row's
    // copy of the even row's y in its first result (block hb = 0), and
    // the odd row's x copy plus the odd row's y in its second (hb = 1).
#pragma unroll
    for (int q = 0; q < NB / 4; ++q) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const auto sw = __builtin_amdgcn_permlane16_swap(r.v[4 * q + 2 * e],
                                                             r.v[4 * q + 2 * e + 1], false, false);
            st.acc[4 * q + e] = mfma32(P, value_codes8(sw[0]), st.acc[4 * q + e]);
            st.acc[4 * q + 2 + e] = mfma32(P, value_codes8(sw[1]), st.acc[4 * q + 2 + e]);
        }
    }
    st.cr = mfma32(P, offset_col, st.cr);
}

// Staged q rows are kQRow floats apart: the pad of one float4 puts the
// same column of eight consecutive rows on eight different bank quads, so
// build_qops' row-strided float4 reads are conflict-free (D apart, they all
// fall on one quad).
template <int D>
constexpr int kQRow = D + 4;

// Rotate this wave's q rows (g = wave, wave + 4, ...; lane owns channels
// lane*CPL ..), fold inv_sqrt_len and the softmax scale, normalise each row
// by a power of two and stage it in q_st [G][kQRow<D>] (exponent in q_exp[g]).
template <int D>
__device__ __forceinline__ void stage_q_rows(const DecodeParams& p,
                                             const uint16_t (&qraw)[4][D / 64],
                                             const float (&sg)[D / 64], bool rotate, float* q_st,
                                             int* q_exp, int wave, int lane)
{
    constexpr int CPL = D / 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t g = wave + kWaves * i;
        if (g >= p.G) continue;
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[j] = bf16_to_f32(qraw[i][j]);
        if (rotate) {
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
        a = wave_max(a);
        const int kq = a > 0.0f ? exponent_of(a) : 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) q_st[g * kQRow<D> + lane * CPL + j] = ldexpf(v[j], -kq);
        if (lane == 0) q_exp[g] = kq;
    }
}

// This lane's operands from the staged rows (after a barrier).
template <int D>
__device__ __forceinline__ void build_qops(QOps<D>& qo, const float* q_st, const int* q_exp,
                                           uint32_t G, int lane)
{
    constexpr int NJ = D / 32;
    const int n = lane & 15, g4 = lane >> 4;
    qo.row_live = (uint32_t)n < G;
    float bias = 0.0f;  // sum of q times each key_codes8 half's offset (negated below)
    qo.cf = 1.0f;
    if (qo.row_live) {
        const float* qrow = q_st + n * kQRow<D> + g4 * (D / 4);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const float4 lo = *(const float4*)(qrow + 8 * j);
            const float4 hi = *(const float4*)(qrow + 8 * j + 4);
            const h8_t h = h8_t{(_Float16)lo.x, (_Float16)hi.x, (_Float16)lo.y, (_Float16)hi.y,
                                (_Float16)lo.z, (_Float16)hi.z, (_Float16)lo.w, (_Float16)hi.w};
            qo.qop[j] = h;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                bias += (float)h[e] * ((e & 2) == 0 ? kCodeOffsetLo : kCodeOffset);
        }
        qo.cf = ldexpf(kKeyUnit * kLog2e, q_exp[n]);
    } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) qo.qop[j] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
    bias = -col_sum(bias);
    qo.bias4 = f4_t{bias, bias, bias, bias};
}

// Park one wave's rows for the merge: (m, l, 2^-sh) per row at [row][wave]
// (one 16-byte read gives a row's four waves), with EXACT the row's exact
// maximum score at t_x, and the raw rows (offset column removed) at part
// [wave][G][D].
template <int D, bool EXACT>
__device__ __forceinline__ void park_rows(const RowState<D>& st, bool row_live, float* m_x,
                                          float* l_x, float* u_x, float* t_x, float* part,
                                          uint32_t G, int wave, int lane)
{
    constexpr int NB = D / 16;
    const int n = lane & 15, g4 = lane >> 4;
    const float lsum = col_sum(st.lpart);
    if constexpr (EXACT) {
        const float tm = col_max(st.smax);
        if (g4 == 0) t_x[n * kWaves + wave] = row_live ? tm : -INFINITY;
    }
    if (g4 == 0) {
        m_x[n * kWaves + wave] = row_live ? st.m_used : -INFINITY;
        l_x[n * kWaves + wave] = lsum;
        u_x[n * kWaves + wave] = ldexpf(1.0f, -(int)st.sh);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = 4 * g4 + i;
        if (r < G) {
            float* dst = part + ((size_t)wave * G + r) * D + n * NB;  // channel n*d/16 + b
#pragma unroll
            for (int b = 0; b < NB; ++b) dst[b] = st.acc[b][i] - st.cr[i];
        }
    }
}

// The end of one work item: merge the four waves' rows, then MODE 0 exports
// the partial record; MODE 1 takes the split's place in the fused combine
// (export, or finalise from LDS when it is the only live split, or combine as
// the last ticket). region: the item's q staging / merge region.
template <int D, int MODE, bool OWN>
__device__ __forceinline__ void finish_item(const DecodeParams& p, uint32_t seq, uint32_t kvh,
                                            uint32_t split, uint32_t k_live, uint32_t ticket,
                                            const RowState<D>& st, bool row_live, float* region)
{
    constexpr int RS = D + 4;  // record stride in floats
    extern __shared__ float smem[];
    const uint32_t G = p.G;
    float* m_x = smem;               // [16][4] (row, wave)
    float* l_x = smem + 64;          // [16][4]
    int* flag = (int*)(smem + 144);  // the combiner / withheld-record flags
    float* u_x = smem + 416;         // [16][4] (row, wave) 2^-sh
    float* t_x = smem + 480;         // [16][4] (row, wave) exact maximum (partials)
    const int tid = fresh_tid(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // ---- merge the four waves. Each parks its raw rows (offset column
    // removed) and (m, l, 2^-sh) in LDS; then every output float4 combines
    // the four copies with the row's common maximum.
    float* part = region + G * kQRow<D>;  // [kWaves][G][D], past the q staging rows
    park_rows<D, MODE == 0>(st, row_live, m_x, l_x, u_x, t_x, part, G, wave, lane);
    if constexpr (MODE == 1) {
        if (p.K > 1 && tid == 0) {
            // The last ticket combines; every live split of this (seq, kv
            // head) took its ticket before it, so all of them are running.
            // Bit 1: the test hook's withheld record (the first ticket's,
            // never the combiner's when more than one split is live).
            const int last = ticket == k_live - 1;
            if (last)
                __hip_atomic_store(p.counters + ((size_t)seq * p.Hkv + kvh) * kTicketStride, 0u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last | (p.withhold && ticket == 0 && !last ? 2 : 0);
        }
    }
    lds_barrier();
    TQ4_STAMP(5, TQ4_NOW);
    TQ4_STAMP(6, 0);
    TQ4_STAMP(7, 0);
    TQ4_STAMP(8, 0);
    // Per-wave weights of row r (exp2(m_w - M) * 2^-sh_w), the row's M and L;
    // branch-free: a wave with no live token gets exp2(-inf) = 0.
    auto row_weights = [&](uint32_t r, float (&f)[kWaves], float& M, float& L) {
        const float4 m4 = *(const float4*)(m_x + r * kWaves);
        const float4 l4 = *(const float4*)(l_x + r * kWaves);
        const float4 u4 = *(const float4*)(u_x + r * kWaves);
        const float mw[kWaves] = {m4.x, m4.y, m4.z, m4.w};
        const float lw[kWaves] = {l4.x, l4.y, l4.z, l4.w};
        const float uw[kWaves] = {u4.x, u4.y, u4.z, u4.w};
        M = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
        if constexpr (MODE == 0) {
            // the record's m is the row's exact running maximum, as the
            // contract has it: every wave's weight moves down to it
            const float4 t4 = *(const float4*)(t_x + r * kWaves);
            M = fmaxf(fmaxf(t4.x, t4.y), fmaxf(t4.z, t4.w));
        }
        L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float d = (mw[w] == -INFINITY) ? -INFINITY : mw[w] - M;
            f[w] = __builtin_amdgcn_exp2f(d) * uw[w];
            L += lw[w] * f[w];
        }
    };
    const uint32_t outs4 = G * D / 4;  // float4 outputs
    auto combined4 = [&](uint32_t e4, const float (&f)[kWaves]) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float4 x = *(const float4*)(part + (size_t)w * G * D + 4 * e4);
            const float fw = f[w] * kValueUnit;
            v.x += x.x * fw;
            v.y += x.y * fw;
            v.z += x.z * fw;
            v.w += x.w * fw;
        }
        return v;
    };

    constexpr int CC = D / 32;
    if constexpr (MODE == 0) {
        // ---- export one record per q head: [m (natural log), l, 0, 0, acc].
        const __amdgpu_buffer_rsrc_t rsrc = records_rsrc(
            p.records + (((size_t)seq * p.Hq + (size_t)kvh * G) * p.K + split) * RS);
        const uint32_t row_bytes = p.K * RS * 4u;
        for (uint32_t e4 = tid; e4 < outs4; e4 += kThreads) {
            const uint32_t r = 4 * e4 / D, ch = 4 * e4 % D;
            float f[kWaves], M, L;
            row_weights(r, f, M, L);
            const float4 v = combined4(e4, f);
            const float vv[4] = {v.x, v.y, v.z, v.w};
            rec_store<4, false>(rsrc, r * row_bytes + (4 + ch) * 4u, vv);
            if (ch == 0) {
                const float h[4] = {M == -INFINITY ? kMasked : M * kLn2, L, 0.0f, 0.0f};
                rec_store<4, false>(rsrc, r * row_bytes, h);
            }
        }
        return;
    } else {
        // One live split (K == 1, or a sequence shorter than one split's
        // window) finalises from LDS; otherwise every split exports and the
        // last ticket combines.
        const bool local = p.K == 1 || k_live == 1;
        const int fl = *flag;
        const bool combiner = local || (fl & 1);
        float es[CC];
        if (!local && (fl & 2)) return;  // test hook: this record is never written
        if (!local && (!combiner || !OWN)) {
            // ---- export this split's encoded record.
            const __amdgpu_buffer_rsrc_t rsrc = records_rsrc(
                p.records + (((size_t)seq * p.Hq + (size_t)kvh * G) * p.K + split) * RS);
            const uint32_t row_bytes = p.K * RS * 4u;
            for (uint32_t e4 = tid; e4 < outs4; e4 += kThreads) {
                const uint32_t r = 4 * e4 / D, ch = 4 * e4 % D;
                float f[kWaves], M, L;
                row_weights(r, f, M, L);
                const float4 v = combined4(e4, f);
                const float vv[4] = {v.x, v.y, v.z, v.w};
                rec_store<4, true>(rsrc, r * row_bytes + (4 + ch) * 4u, vv);
                if (ch == 0) {
                    const float h[4] = {M == -INFINITY ? kMasked : M * kLn2, L, 0.0f, 0.0f};
                    rec_store<4, true>(rsrc, r * row_bytes, h);
                }
            }
            TQ4_STAMP(6, TQ4_NOW);
            if (!combiner) return;
        }
        if (!local) {
            // ---- the combiner: poll the records of its rows and combine
            // them. With OWN its own record is never stored: its words are
            // made from LDS (the export's arithmetic, in the combine layout)
            // while the first poll is in flight. The sign and gate loads
            // ride with that poll.
            if (p.output_stage >= 1) load_lane_floats<D>(p.pi_signs, lane, es);
            for (uint32_t g = wave; g < G; g += kWaves) {
                const size_t qh = (size_t)seq * p.Hq + kvh * G + g;
                float gt[CC];
                if (p.output_stage == 2) load_lane_floats<D>(p.gate + qh * D, lane, gt);
                auto own = [&](uint32_t (&h)[2], uint32_t (&a)[CC]) {
                    float f[kWaves], M, L;
                    row_weights(g, f, M, L);
                    h[0] = __float_as_uint(M == -INFINITY ? kMasked : M * kLn2) ^ kRecMagic;
                    h[1] = __float_as_uint(L) ^ kRecMagic;
                    if constexpr (CC >= 4) {
#pragma unroll
                        for (int j = 0; j < CC; j += 4) {
                            const float4 v = combined4((g * D + (lane & 31) * CC + j) / 4, f);
                            a[j] = __float_as_uint(v.x) ^ kRecMagic;
                            a[j + 1] = __float_as_uint(v.y) ^ kRecMagic;
                            a[j + 2] = __float_as_uint(v.z) ^ kRecMagic;
                            a[j + 3] = __float_as_uint(v.w) ^ kRecMagic;
                        }
                    } else {  // d = 64: the lane's two channels of a float4
                        const uint32_t ch = (lane & 31) * CC;
                        const float4 v = combined4((g * D + ch) / 4, f);
                        const bool hi = (ch & 2) != 0;
                        a[0] = __float_as_uint(hi ? v.z : v.x) ^ kRecMagic;
                        a[1] = __float_as_uint(hi ? v.w : v.y) ^ kRecMagic;
                    }
                };
                auto none = [](uint32_t(&)[2], uint32_t(&)[CC]) {};
                float v[CC];
                // 16 splits per chunk: wider chunks (32 per round trip)
                // measured slower at every split count from 17 to 64
                if constexpr (OWN)
                    combine_records<D, true, 8>(p.records + qh * p.K * RS, k_live, lane, v,
                                                split, own, p.poll_limit, p.timeouts);
                else
                    combine_records<D, true, 8>(p.records + qh * p.K * RS, k_live, lane, v, ~0u,
                                                none, p.poll_limit, p.timeouts);
                if (g == 0) TQ4_STAMP(7, TQ4_NOW);
                egress_row<D>(v, es, gt, p.out + qh * D, p.inv_sqrt_len, p.output_stage, lane);
            }
            TQ4_STAMP(8, TQ4_NOW);
            return;
        }
        if (p.output_stage >= 1) load_lane_floats<D>(p.pi_signs, lane, es);
        // ---- one live split: normalise into the wave-0 slice (each thread
        // reads and writes only its own float4), then the egress.
        for (uint32_t e4 = tid; e4 < outs4; e4 += kThreads) {
            float f[kWaves], M, L;
            row_weights(4 * e4 / D, f, M, L);
            float4 v = combined4(e4, f);
            const float inv = L == 0.0f ? 0.0f : 1.0f / L;
            v = L == 0.0f ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                          : make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
            *(float4*)(part + 4 * e4) = v;
        }
        lds_barrier();
        for (uint32_t g = wave; g < G; g += kWaves) {
            const size_t qh = (size_t)seq * p.Hq + kvh * G + g;
            float gt[CC];
            if (p.output_stage == 2) load_lane_floats<D>(p.gate + qh * D, lane, gt);
            float v[CC];
#pragma unroll
            for (int j = 0; j < CC; ++j) v[j] = part[g * D + (lane & 31) * CC + j];
            egress_row<D>(v, es, gt, p.out + qh * D, p.inv_sqrt_len, p.output_stage, lane);
        }
    }
}

// One (seq, kv head, split) work item: MODE 0 exports the partial record,
// MODE 1 is the fused path (ticket, export or local finish, combine).
// OWN (MODE 1): the combining split keeps its own record in registers instead
// of storing and polling it (the one-launch kernel; the persistent kernel
// stores it, which keeps that kernel's register budget).
struct NoHook {
    __device__ void operator()() const {}
};

template <int D, int MODE, bool OWN = true, class Hook = NoHook>
__device__ __forceinline__ void decode_item(const DecodeParams& p, const uint32_t seq,
                                            const uint32_t kvh, const uint32_t split,
                                            Hook&& after_issue = Hook())
{
    constexpr int CPL = D / 64;   // channels per lane in the row layout
    constexpr int NB = D / 16;    // P.V MFMAs (16-channel blocks)
    constexpr int NBUF = D >= 256 ? 2 : 3;
    extern __shared__ float smem[];

    const uint32_t G = p.G, S = p.S;
    int* q_exp = (int*)(smem + 128);         // [16]
    int* bad_w = (int*)(smem + 152);         // [4] per-wave invalid-page flags
    float* sc_wave = smem + 160 + 64 * (threadIdx.x >> 6);  // [4][64] per-wave scale slot
    uint32_t* strip_lds = (uint32_t*)(smem + kHdrFloats);  // [TQ4 max split strips + padding]
    float* region = smem + kHdrFloats + kStripSlots;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int n = lane & 15, g4 = lane >> 4;
    const int half = g4 & 1, sp = g4 >> 1;  // value/scale lanes: strip sp of the pair, tokens 8*half..

    // ---- phase 0: every small load -- context length, q rows, rotation
    // signs, the split's block-table window -- is issued before any strip
    // load and retired together.
    TQ4_STAMP(0, TQ4_NOW);
    const int32_t ctx_raw = p.context_lens[seq];
    const bool rotate = !(p.flags & kFlagRotated);
    uint16_t qraw[4][CPL];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t g = min((uint32_t)wave + kWaves * i, G - 1);  // branch-free
        const uint16_t* qr = p.q + ((size_t)seq * p.Hq + kvh * G + g) * D + lane * CPL;
#pragma unroll
        for (int j = 0; j < CPL; ++j) qraw[i][j] = qr[j];
    }
    float sg[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) sg[j] = 1.0f;
    if (rotate) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) sg[j] = p.pi_signs[lane * CPL + j];
    }
    // The split's window of the block table: Partition(max_blocks_per_seq,
    // splits, split) (turboquant_paged_decode_attention.cpp:1598-1624),
    // staged in LDS as the first cache row of every strip.
    uint32_t pb, pc;
    partition(p.max_blocks, p.K, split, pb, pc);
    const uint32_t spp = S / kStrip;
    const int32_t* tbl = p.block_tables + (size_t)seq * p.max_blocks + pb;
    // The window's first kThreads entries load beside the context length
    // (the window depends on the partition alone); which of them are live is
    // known once it returns.
    const int32_t phys_first = (uint32_t)tid < pc ? tbl[tid] : 0;
    uint32_t ctx = ctx_raw < 0 ? 0u : (uint32_t)ctx_raw;
    const uint64_t capacity = (uint64_t)p.max_blocks * S;
    if (ctx > capacity) ctx = (uint32_t)capacity;
    const uint64_t tok0 = (uint64_t)pb * S;
    uint32_t ltok = 0;  // live tokens of the window
    if (pc > 0 && ctx > tok0) {
        const uint64_t l = ctx - tok0;
        ltok = l < (uint64_t)pc * S ? (uint32_t)l : pc * S;
    }
    // Fused entry: splits past the context hold no live token. They publish
    // nothing -- the arrival count is the number of non-empty splits,
    // ceil(ceil(ctx / S) / width), which every workgroup of the sequence
    // derives from ctx alone -- and leave at once.
    // split >= that count exactly when the window starts at or past ctx
    // (the window starts at page split * width), a test without divisions.
    uint32_t k_live = p.K;
    if constexpr (MODE == 1) {
        if (p.K > 1) {
            // 32-bit: its division runs while the table window is in flight
            const uint32_t width = p.max_blocks / p.K + (p.max_blocks % p.K != 0u);
            const uint32_t ctx_pages = ctx / S + (ctx % S != 0u);
            k_live = ctx_pages / width + (ctx_pages % width != 0u);
            if (tok0 >= ctx) {
                if (ctx == 0 && split == 0) {
                    // empty context: the normalised context is 0 (l = 0)
                    float es[D / 32], gt[D / 32];
                    if (p.output_stage >= 1) load_lane_floats<D>(p.pi_signs, lane, es);
                    for (uint32_t g = wave; g < G; g += kWaves) {
                        float v[D / 32];
#pragma unroll
                        for (int j = 0; j < D / 32; ++j) v[j] = 0.0f;
                        const size_t qh = (size_t)seq * p.Hq + kvh * G + g;
                        if (p.output_stage == 2) load_lane_floats<D>(p.gate + qh * D, lane, gt);
                        egress_row<D>(v, es, gt, p.out + qh * D, p.inv_sqrt_len, p.output_stage,
                                      lane);
                    }
                }
                after_issue();  // exactly once per item, whichever way it leaves
                return;
            }
        }
    }
    int bad = 0;
    auto stage = [&](uint32_t t, uint32_t phys) {
        const bool ok = phys < p.P;
        if (!ok && t * S < ltok) bad = 1;  // page t holds a live token
        const uint32_t row = (phys * p.Hkv + kvh) * S;
        for (uint32_t s = 0; s < spp; ++s) strip_lds[t * spp + s] = ok ? row + kStrip * s : kBadStrip;
        // one padding row past the window: the second strip of a partial
        // last pair reads it (its tokens are masked)
        if (t == pc - 1) strip_lds[pc * spp] = ok ? row : 0u;
    };
    if ((uint32_t)tid < pc) stage(tid, (uint32_t)phys_first);
    for (uint32_t t = tid + kThreads; t < pc; t += kThreads) stage(t, (uint32_t)tbl[t]);
    // One barrier: every wave writes its own flag, so nothing needs clearing.
    {
        const int wb = __any(bad);
        if (lane == 0) bad_w[wave] = wb;
        lds_barrier();
        const int4 bw = *(const int4*)bad_w;
        bad = bw.x | bw.y | bw.z | bw.w;
    }
    // Every phase-0 load is complete here; saying so (vmcnt(0), expcnt and
    // lgkmcnt left at their maxima) keeps the compiler's wait analysis from
    // later waiting on them -- and so on the strip loads queued after them.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    TQ4_STAMP(1, TQ4_NOW);
    const uint32_t np_total = (ltok + 2 * kStrip - 1) / (2 * kStrip);
    const uint32_t np_full = bad ? 0u : ltok / (2 * kStrip);
    const uint32_t nws = pc * spp;  // strips in the window
    const size_t plane_floats = (size_t)p.P * p.Hkv * S;

    // Operands of pair gp (window strips 2gp, 2gp+1). `safe`: strips past the
    // window or on invalid pages read row 0 (their tokens are masked).
    auto fetch = [&](PairRegs<D>& r, uint32_t gp, bool safe) {
        const uint32_t s0 = 2 * gp;
        uint32_t sk = s0 + (n >> 3), sv = s0 + sp;
        if (safe) {
            sk = min(sk, nws - 1);
            sv = min(sv, nws - 1);
        }
        uint32_t rk = strip_lds[sk], rv = strip_lds[sv];
        if (safe) {
            rk = rk == kBadStrip ? 0u : rk;
            rv = rv == kBadStrip ? 0u : rv;
        }
        const uint32_t t1 = 8 * ((n >> 2) & 1) + (n & 3);
        const int8_t* kb = p.key_cache + (size_t)(rk + t1) * (D / 2) + g4 * (D / 8);
        load_row_chunk<D>(r.k1, kb);
        load_row_chunk<D>(r.k2, kb + 4 * (D / 2));
        // value strip: lane (n, half) takes 16 B chunks q = 0.. of channel
        // group n -- both token halves of channels n*d/16 + 4q + 2*half + {0,1}
        const int8_t* vb8 = p.value_cache + (size_t)rv * (D / 2) + n * (D / 2) + 16 * half;
#pragma unroll
        for (int q = 0; q < NB / 4; ++q) {
            const uint4 w = *(const uint4*)(vb8 + 32 * q);
            r.v[4 * q + 0] = w.x;
            r.v[4 * q + 1] = w.y;
            r.v[4 * q + 2] = w.z;
            r.v[4 * q + 3] = w.w;
        }
        // the pair's 64 scales, one per lane: plane `half`, strip sp, token n
        r.sc = p.scale_cache[(size_t)half * plane_floats + rv + n];
    };

    // ---- this wave's pairs are gp = wave + 4j. Without an invalid page at
    // most the window's last pair is partial (np_total - np_full <= 1); it
    // is gp = np_full, the LAST pair of wave np_full % 4, so the ring
    // prefetches it like the others (with clamped, "safe" indices) and only
    // its processing is masked. The first pairs go out before the q prologue.
    const bool tail_in_ring = !bad && np_total > np_full;
    const uint32_t np_ring = bad ? 0u : np_total;
    const uint32_t nw = np_ring > (uint32_t)wave ? (np_ring - wave + kWaves - 1) / kWaves : 0u;
    const bool tail_mine = tail_in_ring && (np_full & (kWaves - 1)) == (uint32_t)wave;
    const uint32_t nfw = tail_mine ? nw - 1 : nw;  // this wave's full pairs
    auto gp_of = [&](uint32_t j) { return (uint32_t)wave + kWaves * min(j, nw - 1); };
    PairRegs<D> b0, b1;
    [[maybe_unused]] PairRegs<D> b2;
    if (nw > 0) {
        fetch(b0, gp_of(0), false);
        if constexpr (NBUF == 3) fetch(b1, gp_of(1), false);
    }
    TQ4_STAMP(2, TQ4_NOW);
    // Fused entry: this split's ticket, and the caller's atomics (the
    // persistent kernel's queue fetch), issued only now: atomics on one
    // counter queue behind each other (about 50 ns per earlier one), and a
    // wave's loads complete in issue order, so an atomic issued before the
    // first strip loads would hold their processing until its return. Issued
    // after them, it is first waited for at the wave's third pair or at the
    // merge, where the ticket is read.
    uint32_t ticket = 0;
    if constexpr (MODE == 1) {
        if (p.K > 1 && tid == 0)
            ticket = __hip_atomic_fetch_add(p.counters + ((size_t)seq * p.Hkv + kvh) * kTicketStride,
                                            1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    after_issue();

    // ---- phase 1: rotate q (Pi = M * inv_sqrt_len), fold the softmax scale,
    // normalise each row by a power of two, stage in LDS; then every lane
    // builds its operands.
    float* q_st = region;
    stage_q_rows<D>(p, qraw, sg, rotate, q_st, q_exp, wave, lane);
    lds_barrier();
    QOps<D> qo;
    build_qops<D>(qo, q_st, q_exp, G, lane);
    TQ4_STAMP(3, TQ4_NOW);
    // The merge rows lie past q_st, so a wave without pairs may park its
    // rows while the others still read q here; q_st is next written by the
    // next item's prologue, behind the item's closing barriers.
    RowState<D> st;
    st.reset(qo.row_live);

    auto process = [&](const PairRegs<D>& r, uint32_t gp, bool masked) {
        bool ok = true;
        if (masked) ok = strip_lds[min(2 * gp + sp, nws - 1)] != kBadStrip;
        process_pair<D, MODE == 0>(st, qo, r, sc_wave, lane, masked, ltok - 32 * gp, ok);
    };

    // ---- the three-deep (two-deep at d = 256) register ring: full pairs,
    // then this wave's masked tail pair, already in flight (its second strip
    // may lie past the window: the staged window has one padding row).
    auto pick = [](const PairRegs<D>& x, const PairRegs<D>& y, bool take_y) {
        PairRegs<D> r;
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            r.k1[i] = take_y ? y.k1[i] : x.k1[i];
            r.k2[i] = take_y ? y.k2[i] : x.k2[i];
        }
#pragma unroll
        for (int i = 0; i < D / 16; ++i) r.v[i] = take_y ? y.v[i] : x.v[i];
        r.sc = take_y ? y.sc : x.sc;
        return r;
    };
    if (nw > 0) {
        if constexpr (NBUF == 3) {
            uint32_t j = 0;
            for (; j + 3 <= nfw; j += 3) {
                fetch(b2, gp_of(j + 2), false);
                process(b0, gp_of(j), false);
                fetch(b0, gp_of(j + 3), false);
                process(b1, gp_of(j + 1), false);
                fetch(b1, gp_of(j + 4), false);
                process(b2, gp_of(j + 2), false);
            }
            fetch(b2, gp_of(j + 2), false);  // pair j+2 (clamped): the tail when nfw = j + 2
            if (j < nfw) process(b0, gp_of(j), false);
            if (j + 1 < nfw) process(b1, gp_of(j + 1), false);
            if (tail_mine) {  // the tail is pair nfw, in b0, b1 or b2
                const uint32_t r = nfw - j;
                process(pick(pick(b0, b1, r == 1), b2, r == 2), gp_of(nfw), true);
            }
        } else {
            uint32_t j = 0;
            for (; j + 2 <= nfw; j += 2) {
                fetch(b1, gp_of(j + 1), false);
                process(b0, gp_of(j), false);
                fetch(b0, gp_of(j + 2), false);
                process(b1, gp_of(j + 1), false);
            }
            fetch(b1, gp_of(j + 1), false);  // pair j+1 (clamped): the tail when nfw = j + 1
            if (j < nfw) process(b0, gp_of(j), false);
            if (tail_mine) process(pick(b0, b1, nfw - j == 1), gp_of(nfw), true);
        }
    }
    // ---- a window holding an invalid page: every pair masked, one at a time.
    if (bad) {
        for (uint32_t gp = wave; gp < np_total; gp += kWaves) {
            PairRegs<D> bm;
            fetch(bm, gp, true);
            process(bm, gp, true);
        }
    }

    TQ4_STAMP(4, TQ4_NOW);
    finish_item<D, MODE, OWN>(p, seq, kvh, split, k_live, ticket, st, qo.row_live, region);
}

// Waves per SIMD the register ring allows without spilling: two at d = 64
// and d = 128 (<= 256 VGPRs), one at d = 256.
#define TQ4_DECODE_ATTRS                                                                   \
    __launch_bounds__(kThreads)                                                            \
    __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2, 2)))

// One workgroup per (seq, kv head, split), splits fastest.
template <int D, int MODE>
__global__ TQ4_DECODE_ATTRS void decode_kernel(DecodeParams p)
{
    const uint32_t item = blockIdx.x;
    decode_item<D, MODE>(p, item / (p.K * p.Hkv), (item / p.K) % p.Hkv, item % p.K);
}

// Persistent fused decode for launches with more work items than
// workgroup slots. The items are the LIVE (seq, kv head, split) triples only.
// Every split but a sequence's last covers exactly the partition width, so
// the queue lists those equal items first -- (seq, kv head, split) order --
// and the last, shorter splits after them (one per (seq, kv head), or the
// zero-context item of an empty sequence), longest first for batches of up to
// kLptMaxSeqs sequences, so their spread of sizes packs the tail. Every
// workgroup derives the order from the context lengths (a prefix over
// sequences and a rank of the last splits, staged in LDS). The items are
// dealt over kSubQueues interleaved sub-queues (items x, x + nq, ...), each
// an agent-scope counter on its own 128-byte line serving workgroups x,
// x + nq, ...: one counter for the whole launch serves its fetches one at a
// time. A workgroup takes item blockIdx.x, then one item at a time from its
// sub-queue, fetched once the current item's first strip loads are out, so
// its round trip hides under the item. Each of a sub-queue's `count`
// fetches returns a distinct value and the one that returns count - 1 is the
// last: it resets the counter (every workgroup's final fetch is its failing
// one, so the fetches number exactly `count`). Nothing waits on a
// workgroup that has not started: the combiner of a (seq, kv head) waits only
// for splits that took their ticket before it, each in the hands of a running
// workgroup that only streams and exports before it fetches again.
// The persistent kernels' plan, the same in every workgroup: per sequence
// its live splits (at least 1) and the inclusive prefix of its full items
// (p.Hkv * (splits - 1)), the context length (when ctx_l is not null), and,
// for up to kLptMaxSeqs sequences (lpt), the order of the last splits,
// longest first (ties in sequence order) -- a stable descending rank,
// counted from keys staged in LDS. scratch: 256 free LDS words. Returns the
// number of full items.
__device__ uint32_t plan_items(const DecodeParams& p, uint32_t* full, uint32_t* splits,
                               uint32_t* order, uint32_t* ctx_l, bool lpt, uint32_t* scratch)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t width = (p.max_blocks + p.K - 1) / p.K;
    const uint64_t capacity = (uint64_t)p.max_blocks * p.S;
    for (uint32_t s = tid; s < p.B; s += kThreads) {
        // 32-bit arithmetic: a context length is below 2^31
        const int32_t c = p.context_lens[s];
        uint32_t ctx = c < 0 ? 0u : (uint32_t)c;
        if (ctx > capacity) ctx = (uint32_t)capacity;
        const uint32_t pages = (ctx + p.S - 1) / p.S;
        uint32_t kl = (pages + width - 1) / width;
        kl = kl > 0 ? kl : 1u;
        splits[s] = kl;
        full[s] = p.Hkv * (kl - 1);
        if (ctx_l != nullptr) ctx_l[s] = ctx;
        if (lpt) order[s] = pages - (kl - 1) * width;  // the last split's pages (the sort key)
    }
    __syncthreads();
    // Ranks are kept in registers until all keys are read. Up to 64
    // sequences, the four waves each count over a quarter of the keys
    // (partial ranks in scratch [4][64], summed at placing).
    constexpr int kRanks = kLptMaxSeqs / kThreads;
    uint32_t rank[kRanks];
    if (lpt && p.B <= 64) {
        const uint32_t s = tid & 63, part = tid >> 6;
        uint32_t r = 0;
        if (s < p.B) {
            const uint32_t key = order[s];
            const uint32_t t1 = min(part * 16 + 16, p.B);
#pragma unroll 4
            for (uint32_t t = part * 16; t < t1; ++t) {
                const uint32_t kt = order[t];
                r += (kt > key || (kt == key && t < s)) ? 1u : 0u;
            }
        }
        scratch[part * 64 + s] = r;
    } else if (lpt) {
#pragma unroll
        for (int i = 0; i < kRanks; ++i) {
            const uint32_t s = tid + i * kThreads;
            if (s < p.B) {
                const uint32_t key = order[s];
                uint32_t r = 0;
#pragma unroll 4
                for (uint32_t t = 0; t < p.B; ++t) {
                    const uint32_t kt = order[t];
                    r += (kt > key || (kt == key && t < s)) ? 1u : 0u;
                }
                rank[i] = r;
            }
        }
    }
    if (tid < 64) {  // inclusive prefix of the full items, 64 sequences per step
        uint32_t carry = 0;
        for (uint32_t b = 0; b < p.B; b += 64) {
            const uint32_t i = b + lane;
            uint32_t v = i < p.B ? full[i] : 0u;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t u = __shfl_up(v, o, 64);
                if (lane >= o) v += u;
            }
            v += carry;
            if (i < p.B) full[i] = v;
            carry = __shfl(v, 63, 64);
        }
    }
    __syncthreads();  // every key is read: the ranks can be placed
    if (lpt && p.B <= 64) {
        if ((uint32_t)tid < p.B)
            order[scratch[tid] + scratch[64 + tid] + scratch[128 + tid] + scratch[192 + tid]] = tid;
        __syncthreads();
    } else if (lpt) {
#pragma unroll
        for (int i = 0; i < kRanks; ++i) {
            const uint32_t s = tid + i * kThreads;
            if (s < p.B) order[rank[i]] = s;
        }
        __syncthreads();
    }
    return full[p.B - 1];
}

// (seq, kv head, split) of queue item `item` under the plan: the full splits
// first, in (seq, kv head, split) order, then the last splits.
__device__ __forceinline__ void item_coords(const DecodeParams& p, uint32_t item, uint32_t n_full,
                                            const uint32_t* full, const uint32_t* splits,
                                            const uint32_t* order, bool lpt, uint32_t& seq,
                                            uint32_t& kvh, uint32_t& split)
{
    const int lane = threadIdx.x & 63;
    if (item < n_full) {
        // a full split: its sequence is the first s with full[s] > item
        uint32_t sq = 0;
        for (uint32_t b = 0; b < p.B; b += 64) {
            const uint32_t i = b + lane;
            const uint64_t m = __ballot(i < p.B && full[i] > item);
            if (m != 0) {
                sq = b + (uint32_t)__builtin_ctzll(m);
                break;
            }
        }
        seq = __builtin_amdgcn_readfirstlane(sq);
        const uint32_t r = item - (seq > 0 ? full[seq - 1] : 0u);
        const uint32_t per = splits[seq] - 1;
        kvh = r / per;
        split = r % per;
    } else {
        // a last split
        const uint32_t r = item - n_full;
        seq = lpt ? order[r / p.Hkv] : r / p.Hkv;
        kvh = r % p.Hkv;
        split = splits[seq] - 1;
    }
}

template <int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2, 2)))
void decode_persistent_kernel(DecodeParams p)
{
    extern __shared__ float smem[];
    uint32_t* full = (uint32_t*)(smem + kHdrFloats + kStripSlots + region_floats(p.G, D));
    uint32_t* splits = full + p.B;  // max(1, live splits) per sequence
    uint32_t* order = splits + p.B;
    const bool lpt = p.B <= kLptMaxSeqs;
    uint32_t* next_lds = (uint32_t*)(smem + 145);
    const int tid = threadIdx.x;
    const uint32_t n_full =
        plan_items(p, full, splits, order, nullptr, lpt,
                   (uint32_t*)(smem + kHdrFloats + kStripSlots));  // the free q staging region
    const uint32_t n_items = n_full + p.B * p.Hkv;
    // kSubQueues interleaved queues (one counter line each): sub-queue x
    // holds items x, x + nq, x + 2nq, ... and serves workgroups x, x + nq,
    // ...; one shared counter would serve every fetch of the launch in turn.
    const uint32_t nq = gridDim.x < kSubQueues ? gridDim.x : kSubQueues;
    const uint32_t x = blockIdx.x % nq;
    const uint32_t nwg = (gridDim.x - x + nq - 1) / nq;  // workgroups of sub-queue x
    const uint32_t count = n_items > x ? (n_items - x + nq - 1) / nq : 0u;  // its items
    uint32_t* subq = p.queue + kTicketStride * x;
    uint32_t item = blockIdx.x;
    while (item < n_items) {
        uint32_t fetched = 0;
        uint32_t seq, kvh, split;
        TQ4_STAMP_ITEM(item);
        TQ4_STAMP_P(10, TQ4_NOW);
        TQ4_STAMP_P(9, blockIdx.x);
        item_coords(p, item, n_full, full, splits, order, lpt, seq, kvh, split);
        TQ4_STAMP_P(12, seq);
        TQ4_STAMP_P(13, split);
        // the next item's queue fetch goes out after this item's first strip
        // loads (decode_item's hook); its value is read after the item
        decode_item<D, 1, false>(p, seq, kvh, split, [&]() {
            if (tid == 0)
                fetched = __hip_atomic_fetch_add(subq, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        });
        TQ4_STAMP_P(11, TQ4_NOW);
        if (tid == 0) {
            if (fetched == count - 1)
                __hip_atomic_store(subq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *next_lds = x + nq * (nwg + fetched);
        }
        // LDS-only barriers: the item's record stores are not waited for
        // here; the next item's phase-0 loads go out first.
        lds_barrier();
        item = __builtin_amdgcn_readfirstlane(*next_lds);
        lds_barrier();
    }
}

// Stand-alone combine: 16 consecutive (seq, q head) rows per workgroup, four
// per wave.
template <int D>
__global__ __launch_bounds__(kThreads) void combine_kernel(DecodeParams p)
{
    constexpr int CC = D / 32;
    const size_t total = (size_t)p.B * p.Hq;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float es[CC], gt[CC];
    if (p.output_stage >= 1) load_lane_floats<D>(p.pi_signs, lane, es);
    for (int i = 0; i < 4; ++i) {
        const size_t row = (size_t)blockIdx.x * 16 + wave + kWaves * i;
        if (row >= total) break;
        if (p.output_stage == 2) load_lane_floats<D>(p.gate + row * D, lane, gt);
        float v[CC];
        combine_records<D, false>(p.records + row * p.K * (D + 4), p.K, lane, v, ~0u,
                                  [](uint32_t(&)[2], uint32_t(&)[D / 32]) {});
        egress_row<D>(v, es, gt, p.out + row * D, p.inv_sqrt_len, p.output_stage, lane);
    }
}

__global__ void fill_zero_kernel(uint32_t* ptr, size_t words)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (size_t)gridDim.x * blockDim.x)
        ptr[i] = 0u;
}

// Workgroup slots of a persistent kernel on the current device (CUs x
// resident workgroups per CU at this LDS size), 0 if it cannot run.
template <class Kernel>
uint32_t persistent_slots(Kernel kernel, size_t lds)
{
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess)
        return 0;
    return cus > 0 && per_cu > 0 ? (uint32_t)cus * (uint32_t)per_cu : 0u;
}

template <int D>
hipError_t launch_decode_t(hipStream_t stream, const DecodeParams& p, int mode)
{
    const size_t blocks = (size_t)p.B * p.Hkv * p.K;
    const size_t lds = (kHdrFloats + kStripSlots + region_floats(p.G, D)) * sizeof(float);
    if (mode == 0) {
        hipLaunchKernelGGL((decode_kernel<D, 0>), dim3((uint32_t)blocks), dim3(kThreads), lds,
                           stream, p);
        return hipGetLastError();
    }
    // Fused: persistent when the split grid outnumbers the resident slots.
    if (p.queue != nullptr && p.K > 1 && p.B <= kPersistentMaxSeqs) {
        const size_t lds_p = lds + (p.B <= kLptMaxSeqs ? 3 : 2) * (size_t)p.B * sizeof(uint32_t);
        const uint32_t slots = persistent_slots(decode_persistent_kernel<D>, lds_p);
        if (slots > 0 && blocks > slots) {
            hipLaunchKernelGGL((decode_persistent_kernel<D>), dim3(slots), dim3(kThreads), lds_p,
                               stream, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((decode_kernel<D, 1>), dim3((uint32_t)blocks), dim3(kThreads), lds, stream,
                       p);
    return hipGetLastError();
}

template <int D>
hipError_t launch_combine_t(hipStream_t stream, const DecodeParams& p)
{
    const size_t rows = (size_t)p.B * p.Hq;
    const uint32_t blocks = (uint32_t)((rows + 15) / 16);
    hipLaunchKernelGGL((combine_kernel<D>), dim3(blocks), dim3(kThreads), 0, stream, p);
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
    switch (p.D) {
        case 64: return launch_combine_t<64>(stream, p);
        case 128: return launch_combine_t<128>(stream, p);
        case 256: return launch_combine_t<256>(stream, p);
        default: return hipErrorInvalidValue;
    }
}

// The no-allocation decode's workspace: a static device array, one copy per
// GPU the library runs on, held until the process ends. It is zero when the
// code object is loaded (a zero-filled segment) and every decode leaves the
// words it used zero again; after a poll give-up the caller re-zeroes it
// with tq4_paged_decode_noalloc_reset. In host code its name is only a
// stand-in; its device address comes from hipGetSymbolAddress, once per
// device, and only that address is handed to kernels and fills.
static __device__ __align__(256) uint32_t scratch[kNoAllocScratchBytes / sizeof(uint32_t)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_scratch(void** ptr)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        // no fill here: the array is zero at load, and a fill made at a first
        // call under graph capture would become a node of that graph
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

#ifdef TQ4_DECODE_STAMPS
// The measurement build's stamp readout (declared only by its users).
extern "C" int tq4_decode_stamps(void* dst, size_t bytes)
{
    const size_t all = sizeof(uint64_t) * kStampBlocks * kStampSlots;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_stamps), bytes < all ? bytes : all, 0,
                               hipMemcpyDeviceToHost) == hipSuccess
               ? 0
               : -1;
}
#endif

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
