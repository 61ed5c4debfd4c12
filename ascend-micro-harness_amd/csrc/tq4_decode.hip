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


// LDS layout (floats). A fixed header -- m[4][16], l[4][16], q exponents[16],
// the last-arrival flag, the combine's per-row M and L[16+16] -- then one big
// region reused in turn by the q staging area [G][D], the wave-merge slots
// [2][G][D], and the combine's weights [G][K] + normalised rows [G][D].
constexpr int kMaxWindowPages = 1024;  // block-table entries one split may own
constexpr int kHdrFloats = 2 * kWaves * 16 + 16 + 4 + 32 + 12 + kMaxWindowPages;

__host__ __device__ constexpr size_t region_floats(uint32_t G, uint32_t D, uint32_t K)
{
    const size_t merge = 2ull * G * D;
    const size_t comb = 2ull * G * K + (size_t)G * D;
    return merge > comb ? merge : comb;
}

// Workgroup barrier for LDS traffic only: unlike __syncthreads() it does not
// wait for outstanding global loads (vmcnt), so prefetched strips stay in
// flight across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, xor_lanes(v, m));
    return v;
}

// LSE-combine `nrows` rows of K partial records each (row r, split k at
// rec + r*row_stride + k*(D+4)) with all 256 threads, leaving the normalised
// rows acc / L (0 when L == 0) in out[r*D + c]. The (m, l) pairs load in one
// parallel pass; each thread then sums its channel pairs over the splits with
// 16 independent record loads in flight.
// Record traffic between workgroups of one launch: agent-scope atomic
// (device-coherent, sc1) stores and loads, so no whole-L2 write-back or
// invalidate is needed around the arrival counter.
__device__ __forceinline__ void store_coherent(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool COHERENT>
__device__ __forceinline__ float load_rec(const float* p)
{
    if constexpr (COHERENT)
        return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}

template <int D, bool COHERENT>
__device__ void combine_rows(const float* rec, size_t row_stride, uint32_t nrows, uint32_t K,
                             float* w, float* lk, float* ML, float* out)
{
    constexpr int RS = D + 4;
    constexpr int CH = 16;
    const int tid = threadIdx.x;
    const uint32_t nk = nrows * K;
    for (uint32_t t = tid; t < nk; t += kThreads) {
        const float* rr = rec + (t / K) * row_stride + (size_t)(t % K) * RS;
        w[t] = load_rec<COHERENT>(rr);
        lk[t] = load_rec<COHERENT>(rr + 1);
    }
    __syncthreads();
    if ((uint32_t)tid < nrows) {
        float M = kMasked;
        for (uint32_t k = 0; k < K; ++k) M = fmaxf(M, w[tid * K + k]);
        ML[tid] = M;
    }
    __syncthreads();
    for (uint32_t t = tid; t < nk; t += kThreads) {
        const float e = expf(w[t] - ML[t / K]);
        w[t] = e;
        lk[t] *= e;
    }
    __syncthreads();
    if ((uint32_t)tid < nrows) {
        float L = 0.0f;
        for (uint32_t k = 0; k < K; ++k) L += lk[tid * K + k];
        ML[16 + tid] = L;
    }
    const uint32_t npairs = nrows * (D / 2);
    for (uint32_t pi = tid; pi < npairs; pi += kThreads) {
        const uint32_t r = pi / (D / 2), c = 2 * (pi % (D / 2));
        const float* rr = rec + r * row_stride + 4 + c;
        const float* wr = w + r * K;
        float a0 = 0.0f, a1 = 0.0f;
        for (uint32_t k0 = 0; k0 < K; k0 += CH) {
            float2 v[CH];
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                if (k0 + i < K) {
                    const float* at = rr + (size_t)(k0 + i) * RS;
                    if constexpr (COHERENT)
                        v[i] = make_float2(load_rec<true>(at), load_rec<true>(at + 1));
                    else
                        v[i] = *(const float2*)at;
                } else {
                    v[i] = make_float2(0.0f, 0.0f);
                }
            }
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const float wk = k0 + i < K ? wr[k0 + i] : 0.0f;
                a0 += v[i].x * wk;
                a1 += v[i].y * wk;
            }
        }
        out[r * D + c] = a0;
        out[r * D + c + 1] = a1;
    }
    __syncthreads();
    for (uint32_t e = tid; e < nrows * D; e += kThreads) {
        const float L = ML[16 + e / D];
        out[e] = L == 0.0f ? 0.0f : out[e] / L;
    }
    __syncthreads();
}

// Egress of one normalised row (in LDS) by one wave: optionally Pi^T and
// 1/sqrt(d), optionally the gate, BF16 RNE store.
template <int D>
__device__ void egress_row(const float* row, const float* pi_signs, const float* gate,
                           uint16_t* out, float inv_sqrt_len, uint32_t stage, int lane)
{
    constexpr int CPL = D / 64;
    float v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) v[j] = row[lane * CPL + j];
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
    float* m_x = smem;
    float* l_x = m_x + kWaves * 16;
    int* q_exp = (int*)(l_x + kWaves * 16);
    int* flag = q_exp + 16;
    float* ML = (float*)(flag + 4);
    int32_t* page_lds = (int32_t*)(smem + 192);
    float* region = smem + kHdrFloats;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, kg = lane >> 4;
    const uint32_t item = blockIdx.x;
    const uint32_t split = item % p.K;
    const uint32_t kvh = (item / p.K) % p.Hkv;
    const uint32_t seq = item / (p.K * p.Hkv);

    // ---- phase 0: every small load -- context length, q rows, rotation
    // signs, the split's block-table window -- is issued before any strip
    // load: vmcnt retires in order, so a later wait for one of these would
    // otherwise also wait for the strip stream.
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
    // The split's window of the block table: the reference AIC decode's
    // Partition(page_count, splits, split) over the table's max_blocks_per_seq
    // pages (turboquant_paged_decode_attention.cpp:1598-1624), staged in LDS
    // so the strip loop reads page ids without touching vmcnt.
    uint32_t pb, pc;
    partition(p.max_blocks, p.K, split, pb, pc);
    const uint32_t spp = S / kStrip;
    const uint32_t n_window = pc * spp;
    const uint32_t n_win_mine =
        n_window > (uint32_t)wave ? (n_window - wave + kWaves - 1) / kWaves : 0u;
    const int32_t* tbl = p.block_tables + (size_t)seq * p.max_blocks;
    for (uint32_t t = tid; t < pc; t += kThreads) page_lds[t] = tbl[pb + t];
    // Unconditional vmcnt(0) (expcnt and lgkmcnt left at their maxima): the
    // loads above are all complete from here on every path, so the compiler's
    // wait analysis never again waits on them -- or on what is queued after.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    lds_barrier();
    const size_t plane_floats = (size_t)p.P * p.Hkv * S;

    // Operands of this wave's j-th strip; false when its page is out of range
    // (table entries past the live context may hold anything).
    auto fetch = [&](uint32_t j, StripRegs<D>& r) -> bool {
        const uint32_t idx = wave + kWaves * j;
        const uint32_t phys = (uint32_t)__builtin_amdgcn_readfirstlane(page_lds[idx / spp]);
        if (phys >= p.P) return false;
        const size_t row = ((size_t)phys * p.Hkv + kvh) * S + (size_t)(idx % spp) * kStrip;
        load_strip<D>(r, p.key_cache + row * (D / 2), p.value_cache + row * (D / 2),
                      p.scale_cache + row, p.scale_cache + row + plane_floats, n, kg);
        return true;
    };
    StripRegs<D> buf0, buf1, buf2;
    bool ok0 = n_win_mine > 0 ? fetch(0, buf0) : false;
    bool ok1 = n_win_mine > 1 ? fetch(1, buf1) : false;
    bool ok2 = false;

    // Live strips of the window: tokens at or past ctx are masked, strips with
    // none live are not walked (turboquant_decode_tail.hpp:246-272).
    uint32_t ctx = ctx_raw < 0 ? 0u : (uint32_t)ctx_raw;
    const uint64_t capacity = (uint64_t)p.max_blocks * S;
    if (ctx > capacity) ctx = (uint32_t)capacity;
    const uint64_t tok0 = (uint64_t)pb * S;
    uint32_t live = 0;
    if (pc > 0 && ctx > tok0) {
        const uint64_t need = (ctx - tok0 + kStrip - 1) / kStrip;
        live = need < (uint64_t)n_window ? (uint32_t)need : n_window;
    }
    const uint32_t n_mine = live > (uint32_t)wave ? (live - wave + kWaves - 1) / kWaves : 0u;

    // ---- phase 2 (overlaps the strip loads): rotate q (Pi = M * inv_sqrt_len),
    // fold the softmax scale, normalise each row by a power of two, stage in LDS.
    float* q_st = region;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t g = wave + kWaves * i;
        if (g >= G) continue;
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
        for (int j = 0; j < CPL; ++j) q_st[g * D + lane * CPL + j] = ldexpf(v[j], -kq);
        if (lane == 0) q_exp[g] = kq;
    }
    lds_barrier();

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
    // No barrier here: q_st is next overwritten after the merge barrier,
    // which every wave reaches only after building its operands.

    // ---- stream this wave's strips (register double buffer).
    f4_t acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m2 = kMasked, lpart = 0.0f;
    int E = 0;  // running max exponent field of the live value scales

    auto process = [&](const StripRegs<D>& cur, uint32_t j) {
            const uint32_t idx = wave + kWaves * j;
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
            };
    // 3-deep ring: strip j computes while strips j+1 and j+2 are in flight.
    for (uint32_t j = 0; j < n_mine; j += 3) {
        ok2 = j + 2 < n_mine ? fetch(j + 2, buf2) : false;
        if (ok0) process(buf0, j);
        if (j + 1 >= n_mine) break;
        ok0 = j + 3 < n_mine ? fetch(j + 3, buf0) : false;
        if (ok1) process(buf1, j + 1);
        if (j + 2 >= n_mine) break;
        ok1 = j + 4 < n_mine ? fetch(j + 4, buf1) : false;
        if (ok2) process(buf2, j + 2);
    }

    // ---- merge the four waves: common reference M per row, then sum.
    lpart += xor_lanes(lpart, 16);
    lpart += xor_lanes(lpart, 32);
    if (kg == 0) {
        m_x[wave * 16 + n] = m2;
        l_x[wave * 16 + n] = lpart;
    }
    lds_barrier();
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
    float* slot0 = region;
    float* slot1 = region + (size_t)G * D;
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
    lds_barrier();
    if (wave < 2) add(wave == 0 ? slot0 : slot1);
    lds_barrier();
    if (wave == 1) put(slot0);
    lds_barrier();
    if (wave == 0) add(slot0);

    const bool local = (MODE == 1) && p.K == 1;
    if (!local) {
        // ---- export one record per q head: [m (natural log), l, 0, 0, acc].
        float* rec_base = p.records + (((size_t)seq * p.Hq + (size_t)kvh * G) * p.K + split) * RS;
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t r = 4 * kg + i;
                if (r < G) {
                    float* rec = rec_base + (size_t)r * p.K * RS;
                    auto put_rec = [&](int at, float v) {
                        if constexpr (MODE == 1) store_coherent(rec + at, v);
                        else rec[at] = v;
                    };
#pragma unroll
                    for (int b = 0; b < NB; ++b) put_rec(4 + 16 * b + n, acc[b][i]);
                    if (n == 0) {
                        put_rec(0, Mrow[i] == kMasked ? kMasked : Mrow[i] * kLn2);
                        put_rec(1, Lrow[i]);
                        put_rec(2, 0.0f);
                        put_rec(3, 0.0f);
                    }
                }
            }
        }
    }
    if constexpr (MODE == 0) return;

    float* rows = region;  // normalised rows [G][D] for the egress
    if (local) {
        lds_barrier();  // wave 0 finished reading slot0
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t r = 4 * kg + i;
                if (r < G) {
                    const float L = Lrow[i];
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        rows[r * D + 16 * b + n] = L == 0.0f ? 0.0f : acc[b][i] / L;
                }
            }
        }
        lds_barrier();
    } else {
        // ---- the last workgroup of this (seq, kv head) to arrive combines.
        // The records went out as device-coherent stores; waiting for their
        // completion before the increment publishes them (release), and the
        // last arriver reads them with device-coherent loads (acquire).
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            uint32_t* ctr = p.counters + (size_t)seq * p.Hkv + kvh;
            const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == p.K - 1;
            if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last;
        }
        __syncthreads();
        if (!*flag) return;
        float* w = region;
        float* lk = region + (size_t)G * p.K;
        rows = lk + (size_t)G * p.K;
        combine_rows<D, true>(p.records + ((size_t)seq * p.Hq + (size_t)kvh * G) * p.K * RS,
                        (size_t)p.K * RS, G, p.K, w, lk, ML, rows);
    }
    for (uint32_t g = wave; g < G; g += kWaves) {
        const size_t qh = (size_t)seq * p.Hq + kvh * G + g;
        egress_row<D>(rows + g * D, p.pi_signs, p.gate ? p.gate + qh * D : nullptr,
                      p.out + qh * D, p.inv_sqrt_len, p.output_stage, lane);
    }
}

// Stand-alone combine: 16 consecutive (seq, q head) rows per workgroup.
template <int D>
__global__ __launch_bounds__(kThreads) void combine_kernel(DecodeParams p)
{
    extern __shared__ float smem[];
    const size_t total = (size_t)p.B * p.Hq;
    const size_t row0 = (size_t)blockIdx.x * 16;
    const uint32_t nrows = (uint32_t)((total - row0) < 16 ? (total - row0) : 16);
    float* ML = smem;
    float* w = smem + 32;
    float* lk = w + (size_t)16 * p.K;
    float* rows = lk + (size_t)16 * p.K;
    combine_rows<D, false>(p.records + row0 * p.K * (D + 4), (size_t)p.K * (D + 4), nrows, p.K, w, lk,
                    ML, rows);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t r = wave; r < nrows; r += kWaves) {
        const size_t row = row0 + r;
        egress_row<D>(rows + r * D, p.pi_signs, p.gate ? p.gate + row * D : nullptr,
                      p.out + row * D, p.inv_sqrt_len, p.output_stage, lane);
    }
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
    const uint32_t comb_k = (mode == 1 && p.K > 1) ? p.K : 0u;
    const size_t lds = (kHdrFloats + region_floats(p.G, D, comb_k)) * sizeof(float);
    if (mode == 0)
        hipLaunchKernelGGL((decode_kernel<D, 0>), dim3((uint32_t)blocks), dim3(kThreads), lds,
                           stream, p);
    else
        hipLaunchKernelGGL((decode_kernel<D, 1>), dim3((uint32_t)blocks), dim3(kThreads), lds,
                           stream, p);
    return hipGetLastError();
}

template <int D>
hipError_t launch_combine_t(hipStream_t stream, const DecodeParams& p)
{
    const size_t rows = (size_t)p.B * p.Hq;
    const uint32_t blocks = (uint32_t)((rows + 15) / 16);
    const size_t lds = (32 + (size_t)32 * p.K + (size_t)16 * D) * sizeof(float);
    hipLaunchKernelGGL((combine_kernel<D>), dim3(blocks), dim3(kThreads), lds, stream, p);
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
