/*
 * tq4_oracle.c -- CPU restatement of the TurboQuant TQ4 hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see tq4_oracle.h). Built with -ffp-contract=off
 * and no fast-math so FP32 operations happen exactly in the order written.
 *
 * Reference files restated here (paths relative to the reference checkout):
 *   tests/common/turboquant_oracle.hpp          prefill writer, quantiser, slot contract
 *   tests/common/turboquant_scatter_oracle.hpp  general-S index maps, scatter writer
 *   tests/common/rotate_butterfly_oracle.hpp    butterfly stage order, sign placement
 *   tests/common/paged_decode_oracle.hpp        score / recurrence order, egress
 *   tests/common/single_token_decode_oracle.hpp GQA mapping, GoldenDecode
 *   tests/common/aic_splitk_decode_fixture.hpp  partial record, neutral element
 *   tests/common/splitk_decode_fixture.hpp      FP64 full-context reference
 *   tests/common/l2_atomic_oracle.hpp           LSE combine step, egress
 *   include/turboquant_splitk_contract.hpp      Partition
 *   kernels/ops/turboquant/turboquant_decode_tail.hpp  live-token arithmetic
 */
#include "tq4_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bf16 */
static float bits_to_f32(uint32_t bits)
{
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint32_t f32_to_bits(float f)
{
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

/* turboquant_scatter_oracle.hpp:56-71 */
float tq4o_bf16_to_f32(uint16_t raw) { return bits_to_f32((uint32_t)raw << 16); }

uint16_t tq4o_f32_to_bf16(float value)
{
    const uint32_t bits = f32_to_bits(value);
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu))
        return (uint16_t)((bits >> 16) | 0x40u);
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

/* ------------------------------------------------------------ index maps */
/* turboquant_scatter_oracle.hpp:110-132 (general S, strip height 16) */
uint64_t tq4o_key_nibble(uint32_t H, uint32_t S, uint32_t d, uint32_t page, uint32_t head,
                         uint32_t token, uint32_t channel)
{
    return (((uint64_t)page * H + head) * S + token) * d + channel;
}

uint64_t tq4o_value_nibble(uint32_t H, uint32_t S, uint32_t d, uint32_t page, uint32_t head,
                           uint32_t token, uint32_t channel)
{
    const uint64_t base = ((uint64_t)page * H + head) * S * d;
    return base + (uint64_t)(token / TQ4O_STRIP) * TQ4O_STRIP * d +
           (uint64_t)channel * TQ4O_STRIP + token % TQ4O_STRIP;
}

uint64_t tq4o_scale_index(uint32_t P, uint32_t H, uint32_t S, uint32_t plane, uint32_t page,
                          uint32_t head, uint32_t token)
{
    return (((uint64_t)plane * P + page) * H + head) * S + token;
}

/* turboquant_scatter_oracle.hpp:220-235 */
int tq4o_read_nibble(const int8_t* cache, uint64_t nibble)
{
    const uint8_t byte = (uint8_t)cache[nibble / 2];
    const int raw = (nibble % 2 == 0) ? (byte & 0xF) : ((byte >> 4) & 0xF);
    return raw >= 8 ? raw - 16 : raw;
}

void tq4o_write_nibble(int8_t* cache, uint64_t nibble, int value)
{
    const uint8_t nib = (uint8_t)(value & 0xF);
    uint8_t* byte = (uint8_t*)&cache[nibble / 2];
    if (nibble % 2 == 0)
        *byte = (uint8_t)((*byte & 0xF0u) | nib);
    else
        *byte = (uint8_t)((*byte & 0x0Fu) | (uint8_t)(nib << 4));
}

/* -------------------------------------------------------------- rotation */
/* turboquant_oracle.hpp:77-80, rotate_butterfly_oracle.hpp:69-72 */
int tq4o_pi_sign(int channel)
{
    return ((channel * channel + 3 * channel + 1) % 7 < 3) ? -1 : 1;
}

void tq4o_canonical_signs(uint32_t d, float* signs)
{
    for (uint32_t c = 0; c < d; ++c) signs[c] = (float)tq4o_pi_sign((int)c);
}

static int parity(unsigned v)
{
    int p = 0;
    while (v) {
        p ^= (int)(v & 1u);
        v >>= 1;
    }
    return p;
}

static int hadamard(int i, int j) { return parity((unsigned)(i & j)) ? -1 : 1; }

/* turboquant_oracle.hpp:157-171: T[s][g][c0][i] = (s?-1:+1) * sign[g*32+c0] * H32[c0][i] */
void tq4o_build_tables_i8(uint32_t d, const float* signs, int8_t* tables)
{
    const uint32_t groups = d / 32;
    for (uint32_t s = 0; s < 2; ++s)
        for (uint32_t g = 0; g < groups; ++g)
            for (uint32_t c0 = 0; c0 < 32; ++c0)
                for (uint32_t i = 0; i < 32; ++i)
                    tables[((s * groups + g) * 32 + c0) * 32 + i] =
                        (int8_t)((s ? -1 : 1) * (signs[g * 32 + c0] < 0 ? -1 : 1) *
                                 hadamard((int)c0, (int)i));
}

/* Signs are recoverable from the tables: T[0][g][c0][0] = sign[g*32+c0]
 * (H32[c0][0] = +1). Returns 0 if every block also matches the Hadamard
 * structure of turboquant_oracle.hpp:177-195, -1 otherwise. */
int tq4o_signs_from_tables_i8(uint32_t d, const int8_t* tables, float* signs)
{
    const uint32_t groups = d / 32;
    for (uint32_t g = 0; g < groups; ++g)
        for (uint32_t c0 = 0; c0 < 32; ++c0) signs[g * 32 + c0] = (float)tables[(g * 32 + c0) * 32];
    for (uint32_t s = 0; s < 2; ++s)
        for (uint32_t g = 0; g < groups; ++g)
            for (uint32_t c0 = 0; c0 < 32; ++c0)
                for (uint32_t i = 0; i < 32; ++i) {
                    const int want = (s ? -1 : 1) * (signs[g * 32 + c0] < 0 ? -1 : 1) *
                                     hadamard((int)c0, (int)i);
                    if (tables[((s * groups + g) * 32 + c0) * 32 + i] != want) return -1;
                }
    return 0;
}

/* rotate_butterfly_oracle.hpp:120-128: out[i] = in[i^s] + ((i&s) ? -in[i] : in[i]) */
static void butterfly_stage(float* v, float* tmp, uint32_t d, uint32_t stride)
{
    for (uint32_t i = 0; i < d; ++i) {
        const float self = v[i];
        const float partner = v[i ^ stride];
        tmp[i] = (i & stride) ? partner - self : partner + self;
    }
    memcpy(v, tmp, d * sizeof(float));
}

/* Ingress: strides 1,2,4,8,16 | signs | 32,...,d/2
 * (rotate_butterfly_oracle.hpp:44-48,130-142 at d=256; the inner H32 is fixed
 * at 32 and the outer factor is H_{d/32}, turboquant_oracle.hpp:382-410). */
void tq4o_rotate_ingress(const float* x, const float* signs, uint32_t d, float* y)
{
    float tmp[512];
    memcpy(y, x, d * sizeof(float));
    for (uint32_t s = 1; s < 32 && s < d; s <<= 1) butterfly_stage(y, tmp, d, s);
    for (uint32_t i = 0; i < d; ++i) y[i] *= signs[i];
    for (uint32_t s = 32; s < d; s <<= 1) butterfly_stage(y, tmp, d, s);
}

/* Egress (transpose): strides 32,...,d/2 | signs | 1,2,4,8,16
 * (paged_decode_oracle.hpp:634-665, rotate_butterfly_oracle.hpp:44-48). */
void tq4o_rotate_egress(const float* x, const float* signs, uint32_t d, float* y)
{
    float tmp[512];
    memcpy(y, x, d * sizeof(float));
    for (uint32_t s = 32; s < d; s <<= 1) butterfly_stage(y, tmp, d, s);
    for (uint32_t i = 0; i < d; ++i) y[i] *= signs[i];
    for (uint32_t s = 1; s < 32 && s < d; s <<= 1) butterfly_stage(y, tmp, d, s);
}

/* The definition: M[c1*32+c0][g*32+i] = H[c1][g] * sign[g*32+c0] * H32[c0][i]
 * (rotate_butterfly_oracle.hpp:84-92), applied as a dense product in double.
 * transpose=0: y = M x; transpose=1: y = M^T x. */
void tq4o_rotate_dense(const float* x, const float* signs, uint32_t d, int transpose, double* y)
{
    for (uint32_t r = 0; r < d; ++r) {
        double acc = 0.0;
        for (uint32_t c = 0; c < d; ++c) {
            const uint32_t row = transpose ? c : r;
            const uint32_t col = transpose ? r : c;
            const int c1 = (int)(row / 32), c0 = (int)(row % 32);
            const int g = (int)(col / 32), i = (int)(col % 32);
            const double m = (double)hadamard(c1, g) * (double)signs[g * 32 + c0] *
                             (double)hadamard(c0, i);
            acc += m * (double)x[c];
        }
        y[r] = acc;
    }
}

/* ------------------------------------------------------------- quantiser */
/* Exponent e with 2^e <= a < 2^(e+1), for finite a > 0 (ilogb). */
static int exponent_of(float a)
{
    const uint32_t bits = f32_to_bits(a);
    const uint32_t field = (bits >> 23) & 0xFFu;
    if (field != 0) return (int)field - 127;
    /* subnormal: a = m * 2^-149 */
    const uint32_t m = bits & 0x7FFFFFu;
    int top = 31;
    while (top > 0 && !((m >> top) & 1u)) --top;
    return top - 149;
}

/* Prefill: turboquant_oracle.hpp:412-448 (absmax floored at 1.0, scale =
 * 2^(e-2) * invSqrtLen, q = min(rint_even(y * 2^(2-e)), 7)); the FP32 bit form
 * is turboquant_reshape_and_cache_bf16.cpp:1470-1491.
 * Exact: turboquant_scatter_oracle.hpp:185-217 (no floor, absmax == 0 gives
 * scale 1.0 and q = 0). y * 2^(2-e) is exact, so the one rounding is RNE. */
void tq4o_quantise_row(const float* y, uint32_t d, float inv_sqrt_len, int policy, int8_t* q,
                       float* scale)
{
    float absmax = 0.0f;
    for (uint32_t c = 0; c < d; ++c) {
        const float a = fabsf(y[c]);
        if (a > absmax) absmax = a;
    }
    if (policy == TQ4O_POLICY_PREFILL) {
        if (absmax < 1.0f) absmax = 1.0f;
    } else if (absmax == 0.0f) {
        for (uint32_t c = 0; c < d; ++c) q[c] = 0;
        *scale = 1.0f;
        return;
    }
    const int e = exponent_of(absmax);
    *scale = ldexpf(1.0f, e - 2) * inv_sqrt_len;
    for (uint32_t c = 0; c < d; ++c) {
        float v = rintf(ldexpf(y[c], 2 - e));  /* default rounding mode: ties to even */
        if (v > 7.0f) v = 7.0f;
        q[c] = (int8_t)(int)v;
    }
}

/* --------------------------------------------------------------- writers */
static float load_input(int in_dtype, const void* base, uint64_t index)
{
    if (in_dtype == TQ4O_IN_INT8) return (float)((const int8_t*)base)[index];
    return tq4o_bf16_to_f32(((const uint16_t*)base)[index]);
}

/* One (token row, head, plane) row: rotate, quantise, pack at (page, token). */
static void write_row(int in_dtype, const void* src, uint64_t row_offset, int8_t* cache,
                      float* scale_cache, uint32_t plane, uint32_t page, uint32_t head,
                      uint32_t token_in_page, const float* signs, uint32_t H, uint32_t d,
                      uint32_t S, uint32_t P, float inv_sqrt_len, int policy)
{
    float x[512], y[512];
    int8_t q[512];
    float scale;
    for (uint32_t c = 0; c < d; ++c) x[c] = load_input(in_dtype, src, row_offset + c);
    tq4o_rotate_ingress(x, signs, d, y);
    tq4o_quantise_row(y, d, inv_sqrt_len, policy, q, &scale);
    for (uint32_t c = 0; c < d; ++c) {
        const uint64_t n = plane == 0 ? tq4o_key_nibble(H, S, d, page, head, token_in_page, c)
                                      : tq4o_value_nibble(H, S, d, page, head, token_in_page, c);
        tq4o_write_nibble(cache, n, q[c]);
    }
    scale_cache[tq4o_scale_index(P, H, S, plane, page, head, token_in_page)] = scale;
}

/* Strip slot contract (turboquant_oracle.hpp:274-287, restated per 16-token
 * strip): slot[16s+i] == slot[16s] + i, slot[16s] % 16 == 0, page < P.
 * Returns the first slot of the strip, or -1 when the strip violates it. */
static int64_t strip_first_slot(const int32_t* slots, uint32_t strip, uint32_t S, uint32_t P)
{
    const int32_t first = slots[(uint64_t)strip * TQ4O_STRIP];
    if (first < 0 || first % (int32_t)TQ4O_STRIP != 0) return -1;
    for (uint32_t i = 1; i < TQ4O_STRIP; ++i)
        if (slots[(uint64_t)strip * TQ4O_STRIP + i] != first + (int32_t)i) return -1;
    if ((uint32_t)first / S >= P) return -1;
    return first;
}

typedef struct {
    int in_dtype;
    const void* key;
    const void* value;
    int8_t* key_cache;
    int8_t* value_cache;
    float* scale_cache;
    const int32_t* slots;
    const float* signs;
    uint32_t num_tokens, H, d, S, P;
    float inv_sqrt_len;
    int policy;
    uint32_t strip_begin, strip_end;
    int64_t skipped;
} WriterJob;

static void writer_run(WriterJob* j)
{
    j->skipped = 0;
    for (uint32_t strip = j->strip_begin; strip < j->strip_end; ++strip) {
        const int64_t first = strip_first_slot(j->slots, strip, j->S, j->P);
        if (first < 0) {
            ++j->skipped;
            continue;
        }
        const uint32_t page = (uint32_t)first / j->S;
        const uint32_t tip0 = (uint32_t)first % j->S;
        for (uint32_t t = 0; t < TQ4O_STRIP; ++t) {
            const uint64_t token = (uint64_t)strip * TQ4O_STRIP + t;
            for (uint32_t h = 0; h < j->H; ++h) {
                const uint64_t row = (token * j->H + h) * j->d;
                write_row(j->in_dtype, j->key, row, j->key_cache, j->scale_cache, 0, page, h,
                          tip0 + t, j->signs, j->H, j->d, j->S, j->P, j->inv_sqrt_len,
                          j->policy);
                write_row(j->in_dtype, j->value, row, j->value_cache, j->scale_cache, 1, page, h,
                          tip0 + t, j->signs, j->H, j->d, j->S, j->P, j->inv_sqrt_len,
                          j->policy);
            }
        }
    }
}

static void* writer_thread(void* arg)
{
    writer_run((WriterJob*)arg);
    return NULL;
}

static int writer_geometry_ok(uint32_t num_tokens, uint32_t H, uint32_t d, uint32_t S,
                              uint32_t P)
{
    return num_tokens % TQ4O_STRIP == 0 && H > 0 && d >= 32 && d <= 512 && d % 32 == 0 &&
           (d & (d - 1)) == 0 && S > 0 && S % TQ4O_STRIP == 0 && P > 0;
}

/* The aligned prefill writer: compute_oracle_reference
 * (turboquant_oracle.hpp:476-513) per 16-token strip. A strip whose slots
 * violate the contract writes nothing and is counted (bad_slot_strip).
 * Returns the number of skipped strips, or -1 on bad geometry. */
int64_t tq4o_reshape_and_cache_mt(int in_dtype, const void* key, const void* value,
                                  int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                                  const int32_t* slot_mapping, const float* pi_signs,
                                  uint32_t num_tokens, uint32_t num_kv_heads, uint32_t head_size,
                                  uint32_t block_size, uint32_t num_blocks, float inv_sqrt_len,
                                  int policy, uint32_t threads)
{
    if (!writer_geometry_ok(num_tokens, num_kv_heads, head_size, block_size, num_blocks))
        return -1;
    const uint32_t strips = num_tokens / TQ4O_STRIP;
    if (threads < 1) threads = 1;
    if (threads > strips && strips > 0) threads = strips;
    if (threads > 256) threads = 256;
    WriterJob jobs[256];
    pthread_t tids[256];
    for (uint32_t t = 0; t < threads; ++t) {
        WriterJob* j = &jobs[t];
        j->in_dtype = in_dtype;
        j->key = key;
        j->value = value;
        j->key_cache = key_cache;
        j->value_cache = value_cache;
        j->scale_cache = scale_cache;
        j->slots = slot_mapping;
        j->signs = pi_signs;
        j->num_tokens = num_tokens;
        j->H = num_kv_heads;
        j->d = head_size;
        j->S = block_size;
        j->P = num_blocks;
        j->inv_sqrt_len = inv_sqrt_len;
        j->policy = policy;
        j->strip_begin = (uint32_t)((uint64_t)strips * t / threads);
        j->strip_end = (uint32_t)((uint64_t)strips * (t + 1) / threads);
    }
    if (threads == 1) {
        writer_run(&jobs[0]);
    } else {
        for (uint32_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, writer_thread, &jobs[t]);
        for (uint32_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    int64_t skipped = 0;
    for (uint32_t t = 0; t < threads; ++t) skipped += jobs[t].skipped;
    return skipped;
}

int64_t tq4o_reshape_and_cache(int in_dtype, const void* key, const void* value,
                               int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                               const int32_t* slot_mapping, const float* pi_signs,
                               uint32_t num_tokens, uint32_t num_kv_heads, uint32_t head_size,
                               uint32_t block_size, uint32_t num_blocks, float inv_sqrt_len,
                               int policy)
{
    return tq4o_reshape_and_cache_mt(in_dtype, key, value, key_cache, value_cache, scale_cache,
                                     slot_mapping, pi_signs, num_tokens, num_kv_heads, head_size,
                                     block_size, num_blocks, inv_sqrt_len, policy, 1);
}

/* The arbitrary-slot writer: turboquant_reshape_scatter_aiv.cpp:684-722 item
 * loop over (request, kv_head), tokens from cu_seqlens (NULL = one token per
 * request), slot < 0 skipped; per-row reference turboquant_scatter_oracle.hpp
 * :291-342 (exact-absmax quantiser, write_nibble preserving the partner
 * nibble, so every unowned lane of the value strip is preserved).
 * Returns the number of rows written, or -1 on bad geometry. */
int64_t tq4o_reshape_scatter(const uint16_t* key, const uint16_t* value, int8_t* key_cache,
                             int8_t* value_cache, float* scale_cache,
                             const int32_t* slot_mapping, const float* pi_signs,
                             const int32_t* cu_seqlens, uint32_t num_requests,
                             uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                             uint32_t num_blocks, uint32_t item_begin, uint32_t item_count,
                             float inv_sqrt_len)
{
    if (num_kv_heads == 0 || head_size < 32 || head_size > 512 || head_size % 32 ||
        (head_size & (head_size - 1)) || block_size == 0 || block_size % TQ4O_STRIP ||
        num_blocks == 0)
        return -1;
    int64_t written = 0;
    const uint32_t H = num_kv_heads, d = head_size, S = block_size, P = num_blocks;
    for (uint64_t item = item_begin; item < (uint64_t)item_begin + item_count; ++item) {
        const uint32_t request = (uint32_t)(item / H);
        const uint32_t head = (uint32_t)(item % H);
        if (request >= num_requests) continue;
        const uint32_t t0 = cu_seqlens ? (uint32_t)cu_seqlens[request] : request;
        const uint32_t t1 = cu_seqlens ? (uint32_t)cu_seqlens[request + 1] : request + 1;
        for (uint32_t token = t0; token < t1; ++token) {
            const int32_t slot = slot_mapping[token];
            if (slot < 0) continue;
            const uint32_t page = (uint32_t)slot / S;
            if (page >= P) continue;
            const uint32_t tip = (uint32_t)slot % S;
            const uint64_t row = ((uint64_t)token * H + head) * d;
            write_row(TQ4O_IN_BF16, key, row, key_cache, scale_cache, 0, page, head, tip,
                      pi_signs, H, d, S, P, inv_sqrt_len, TQ4O_POLICY_EXACT);
            write_row(TQ4O_IN_BF16, value, row, value_cache, scale_cache, 1, page, head, tip,
                      pi_signs, H, d, S, P, inv_sqrt_len, TQ4O_POLICY_EXACT);
            written += 2;
        }
    }
    return written;
}

/* ---------------------------------------------------------------- decode */
/* include/turboquant_splitk_contract.hpp:123-130 */
void tq4o_partition(uint32_t pages, uint32_t splits, uint32_t split, uint32_t* begin,
                    uint32_t* count)
{
    const uint32_t width = (pages + splits - 1u) / splits;
    const uint32_t b = split * width;
    const uint32_t remaining = b < pages ? pages - b : 0u;
    *begin = b;
    *count = remaining < width ? remaining : width;
}

/* turboquant_decode_tail.hpp:109-118 */
uint32_t tq4o_active_in_strip(uint64_t token_base, uint32_t seq_len)
{
    const uint64_t live = seq_len;
    if (token_base >= live) return 0u;
    return live - token_base >= TQ4O_STRIP ? TQ4O_STRIP : (uint32_t)(live - token_base);
}

uint32_t tq4o_record_floats(uint32_t head_size) { return head_size + 4u; }

/* q_eff = (M q) * inv_sqrt_len * scale: Pi = M / sqrt(d) applied to the
 * query, with the softmax scale folded in (paged_decode_oracle.hpp:127-143,
 * single_token_decode_oracle.hpp:121-134; the reference rounds q_rot to
 * BF16, this restatement keeps FP32). */
void tq4o_rotate_query(const uint16_t* q, const float* signs, uint32_t d, float inv_sqrt_len,
                       float scale, float* q_eff)
{
    float x[512], y[512];
    for (uint32_t c = 0; c < d; ++c) x[c] = tq4o_bf16_to_f32(q[c]);
    tq4o_rotate_ingress(x, signs, d, y);
    for (uint32_t c = 0; c < d; ++c) q_eff[c] = (y[c] * inv_sqrt_len) * scale;
}

/* l2_atomic_oracle.hpp:156-166, in the same FP32 instruction order */
void tq4o_combine_step(float* m, float* l, float* acc, float m_t, float l_t, const float* acc_t,
                       uint32_t d)
{
    const float m_new = *m > m_t ? *m : m_t;
    const float a_curr = expf(*m - m_new);
    const float a_tile = expf(m_t - m_new);
    *l = *l * a_curr + l_t * a_tile;
    for (uint32_t c = 0; c < d; ++c) acc[c] = acc[c] * a_curr + acc_t[c] * a_tile;
    *m = m_new;
}

#define TQ4O_FLAG_QUERY_ROTATED 1u
#define TQ4O_FLAG_QROT_BF16 2u

/* q_eff = bf16(Pi q) * scale: the rotated query rounded to BF16 before the
 * score, as the reference device's Fixpipe leaves it
 * (paged_decode_oracle.hpp:506-514, GoldenQRotBf16). */
static void rotate_query_bf16(const uint16_t* q, const float* signs, uint32_t d,
                              float inv_sqrt_len, float scale, float* q_eff)
{
    float x[512], y[512];
    for (uint32_t c = 0; c < d; ++c) x[c] = tq4o_bf16_to_f32(q[c]);
    tq4o_rotate_ingress(x, signs, d, y);
    for (uint32_t c = 0; c < d; ++c)
        q_eff[c] = tq4o_bf16_to_f32(tq4o_f32_to_bf16(y[c] * inv_sqrt_len)) * scale;
}

typedef struct {
    const uint16_t* q;
    const int8_t* key_cache;
    const int8_t* value_cache;
    const float* scale_cache;
    const int32_t* block_tables;
    const int32_t* context_lens;
    const float* signs;
    float* workspace;
    uint32_t B, Hq, Hkv, d, S, P, max_blocks, splits;
    float scale, inv_sqrt_len;
    uint32_t flags;
    uint32_t item_begin, item_end; /* items over (seq, kv head, split) */
} DecodeJob;

/* One (seq, kv head, split) task: every q head of the group walks the
 * split's live strips in order with the online-softmax recurrence of
 * single_token_decode_oracle.hpp:257-310 (scores, tile max, alpha, p, value
 * scale folded into p, l and acc updates), tail masking by overwrite
 * (turboquant_decode_tail.hpp:56-72), fully dead strips skipped, and the
 * neutral element (m = -3e38, l = 0, acc = 0) for an empty split
 * (turboquant_paged_decode_attention.cpp:1630-1633). */
static void decode_item(const DecodeJob* j, uint32_t item)
{
    const uint32_t split = item % j->splits;
    const uint32_t kvh = (item / j->splits) % j->Hkv;
    const uint32_t seq = item / (j->splits * j->Hkv);
    const uint32_t G = j->Hq / j->Hkv;
    const uint32_t d = j->d, S = j->S;
    const uint32_t rec = tq4o_record_floats(d);
    const uint32_t ctx = (uint32_t)j->context_lens[seq];
    /* The split partitions the block-table window of max_blocks pages, as the
     * reference AIC decode partitions its page window
     * (turboquant_paged_decode_attention.cpp:1598-1624); pages past ctx hold
     * no live strip and are skipped, so such splits stay neutral. */
    uint32_t pbegin, pcount;
    tq4o_partition(j->max_blocks, j->splits, split, &pbegin, &pcount);

    for (uint32_t g = 0; g < G; ++g) {
        const uint32_t qh = kvh * G + g;
        float q_eff[512];
        const uint16_t* qrow = j->q + ((uint64_t)seq * j->Hq + qh) * d;
        if (j->flags & TQ4O_FLAG_QUERY_ROTATED) {
            for (uint32_t c = 0; c < d; ++c) q_eff[c] = tq4o_bf16_to_f32(qrow[c]) * j->scale;
        } else if (j->flags & TQ4O_FLAG_QROT_BF16) {
            rotate_query_bf16(qrow, j->signs, d, j->inv_sqrt_len, j->scale, q_eff);
        } else {
            tq4o_rotate_query(qrow, j->signs, d, j->inv_sqrt_len, j->scale, q_eff);
        }
        float m = TQ4O_MASKED, l = 0.0f;
        float acc[512];
        for (uint32_t c = 0; c < d; ++c) acc[c] = 0.0f;

        for (uint32_t lp = pbegin; lp < pbegin + pcount; ++lp) {
            const uint32_t phys = (uint32_t)j->block_tables[(uint64_t)seq * j->max_blocks + lp];
            for (uint32_t sip = 0; sip < S / TQ4O_STRIP; ++sip) {
                const uint64_t tbase = (uint64_t)lp * S + sip * TQ4O_STRIP;
                const uint32_t active = tq4o_active_in_strip(tbase, ctx);
                if (active == 0) continue;
                float scores[TQ4O_STRIP];
                float tile_max = TQ4O_MASKED;
                for (uint32_t t = 0; t < TQ4O_STRIP; ++t) {
                    if (t >= active) {
                        scores[t] = TQ4O_MASKED;
                        continue;
                    }
                    const uint32_t tip = sip * TQ4O_STRIP + t;
                    float dot = 0.0f;
                    for (uint32_t c = 0; c < d; ++c)
                        dot += q_eff[c] *
                               (float)tq4o_read_nibble(j->key_cache,
                                                       tq4o_key_nibble(j->Hkv, S, d, phys, kvh, tip, c));
                    scores[t] =
                        dot * j->scale_cache[tq4o_scale_index(j->P, j->Hkv, S, 0, phys, kvh, tip)];
                    if (scores[t] > tile_max) tile_max = scores[t];
                }
                const float m_new = m > tile_max ? m : tile_max;
                const float alpha = expf(m - m_new);
                float p[TQ4O_STRIP];
                float p_sum = 0.0f;
                for (uint32_t t = 0; t < TQ4O_STRIP; ++t) {
                    p[t] = t < active ? expf(scores[t] - m_new) : 0.0f;
                    p_sum += p[t];
                }
                float ps[TQ4O_STRIP];
                for (uint32_t t = 0; t < active; ++t)
                    ps[t] = p[t] * j->scale_cache[tq4o_scale_index(j->P, j->Hkv, S, 1, phys, kvh,
                                                                   sip * TQ4O_STRIP + t)];
                for (uint32_t c = 0; c < d; ++c) {
                    float weighted = 0.0f;
                    for (uint32_t t = 0; t < active; ++t)
                        weighted += ps[t] * (float)tq4o_read_nibble(
                                                j->value_cache,
                                                tq4o_value_nibble(j->Hkv, S, d, phys, kvh,
                                                                  sip * TQ4O_STRIP + t, c));
                    acc[c] = acc[c] * alpha + weighted;
                }
                l = l * alpha + p_sum;
                m = m_new;
            }
        }
        float* out = j->workspace + (((uint64_t)seq * j->Hq + qh) * j->splits + split) * rec;
        out[0] = m;
        out[1] = l;
        out[2] = 0.0f;
        out[3] = 0.0f;
        for (uint32_t c = 0; c < d; ++c) out[4 + c] = acc[c];
    }
}

static void* decode_thread(void* arg)
{
    const DecodeJob* j = (const DecodeJob*)arg;
    for (uint32_t item = j->item_begin; item < j->item_end; ++item) decode_item(j, item);
    return NULL;
}

static int decode_geometry_ok(uint32_t B, uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t S,
                              uint32_t splits)
{
    return B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && d >= 32 && d <= 512 && d % 32 == 0 &&
           (d & (d - 1)) == 0 && S > 0 && S % TQ4O_STRIP == 0 && splits > 0;
}

static int decode_partials_mt(const uint16_t* q, const int8_t* key_cache,
                              const int8_t* value_cache, const float* scale_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              const float* pi_signs, float* workspace, uint32_t num_seqs,
                              uint32_t num_heads, uint32_t num_kv_heads, uint32_t head_size,
                              uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                              float inv_sqrt_len, uint32_t flags, uint32_t threads)
{
    if (!decode_geometry_ok(num_seqs, num_heads, num_kv_heads, head_size, block_size,
                            num_splits))
        return -1;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        if (context_lens[b] < 0) return -1;
        if ((uint64_t)context_lens[b] > (uint64_t)max_blocks_per_seq * block_size) return -1;
    }
    const uint32_t items = num_seqs * num_kv_heads * num_splits;
    if (threads < 1) threads = 1;
    if (threads > items) threads = items;
    if (threads > 256) threads = 256;
    DecodeJob jobs[256];
    pthread_t tids[256];
    for (uint32_t t = 0; t < threads; ++t) {
        DecodeJob* j = &jobs[t];
        j->q = q;
        j->key_cache = key_cache;
        j->value_cache = value_cache;
        j->scale_cache = scale_cache;
        j->block_tables = block_tables;
        j->context_lens = context_lens;
        j->signs = pi_signs;
        j->workspace = workspace;
        j->B = num_seqs;
        j->Hq = num_heads;
        j->Hkv = num_kv_heads;
        j->d = head_size;
        j->S = block_size;
        j->P = num_blocks;
        j->max_blocks = max_blocks_per_seq;
        j->splits = num_splits;
        j->scale = scale;
        j->inv_sqrt_len = inv_sqrt_len;
        j->flags = flags;
        j->item_begin = (uint32_t)((uint64_t)items * t / threads);
        j->item_end = (uint32_t)((uint64_t)items * (t + 1) / threads);
    }
    if (threads == 1) {
        decode_thread(&jobs[0]);
    } else {
        for (uint32_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, decode_thread, &jobs[t]);
        for (uint32_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    return 0;
}

int tq4o_decode_partials(const uint16_t* q, const int8_t* key_cache, const int8_t* value_cache,
                         const float* scale_cache, const int32_t* block_tables,
                         const int32_t* context_lens, const float* pi_signs, float* workspace,
                         uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                         uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                         uint32_t max_blocks_per_seq, uint32_t num_splits, float scale,
                         float inv_sqrt_len, uint32_t flags)
{
    return decode_partials_mt(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                              pi_signs, workspace, num_seqs, num_heads, num_kv_heads, head_size,
                              block_size, num_blocks, max_blocks_per_seq, num_splits, scale,
                              inv_sqrt_len, flags, 1);
}

/* Combine + egress per (seq, q head): the splits merged in split order with
 * combine_step from the identity (l2_atomic_oracle.hpp:100-108,156-176),
 * normalised acc / l (0 when l == 0, paged_decode_oracle.hpp:603-608),
 * then output_stage 0: rotated basis; 1: egress butterfly times invSqrtLen
 * (paged_decode_oracle.hpp:648-665); 2: also divided by 1 + exp(-gate)
 * (single_token_decode_oracle.hpp:325-330). BF16 RNE. */
int tq4o_combine(const float* workspace, const float* pi_signs, const float* gate, uint16_t* out,
                 float* out_f32, uint32_t num_seqs, uint32_t num_heads, uint32_t head_size,
                 uint32_t num_splits, float inv_sqrt_len, uint32_t output_stage)
{
    const uint32_t d = head_size, rec = tq4o_record_floats(d);
    if (output_stage > 2 || (output_stage == 2 && gate == NULL) || num_splits == 0) return -1;
    for (uint64_t row = 0; row < (uint64_t)num_seqs * num_heads; ++row) {
        float m = TQ4O_MASKED, l = 0.0f, acc[512], norm[512], rot[512];
        for (uint32_t c = 0; c < d; ++c) acc[c] = 0.0f;
        for (uint32_t k = 0; k < num_splits; ++k) {
            const float* r = workspace + (row * num_splits + k) * rec;
            tq4o_combine_step(&m, &l, acc, r[0], r[1], r + 4, d);
        }
        for (uint32_t c = 0; c < d; ++c) norm[c] = l == 0.0f ? 0.0f : acc[c] / l;
        if (output_stage == 0) {
            memcpy(rot, norm, d * sizeof(float));
        } else {
            tq4o_rotate_egress(norm, pi_signs, d, rot);
            for (uint32_t c = 0; c < d; ++c) rot[c] *= inv_sqrt_len;
            if (output_stage == 2)
                for (uint32_t c = 0; c < d; ++c) rot[c] = rot[c] / (1.0f + expf(-gate[row * d + c]));
        }
        for (uint32_t c = 0; c < d; ++c) {
            if (out) out[row * d + c] = tq4o_f32_to_bf16(rot[c]);
            if (out_f32) out_f32[row * d + c] = rot[c];
        }
    }
    return 0;
}

int tq4o_paged_decode(const uint16_t* q, const int8_t* key_cache, const int8_t* value_cache,
                      const float* scale_cache, const int32_t* block_tables,
                      const int32_t* context_lens, const float* pi_signs, const float* gate,
                      uint16_t* out, float* out_f32, uint32_t num_seqs, uint32_t num_heads,
                      uint32_t num_kv_heads, uint32_t head_size, uint32_t block_size,
                      uint32_t num_blocks, uint32_t max_blocks_per_seq, uint32_t num_splits,
                      float scale, float inv_sqrt_len, uint32_t output_stage, uint32_t flags,
                      uint32_t threads)
{
    if (num_splits == 0) return -1;
    const size_t floats = (size_t)num_seqs * num_heads * num_splits * tq4o_record_floats(head_size);
    float* ws = (float*)malloc(floats * sizeof(float));
    if (!ws) return -2;
    int rc = decode_partials_mt(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                                pi_signs, ws, num_seqs, num_heads, num_kv_heads, head_size,
                                block_size, num_blocks, max_blocks_per_seq, num_splits, scale,
                                inv_sqrt_len, flags, threads);
    if (rc == 0)
        rc = tq4o_combine(ws, pi_signs, gate, out, out_f32, num_seqs, num_heads, head_size,
                          num_splits, inv_sqrt_len, output_stage);
    free(ws);
    return rc;
}

/* Independent full-context FP64 reference (splitk_decode_fixture.hpp:193-248):
 * direct softmax over the live tokens read through the block table, dead
 * tokens skipped (never weighted by zero), the query rotated by the dense
 * matrix in double, the output rotated back by the dense transpose. */
int tq4o_decode_reference_f64(const uint16_t* q, const int8_t* key_cache,
                              const int8_t* value_cache, const float* scale_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              const float* pi_signs, const float* gate, double* out,
                              uint32_t num_seqs, uint32_t num_heads, uint32_t num_kv_heads,
                              uint32_t head_size, uint32_t block_size, uint32_t num_blocks,
                              uint32_t max_blocks_per_seq, float scale, float inv_sqrt_len,
                              uint32_t output_stage, uint32_t flags)
{
    if (!decode_geometry_ok(num_seqs, num_heads, num_kv_heads, head_size, block_size, 1))
        return -1;
    if (output_stage > 2 || (output_stage == 2 && gate == NULL)) return -1;
    const uint32_t d = head_size, S = block_size, G = num_heads / num_kv_heads;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint32_t ctx = (uint32_t)context_lens[b];
        if ((uint64_t)ctx > (uint64_t)max_blocks_per_seq * S) return -1;
        double* scores = (double*)malloc(sizeof(double) * (ctx ? ctx : 1));
        for (uint32_t qh = 0; qh < num_heads; ++qh) {
            const uint32_t kvh = qh / G;
            double qr[512], acc[512], norm_d[512];
            const uint16_t* qrow = q + ((uint64_t)b * num_heads + qh) * d;
            if (flags & TQ4O_FLAG_QUERY_ROTATED) {
                for (uint32_t c = 0; c < d; ++c) qr[c] = (double)tq4o_bf16_to_f32(qrow[c]) * scale;
            } else {
                float x[512];
                for (uint32_t c = 0; c < d; ++c) x[c] = tq4o_bf16_to_f32(qrow[c]);
                tq4o_rotate_dense(x, pi_signs, d, 0, qr);
                for (uint32_t c = 0; c < d; ++c) qr[c] *= (double)inv_sqrt_len * (double)scale;
            }
            double mx = -INFINITY;
            for (uint32_t t = 0; t < ctx; ++t) {
                const uint32_t phys = (uint32_t)block_tables[(uint64_t)b * max_blocks_per_seq + t / S];
                const uint32_t tip = t % S;
                double dot = 0.0;
                for (uint32_t c = 0; c < d; ++c)
                    dot += qr[c] * (double)tq4o_read_nibble(
                                       key_cache, tq4o_key_nibble(num_kv_heads, S, d, phys, kvh, tip, c));
                scores[t] =
                    dot * (double)scale_cache[tq4o_scale_index(num_blocks, num_kv_heads, S, 0, phys, kvh, tip)];
                if (scores[t] > mx) mx = scores[t];
            }
            double den = 0.0;
            for (uint32_t c = 0; c < d; ++c) acc[c] = 0.0;
            for (uint32_t t = 0; t < ctx; ++t) {
                const uint32_t phys = (uint32_t)block_tables[(uint64_t)b * max_blocks_per_seq + t / S];
                const uint32_t tip = t % S;
                const double w = exp(scores[t] - mx);
                den += w;
                const double pv =
                    w * (double)scale_cache[tq4o_scale_index(num_blocks, num_kv_heads, S, 1, phys, kvh, tip)];
                for (uint32_t c = 0; c < d; ++c)
                    acc[c] += pv * (double)tq4o_read_nibble(
                                       value_cache, tq4o_value_nibble(num_kv_heads, S, d, phys, kvh, tip, c));
            }
            for (uint32_t c = 0; c < d; ++c) norm_d[c] = den > 0.0 ? acc[c] / den : 0.0;
            double* dst = out + ((uint64_t)b * num_heads + qh) * d;
            if (output_stage == 0) {
                for (uint32_t c = 0; c < d; ++c) dst[c] = norm_d[c];
            } else {
                /* dense M^T applied in double */
                for (uint32_t r = 0; r < d; ++r) {
                    double s = 0.0;
                    for (uint32_t c = 0; c < d; ++c) {
                        const int c1 = (int)(c / 32), c0 = (int)(c % 32);
                        const int g = (int)(r / 32), i = (int)(r % 32);
                        s += (double)hadamard(c1, g) * (double)pi_signs[g * 32 + c0] *
                             (double)hadamard(c0, i) * norm_d[c];
                    }
                    s *= (double)inv_sqrt_len;
                    if (output_stage == 2)
                        s = s / (1.0 + exp(-(double)gate[((uint64_t)b * num_heads + qh) * d + r]));
                    dst[r] = s;
                }
            }
        }
        free(scores);
    }
    return 0;
}

/* ==================================================================== codebooks
 * The reference's codebook quantiser leaves (standalone vector routines):
 *   ICDF (scaled sigmoid, signed int4)  routines/routine_vector_icdf_quantize.hpp:10-30,
 *                                       oracle tests/cpu/icdf_fixture.hpp:122-142,222-232
 *   Lloyd-Max (2/4-bit, unsigned codes) include/routines/routine_vector_lloydmax_quantize.hpp:8-37
 *   Gaussian-CDF compander              tests/common/lloydmax_oracle.hpp:19-28,
 *                                       include/routines/routine_vector_gaussian_cdf_quantize.hpp:6-19
 *   packing (low bits first)            tests/common/lloydmax_oracle.hpp:58-62
 * Pins: the reference's fixtures through oracle/_ref (tests/golden/cb_*),
 * plus the closed forms -- centroids are the N(0,1) conditional means of
 * their cells, thresholds the centroid midpoints, the CDF centroids the
 * quantiles (i + 1/2) / 2^b. */

static const float kLm2Centroids[4] = {-1.510418f, -0.452794f, 0.452794f, 1.510418f};
static const float kLm2Thresholds[3] = {-0.981606f, 0.f, 0.981606f};
static const float kLm4Centroids[16] = {
    -2.732589571f, -2.069017227f, -1.618046386f, -1.256231197f, -0.942340456f, -0.656759119f,
    -0.388048299f, -0.128395030f, 0.128395030f,  0.388048299f,  0.656759119f,  0.942340456f,
    1.256231197f,  1.618046386f,  2.069017227f,  2.732589571f};
static const float kLm4Thresholds[15] = {
    -2.400803399f, -1.843531806f, -1.437138792f, -1.099285827f, -0.799549788f,
    -0.522403709f, -0.258221665f, 0.f,           0.258221665f,  0.522403709f,
    0.799549788f,  1.099285827f,  1.437138792f,  1.843531806f,  2.400803399f};
static const float kCdf2Centroids[4] = {-1.1503493804f, -0.318639364f, 0.318639364f,
                                        1.1503493804f};
static const float kCdf4Centroids[16] = {
    -1.8627318674f, -1.3180108973f, -1.0099901692f, -0.7764217611f, -0.5791321623f,
    -0.4022500653f, -0.2372021093f, -0.0784124127f, 0.0784124127f,  0.2372021093f,
    0.4022500653f,  0.5791321623f,  0.7764217611f,  1.0099901692f,  1.3180108973f,
    1.8627318674f};

float tq4o_codebook_centroid(uint32_t book, uint32_t bits, uint32_t q)
{
    if (book == TQ4O_BOOK_LLOYDMAX) return bits == 2 ? kLm2Centroids[q & 3] : kLm4Centroids[q & 15];
    return bits == 2 ? kCdf2Centroids[q & 3] : kCdf4Centroids[q & 15];
}

float tq4o_lloydmax_threshold(uint32_t bits, uint32_t i)
{
    return bits == 2 ? kLm2Thresholds[i] : kLm4Thresholds[i];
}

/* lloydmax_code<Bits>: the number of thresholds t with x >= t (ties to the
 * upper bin; NaN compares false everywhere and gives 0)
 * (include/routines/routine_vector_lloydmax_quantize.hpp:31-37) */
uint32_t tq4o_lloydmax_code(uint32_t bits, float x)
{
    const uint32_t n = bits == 2 ? 3u : 15u;
    uint32_t q = 0;
    for (uint32_t i = 0; i < n; ++i) q += x >= tq4o_lloydmax_threshold(bits, i);
    return q;
}

/* sigmoid_code<Bits>: floor(2^b / (1 + exp(-(1.5976 + 0.070565 x^2) x))),
 * clamped to [0, 2^b - 1], in the reference oracle's FP32 operation order
 * (tests/common/lloydmax_oracle.hpp:21-28) */
uint32_t tq4o_gaussian_cdf_code(uint32_t bits, float x)
{
    const float xx = x * x;
    const float cubic = 0.070565f * xx;
    const float slope = cubic + 1.5976f;
    const float z = slope * x;
    const float e = expf(-z);
    const float d = e + 1.f;
    const float v = (float)(1u << bits) / d;
    const float f = floorf(v);
    const float lo = f > 0.f ? f : 0.f; /* std::max(0.f, f): NaN gives 0 */
    const uint32_t u = (uint32_t)lo;
    const uint32_t top = (1u << bits) - 1u;
    return u < top ? u : top;
}

/* lloyd::pack: code i at bit (i*bits) % 8 of byte i*bits/8 */
void tq4o_codebook_pack(const uint32_t* q, uint64_t n, uint32_t bits, uint8_t* out)
{
    memset(out, 0, (size_t)(n * bits / 8));
    for (uint64_t i = 0; i < n; ++i) out[i * bits / 8] |= (uint8_t)(q[i] << (i * bits % 8));
}

int tq4o_codebook_quantize(uint32_t book, uint32_t bits, const float* x, uint64_t n, float* recon,
                           uint8_t* packed)
{
    if ((bits != 2 && bits != 4) || book > TQ4O_BOOK_GAUSSIAN_CDF || n % (8 / bits)) return -1;
    uint32_t* q = (uint32_t*)malloc((size_t)(n ? n : 1) * sizeof(uint32_t));
    if (!q) return -2;
    for (uint64_t i = 0; i < n; ++i) {
        q[i] = book == TQ4O_BOOK_LLOYDMAX ? tq4o_lloydmax_code(bits, x[i])
                                          : tq4o_gaussian_cdf_code(bits, x[i]);
        if (recon) recon[i] = tq4o_codebook_centroid(book, bits, q[i]);
    }
    if (packed) tq4o_codebook_pack(q, n, bits, packed);
    free(q);
    return 0;
}

/* lloydmax_dequantize_vf: unpack, then the centroid of each code
 * (include/routines/routine_vector_lloydmax_quantize.hpp:223-255) */
int tq4o_codebook_dequantize(uint32_t book, uint32_t bits, const uint8_t* packed, uint64_t n,
                             float* recon)
{
    if ((bits != 2 && bits != 4) || book > TQ4O_BOOK_GAUSSIAN_CDF || n % (8 / bits)) return -1;
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t q = (packed[i * bits / 8] >> (i * bits % 8)) & ((1u << bits) - 1u);
        recon[i] = tq4o_codebook_centroid(book, bits, q);
    }
    return 0;
}

/* IEEE binary16 bits -> float (exact) */
float tq4o_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        const float mag = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return sign ? -mag : mag;
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* The ICDF leaf's code of one value: y = 14 / (1 + exp(-x)) - 7 evaluated in
 * double, rounded to nearest even, saturated to [-8, 7]
 * (tests/cpu/icdf_fixture.hpp:122-142). NaN gives 0. */
int tq4o_icdf_code(double x)
{
    if (x != x) return 0;
    const double y = 14.0 / (1.0 + exp(-x)) - 7.0;
    const double f = floor(y), r = y - f;
    long long q;
    if (r > 0.5) q = (long long)f + 1;
    else if (r < 0.5) q = (long long)f;
    else q = ((long long)f % 2 == 0) ? (long long)f : (long long)f + 1;
    if (q > 7) q = 7;
    if (q < -8) q = -8;
    return (int)q;
}

/* FP16 / BF16 -> packed signed int4, element 2j in bits [3:0] of byte j and
 * element 2j+1 in bits [7:4] (tests/cpu/icdf_fixture.hpp:222-232) */
int tq4o_icdf_quantize(int in_bf16, const uint16_t* in, uint64_t n, uint8_t* packed)
{
    if (n % 2) return -1;
    for (uint64_t j = 0; j < n / 2; ++j) {
        const float a = in_bf16 ? tq4o_bf16_to_f32(in[2 * j]) : tq4o_f16_to_f32(in[2 * j]);
        const float b = in_bf16 ? tq4o_bf16_to_f32(in[2 * j + 1]) : tq4o_f16_to_f32(in[2 * j + 1]);
        const int q0 = tq4o_icdf_code((double)a), q1 = tq4o_icdf_code((double)b);
        packed[j] = (uint8_t)(((q1 & 0xf) << 4) | (q0 & 0xf));
    }
    return 0;
}

/* ==================================================================== RMS codec
 * The vllm-ascend baseline codec, TurboQuantCodec<4>
 * (kernels/ops/turboquant/baseline/common/turboquant_codec_950.h), applied by
 * the baseline writer to every (token, plane, kv head) vector
 * (kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:98-246):
 *   ApplyPi     x * s, FWHT at strides 1, 2, 4, ..., n/2 (a + b | a - b),
 *               * inv_sqrt_len, * s                       codec_950.h:115-151
 *   scale       sqrt(sum y^2) * inv_sqrt_len + 1e-20       codec_950.h:186-197
 *   level       #{i : y * (-1/scale) + t_i has its sign bit set}
 *               = #{i : t_i < y * (1/scale)}               codec_950.h:199-231
 *   byte        (even level + 16 * odd level) - 128, int8  codec_950.h:234-248
 *   dequantize  byte + 128 -> even/odd level -> centroid   codec_950.h:251-285
 * (-1/s rounds to -(1/s) and y * (-r) to -(y * r), and t - z rounds to a
 * value of the exact difference's sign, never -0 since t_7 is +0, so the
 * sign-bit count is the strict count.) The 15 thresholds and 16 centroids
 * are the Lloyd-Max 4-bit codebook (codec_950.h:43-51; centroid table
 * tests/npu/bench/bench_turboquant_reshape_and_cache.cpp:55-61).
 * The sum of squares runs in this library's order -- 16 sequential partial
 * sums over n/16 consecutive elements, then a pairwise tree over the
 * partials (xor 1, 2, 4, 8), the GPU kernel's lane reduction; the
 * reference device's ReduceSum order belongs to CANN and is not restated.
 * Pins: ApplyPi equals tq4o_kv4fp8_apply_pi (pinned to the reference's
 * fixture) bit for bit; the scale equals the FP64 closed form to a few ulp;
 * the tables equal the pinned Lloyd-Max codebook; levels against a
 * brute-force count at every threshold and its neighbours. */

static const float kRmsThresholds[15] = {
    -2.4008033987632817f, -1.8435318062766393f, -1.4371387916845330f, -1.0992858269170722f,
    -0.7995497875097155f, -0.5224037090113789f, -0.2582216646707196f, 0.0f,
    0.2582216646707196f,  0.5224037090113789f,  0.7995497875097155f,  1.0992858269170722f,
    1.4371387916845330f,  1.8435318062766393f,  2.4008033987632817f};
static const float kRmsCentroids[16] = {
    -2.7325895709951710f, -2.0690172265313920f, -1.6180463860218863f, -1.2562311973471796f,
    -0.9423404564869651f, -0.6567591185324659f, -0.3880482994902919f, -0.1283950298511473f,
    0.1283950298511473f,  0.3880482994902919f,  0.6567591185324659f,  0.9423404564869651f,
    1.2562311973471796f,  1.6180463860218863f,  2.0690172265313920f,  2.7325895709951710f};

float tq4o_rms_threshold(uint32_t i) { return kRmsThresholds[i % 15u]; }
float tq4o_rms_centroid(uint32_t level) { return kRmsCentroids[level & 15u]; }

void tq4o_rms_apply_pi(float* x, const float* signs, float inv_sqrt_len, uint32_t n)
{
    for (uint32_t i = 0; i < n; ++i) x[i] = x[i] * signs[i];
    for (uint32_t s = 1; s < n; s <<= 1)
        for (uint32_t i = 0; i < n; ++i)
            if (!(i & s)) {
                const float a = x[i], b = x[i | s];
                x[i] = a + b;
                x[i | s] = a - b;
            }
    for (uint32_t i = 0; i < n; ++i) x[i] = x[i] * inv_sqrt_len;
    for (uint32_t i = 0; i < n; ++i) x[i] = x[i] * signs[i];
}

float tq4o_rms_scale(const float* y, uint32_t n, float inv_sqrt_len)
{
    float part[16];
    const uint32_t per = n / 16u;
    for (uint32_t l = 0; l < 16u; ++l) {
        float s = y[l * per] * y[l * per];
        for (uint32_t j = 1; j < per; ++j) s = s + y[l * per + j] * y[l * per + j];
        part[l] = s;
    }
    for (uint32_t m = 1; m < 16u; m <<= 1) {
        float nxt[16];
        for (uint32_t l = 0; l < 16u; ++l) nxt[l] = part[l] + part[l ^ m];
        memcpy(part, nxt, sizeof(part));
    }
    return sqrtf(part[0]) * inv_sqrt_len + 1e-20f;
}

uint32_t tq4o_rms_level(float y, float rcp)
{
    const float z = y * rcp;
    uint32_t q = 0;
    for (uint32_t i = 0; i < 15u; ++i) q += kRmsThresholds[i] < z;
    return q;
}

/* One vector: ApplyPi on a copy, scale, levels, packed bytes. */
void tq4o_rms_quantize_row(const float* x, const float* signs, uint32_t n, float inv_sqrt_len,
                           uint8_t* levels, int8_t* packed, float* scale)
{
    float y[256];
    memcpy(y, x, n * sizeof(float));
    tq4o_rms_apply_pi(y, signs, inv_sqrt_len, n);
    const float s = tq4o_rms_scale(y, n, inv_sqrt_len);
    const float r = 1.0f / s;
    for (uint32_t p = 0; p < n / 2u; ++p) {
        const uint32_t lo = tq4o_rms_level(y[2 * p], r), hi = tq4o_rms_level(y[2 * p + 1], r);
        if (levels) {
            levels[2 * p] = (uint8_t)lo;
            levels[2 * p + 1] = (uint8_t)hi;
        }
        packed[p] = (int8_t)(uint8_t)((lo | (hi << 4)) ^ 0x80u);
    }
    *scale = s;
}

uint32_t tq4o_rms_scale_slot_floats(uint32_t num_kv_heads)
{
    return (2u * num_kv_heads + 7u) / 8u * 8u;
}

/* The baseline writer (TurboQuantReshapeAndCache, turboquant_paged_attention.cpp:98-246):
 * tokens below token_limit whose slot lies in [0, num_blocks * block_size)
 * write key row slot*H*(d/2) + h*(d/2), the value row likewise, and the
 * slot's scale record [2H scales (K heads, then V heads), zero padding to
 * a multiple of 8]. in_dtype 0 FP16, 1 BF16. Returns the rows written. */
int64_t tq4o_rms_reshape_and_cache(int in_dtype, const uint16_t* key, const uint16_t* value,
                                   int8_t* key_cache, int8_t* value_cache, float* scale_cache,
                                   const int32_t* slots, const float* signs, uint32_t num_tokens,
                                   uint32_t H, uint32_t d, uint32_t S, uint32_t P,
                                   uint32_t token_limit, float inv_sqrt_len)
{
    if ((d != 64 && d != 128 && d != 256) || !H || !S || !P) return -1;
    const uint64_t slots_total = (uint64_t)P * S;
    const uint32_t ssf = tq4o_rms_scale_slot_floats(H);
    const uint32_t T = token_limit < num_tokens ? token_limit : num_tokens;
    int64_t written = 0;
    for (uint32_t t = 0; t < T; ++t) {
        const int32_t slot = slots[t];
        if (slot < 0 || (uint64_t)slot >= slots_total) continue;
        float* rec = scale_cache + (uint64_t)slot * ssf;
        for (uint32_t i = 0; i < ssf; ++i) rec[i] = 0.0f;
        for (uint32_t plane = 0; plane < 2u * H; ++plane) {
            const uint16_t* src = (plane < H ? key : value) + ((uint64_t)t * H + plane % H) * d;
            float x[256];
            for (uint32_t c = 0; c < d; ++c)
                x[c] = in_dtype ? tq4o_bf16_to_f32(src[c]) : tq4o_f16_to_f32(src[c]);
            int8_t* dst = (plane < H ? key_cache : value_cache) +
                          ((uint64_t)slot * H + plane % H) * (d / 2u);
            tq4o_rms_quantize_row(x, signs, d, inv_sqrt_len, NULL, dst, &rec[plane]);
            ++written;
        }
    }
    return written;
}

/* Dequantize4Bit: packed bytes -> centroids, element 2j from byte j's low
 * nibble (after the +128 bias), 2j+1 from its high nibble. */
void tq4o_rms_dequantize(const int8_t* packed, uint64_t n, float* out)
{
    for (uint64_t j = 0; j < n / 2u; ++j) {
        const uint32_t v = (uint32_t)(uint8_t)packed[j] ^ 0x80u;
        out[2 * j] = kRmsCentroids[v & 15u];
        out[2 * j + 1] = kRmsCentroids[v >> 4];
    }
}
