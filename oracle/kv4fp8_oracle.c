/* kv4fp8_oracle.c -- C restatement of the reference's KV4/FP8 fused decode.
 *
 * TEST INFRASTRUCTURE ONLY (see kv4fp8_oracle.h for what may use it and for
 * the reference files each part follows). Plain C11, -ffp-contract=off, so
 * every FP32 operation is rounded where the reference rounds it: the
 * per-head query operand, the tile logits (S * key scale) * 1/qScale, the
 * online-softmax step, the probability operand, the decayed accumulator,
 * the split merge, 1/(sum + eps), the output stage and the RNE output cast.
 * The two products the reference runs on its matrix unit (Q.K^T and P.V over
 * FP8 operands, FP32 accumulation) are summed here in double and rounded to
 * FP32 once; their operands are exact, so only the summation order differs.
 */
#include "kv4fp8_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define KV4_TILE 64u              /* kCubeTileRows, turboquant_layout.h:51 */
#define KV4_C0 32u                /* kOperandC0, turboquant_layout.h:53 */
#define KV4_SCALE_SLOT 8u         /* FP32 lanes per slot: K scales, then V scales */
#define KV4_MAX_SPLITS 8u         /* kMaxSequenceSplits, turboquant_layout.h:40 */
#define KV4_PARTIAL_TAIL 16u      /* kPartialTail = 2 * kFp32PerBlock */
static const float kGain = 2.9832882881f;       /* TurboQuantModeTraits<KV4_FP8>::kGain */
static const float kOperandMax = 448.0f;        /* OperandMax<KV4_FP8> (e4m3 max) */
static const float kEps = 1e-20f;               /* TurboQuantCodec4::kEps */
static const float kNegInf = -3.4028235e38f;    /* kVectorNegInf */
static const float kMaskGain = -5.0e36f;        /* kMaskGain */
static const float kMaskMidpoint = 0.5f;        /* kMaskMidpoint */
static const float kGateFloor = -80.0f;         /* kGateLogitFloor */

static uint32_t bits_of(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float float_of(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* NzTiledPackedByte: [tile of 64 rows][kv head][32-byte column group][tile row][byte]. */
uint64_t tq4o_nz_byte(uint64_t slot, uint64_t kv_head, uint64_t column, uint64_t kv_heads,
                      uint64_t packed_bytes)
{
    const uint64_t tile_row = slot % KV4_TILE;
    return (slot - tile_row) * kv_heads * packed_bytes + kv_head * KV4_TILE * packed_bytes +
           ((column / KV4_C0) * KV4_TILE + tile_row) * KV4_C0 + column % KV4_C0;
}

/* FP32 -> OCP FP8 e4m3 (bias 7, max 448, no infinities), round to nearest
 * even, subnormals kept (step 2^-9). The decode only ever converts values of
 * magnitude <= 448 (both operand maps scale their maximum to 448); above it
 * this saturates to +-448. NaN -> 0x7F with the sign. */
uint8_t tq4o_fp8_e4m3_encode(float x)
{
    const uint32_t u = bits_of(x);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
    const float a = float_of(au);
    if (a > 464.0f) return (uint8_t)(sign | 0x7eu);
    if (a < 0.015625f) {  /* below the smallest normal 2^-6: multiples of 2^-9 */
        const float r = rintf(a * 512.0f);
        return (uint8_t)(sign | (uint8_t)r);  /* r == 8 is 2^-6, the first normal */
    }
    uint32_t r = au + 0x7ffffu + ((au >> 20) & 1u);  /* RNE to 3 mantissa bits */
    r &= 0xfff00000u;
    const int e = (int)(r >> 23) - 127;
    const uint32_t m = (r >> 20) & 7u;
    if (e > 8) return (uint8_t)(sign | 0x7eu);
    return (uint8_t)(sign | (uint8_t)(((uint32_t)(e + 7) << 3) | m));
}

float tq4o_fp8_e4m3_decode(uint8_t b)
{
    const int e = (b >> 3) & 15, m = b & 7;
    if (e == 15 && m == 7) return NAN;
    const float v = e ? ldexpf(1.0f + (float)m / 8.0f, e - 7) : ldexpf((float)m / 8.0f, -6);
    return (b & 0x80) ? -v : v;
}

static float fp8_round(float x) { return tq4o_fp8_e4m3_decode(tq4o_fp8_e4m3_encode(x)); }

/* FP32 -> FP16, round to nearest even (subnormals, overflow to infinity). */
uint16_t tq4o_f32_to_f16(float x)
{
    const uint32_t u = bits_of(x);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* >= 65520 rounds to inf */
    if (au < 0x38800000u) {  /* below 2^-14: multiples of 2^-24 */
        const float r = rintf(float_of(au) * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t r = au + 0xfffu + ((au >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)((r >> 13) - (112u << 10)));
}

static float f16_to_f32(uint16_t h)
{
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) {
        const float v = ldexpf((float)m, -24);
        return (h & 0x8000u) ? -v : v;
    }
    if (e == 31) return float_of(s | 0x7f800000u | (m << 13));
    return float_of(s | ((e + 112u) << 23) | (m << 13));
}

static uint16_t f32_to_bf16(float x)
{
    const uint32_t u = bits_of(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float tq4o_elem_to_f32(uint32_t element_type, uint16_t bits)
{
    return element_type ? float_of((uint32_t)bits << 16) : f16_to_f32(bits);
}

uint16_t tq4o_f32_to_elem(uint32_t element_type, float x)
{
    return element_type ? f32_to_bf16(x) : tq4o_f32_to_f16(x);
}

/* ApplyPi (turboquant_codec_950.h:115-153): x *= signs; the unnormalised
 * Walsh-Hadamard butterflies at strides 1, 2, 4, ..., n/2 (lower = a + b,
 * upper = a - b); x *= inv_sqrt_len; x *= signs. */
void tq4o_kv4fp8_apply_pi(float* x, const float* signs, float inv_sqrt_len, uint32_t n)
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

/* The raw-query prologue (turboquant_query_basis.h): widen, ApplyPi, FP32. */
void tq4o_kv4fp8_rotate_query(uint32_t element_type, const uint16_t* raw, const float* signs,
                              float inv_sqrt_len, uint64_t vectors, uint32_t n, float* out)
{
    for (uint64_t v = 0; v < vectors; ++v) {
        float* x = out + v * n;
        for (uint32_t c = 0; c < n; ++c) x[c] = tq4o_elem_to_f32(element_type, raw[v * n + c]);
        tq4o_kv4fp8_apply_pi(x, signs, inv_sqrt_len, n);
    }
}

uint32_t tq4o_kv4fp8_partial_floats(uint32_t head_size) { return head_size + KV4_PARTIAL_TAIL; }

/* The level of packed column `col`'s nibble `hi` (signed int4 + 0.5). */
static float level(uint8_t byte, int hi)
{
    int n = hi ? (byte >> 4) : (byte & 15);
    if (n >= 8) n -= 16;
    return (float)n + 0.5f;
}

typedef struct {
    const tq4o_kv4fp8_geom* g;
    const float *query, *scales, *pi_signs;
    const uint8_t *key, *value;
    const int32_t *block_table, *context_lens;
    const uint16_t* gate;
    float* partials;  /* [token][head][split][D + 16] */
    uint16_t* out;
    float* out_f32;
    int status;
} kv4_job;

/* Finish one normalised head row: output stage, then the element cast. */
static void finish_row(const kv4_job* j, uint32_t token, uint32_t head, float* acc)
{
    const tq4o_kv4fp8_geom* g = j->g;
    const uint32_t D = g->head_size;
    const uint64_t row = (uint64_t)token * g->heads + head;
    if (g->output_stage >= 1) tq4o_kv4fp8_apply_pi(acc, j->pi_signs, g->inv_sqrt_len, D);
    if (g->output_stage == 2) {
        for (uint32_t c = 0; c < D; ++c) {
            float gv = tq4o_elem_to_f32(g->element_type, j->gate[row * D + c]);
            gv = gv > kGateFloor ? gv : kGateFloor;  /* Maxs */
            float den = gv * -1.0f;
            den = expf(den);
            den = den + 1.0f;
            acc[c] = acc[c] / den;
        }
    }
    for (uint32_t c = 0; c < D; ++c) {
        if (j->out) j->out[row * D + c] = tq4o_f32_to_elem(g->element_type, acc[c]);
        if (j->out_f32) j->out_f32[row * D + c] = acc[c];
    }
}

/* NormalizeHeads: sum += eps; inv = 1 / sum; acc *= inv. */
static void normalise(float* acc, float sum, uint32_t D)
{
    sum = sum + kEps;
    const float inv = 1.0f / sum;
    for (uint32_t c = 0; c < D; ++c) acc[c] = acc[c] * inv;
}

/* One worker task: (token, kv head, split) over rows [r0, r1), all heads of
 * the group. Leaves (acc, runMax, runSum) per head in the state arrays. */
static void run_task(const kv4_job* j, uint32_t token, uint32_t kvh, uint32_t r0, uint32_t r1,
                     float* acc, float* run_max, float* run_sum)
{
    const tq4o_kv4fp8_geom* g = j->g;
    const uint32_t D = g->head_size, PB = D / 2, H = g->kv_heads, G = g->heads / g->kv_heads;
    const uint32_t S = g->block_size;
    /* BeginTask */
    for (uint32_t h = 0; h < G; ++h) {
        run_max[h] = kNegInf;
        run_sum[h] = 0.0f;
        for (uint32_t c = 0; c < D; ++c) acc[h * D + c] = 0.0f;
    }
    if (r1 <= r0) return;
    /* StageQuery / ComputeQueryOperandRows */
    float* qop = (float*)malloc(sizeof(float) * G * D);
    float* qinv = (float*)malloc(sizeof(float) * G);
    for (uint32_t h = 0; h < G; ++h) {
        const float* q = j->query + ((uint64_t)token * g->heads + kvh * G + h) * D;
        float amax = 0.0f;
        for (uint32_t c = 0; c < D; ++c) {
            const float a = fabsf(q[c]);
            amax = a > amax ? a : amax;
        }
        amax = amax + kEps;
        const float qscale = kOperandMax / amax;
        qinv[h] = 1.0f / qscale;
        for (uint32_t c = 0; c < D; ++c) qop[h * D + c] = fp8_round(q[c] * qscale);
    }
    const float score_scale = g->scale / kGain, inv_gain = 1.0f / kGain;
    float ks[KV4_TILE], vs[KV4_TILE], s[KV4_TILE], p[KV4_TILE], pop[KV4_TILE];
    float kop[KV4_TILE][512], vop[KV4_TILE][512];
    for (uint32_t t0 = r0; t0 < r1; t0 += KV4_TILE) {
        const uint32_t valid = r1 - t0 < KV4_TILE ? r1 - t0 : KV4_TILE;
        const uint32_t page = t0 / S, row0 = t0 % S;
        const int32_t entry = j->block_table[(uint64_t)token * g->max_blocks + page];
        if (entry < 0 || (uint32_t)entry >= g->num_blocks) continue;  /* unmapped: dropped */
        const uint64_t base = (uint64_t)(uint32_t)entry * S * H * PB;
        for (uint32_t r = 0; r < KV4_TILE; ++r) {
            const uint64_t slot = ((uint64_t)(uint32_t)entry * S + row0 + r) * KV4_SCALE_SLOT;
            ks[r] = j->scales[slot + kvh] * score_scale;
            vs[r] = j->scales[slot + H + kvh] * inv_gain;
            for (uint32_t col = 0; col < PB; ++col) {
                const uint64_t at = base + tq4o_nz_byte(row0 + r, kvh, col, H, PB);
                kop[r][col] = level(j->key[at], 0);
                kop[r][col + PB] = level(j->key[at], 1);
                vop[r][col] = level(j->value[at], 0);
                vop[r][col + PB] = level(j->value[at], 1);
            }
        }
        for (uint32_t h = 0; h < G; ++h) {
            /* logits */
            for (uint32_t r = 0; r < KV4_TILE; ++r) {
                double acc_s = 0.0;
                for (uint32_t c = 0; c < D; ++c) acc_s += (double)qop[h * D + c] * kop[r][c];
                float v = (float)acc_s;
                v = v * ks[r];
                v = v * qinv[h];
                if (valid < KV4_TILE) {
                    float mask = (float)r + (kMaskMidpoint - (float)valid);
                    mask = mask * kMaskGain;
                    v = v < mask ? v : mask;  /* Min */
                }
                s[r] = v;
            }
            /* update_max_and_alpha, exponentiate_scores, update_denominator */
            float tile_max = s[0];
            for (uint32_t r = 1; r < KV4_TILE; ++r) tile_max = s[r] > tile_max ? s[r] : tile_max;
            const float new_max = run_max[h] > tile_max ? run_max[h] : tile_max;
            float alpha = run_max[h] - new_max;
            alpha = expf(alpha);
            float part = 0.0f;
            for (uint32_t r = 0; r < KV4_TILE; ++r) {
                p[r] = expf(s[r] - new_max);
                part += p[r];
            }
            run_sum[h] = run_sum[h] * alpha;
            run_sum[h] = run_sum[h] + part;
            /* quantize_probabilities */
            float pm = 0.0f;
            for (uint32_t r = 0; r < KV4_TILE; ++r) {
                p[r] = p[r] * vs[r];
                pm = p[r] > pm ? p[r] : pm;
            }
            pm = pm + kEps;
            const float prob_scale = kOperandMax / pm;
            for (uint32_t r = 0; r < KV4_TILE; ++r) pop[r] = fp8_round(p[r] * prob_scale);
            /* ComputeAccumulatorDecay, then ComputeAccumulate */
            const float inv = 1.0f / prob_scale;
            for (uint32_t c = 0; c < D; ++c) {
                double ctx = 0.0;
                for (uint32_t r = 0; r < KV4_TILE; ++r) ctx += (double)pop[r] * vop[r][c];
                float a = acc[h * D + c] * alpha;
                float x = (float)ctx;
                x = x * inv;
                acc[h * D + c] = a + x;
            }
            run_max[h] = new_max;
        }
    }
    free(qop);
    free(qinv);
}

/* All of one (token, kv head): the tiling's tasks, then the fused write or
 * the split reduce. */
static int run_token_head(kv4_job* j, uint32_t token, uint32_t kvh)
{
    const tq4o_kv4fp8_geom* g = j->g;
    const uint32_t D = g->head_size, G = g->heads / g->kv_heads, S = g->block_size;
    const uint32_t K = g->splits;
    const int32_t raw = j->context_lens[token];
    const uint32_t context = raw > 0 ? (uint32_t)raw : 0u;
    const int fused = K <= 1 || raw <= (int32_t)g->fused_context_limit;
    const uint32_t seq_blocks = (context + S - 1) / S;
    const uint32_t bps = fused ? seq_blocks : (seq_blocks + K - 1) / K;
    float* acc = (float*)malloc(sizeof(float) * G * D * (K + 1));
    float* mx = (float*)malloc(sizeof(float) * G * (K + 1));
    float* sm = (float*)malloc(sizeof(float) * G * (K + 1));
    int status = 0;
    for (uint32_t sp = 0; sp < (fused ? 1u : K); ++sp) {
        float* a = acc + (size_t)sp * G * D;
        uint32_t r0 = 0, r1 = 0;
        const uint32_t b0 = sp * bps;
        if (b0 < seq_blocks) {
            uint32_t b1 = b0 + bps;
            if (b1 > seq_blocks) b1 = seq_blocks;
            if (b1 > g->max_blocks) { status = -2; break; }
            r0 = b0 * S;
            r1 = b1 * S < context ? b1 * S : context;
        }
        run_task(j, token, kvh, r0, r1, a, mx + sp * G, sm + sp * G);
        if (!fused && j->partials) {
            for (uint32_t h = 0; h < G; ++h) {
                float* w = j->partials +
                           (((uint64_t)token * g->heads + kvh * G + h) * K + sp) *
                               tq4o_kv4fp8_partial_floats(D);
                memcpy(w, a + h * D, sizeof(float) * D);
                memset(w + D, 0, sizeof(float) * KV4_PARTIAL_TAIL);
                w[D + 0] = mx[sp * G + h];
                w[D + 8] = sm[sp * G + h];
            }
        }
    }
    if (status == 0) {
        float row[512];
        for (uint32_t h = 0; h < G; ++h) {
            if (fused) {
                memcpy(row, acc + h * D, sizeof(float) * D);
                normalise(row, sm[h], D);
            } else {
                /* TurboQuantPartialReducer::Reduce */
                float run_max = kNegInf, run_sum = 0.0f;
                for (uint32_t c = 0; c < D; ++c) row[c] = 0.0f;
                for (uint32_t sp = 0; sp < K; ++sp) {
                    const float pmax = mx[sp * G + h];
                    float psum = sm[sp * G + h];
                    const float new_max = run_max > pmax ? run_max : pmax;
                    const float alpha = expf(run_max - new_max);
                    const float beta = expf(pmax - new_max);
                    run_sum = run_sum * alpha;
                    psum = psum * beta;
                    run_sum = run_sum + psum;
                    const float* pa = acc + (size_t)sp * G * D + h * D;
                    for (uint32_t c = 0; c < D; ++c) {
                        const float x = row[c] * alpha;
                        const float y = pa[c] * beta;
                        row[c] = x + y;
                    }
                    run_max = new_max;
                }
                normalise(row, run_sum, D);
            }
            finish_row(j, token, kvh * G + h, row);
        }
    }
    free(acc);
    free(mx);
    free(sm);
    return status;
}

typedef struct {
    kv4_job* j;
    uint32_t first, step;
} kv4_thread_arg;

static void* kv4_thread(void* p)
{
    kv4_thread_arg* a = (kv4_thread_arg*)p;
    const tq4o_kv4fp8_geom* g = a->j->g;
    const uint32_t n = g->tokens * g->kv_heads;
    for (uint32_t i = a->first; i < n; i += a->step) {
        const int st = run_token_head(a->j, i / g->kv_heads, i % g->kv_heads);
        if (st) a->j->status = st;
    }
    return NULL;
}

/* Geometry as valid_launch (include/turboquant_fused_decode_opt.hpp:66-96)
 * admits it, less the NPU's grid bounds: D = 256 (kHeadSize), 1..4 KV heads
 * (an eight-lane scale slot), heads % kv_heads == 0, a page that is a
 * power-of-two multiple of 64, 1..8 splits. Returns 0, or -1 on a refused
 * geometry, -2 when a split's pages run past max_blocks. */
int tq4o_kv4fp8_decode(const tq4o_kv4fp8_geom* g, const float* query, const uint8_t* key,
                       const uint8_t* value, const float* scales, const int32_t* block_table,
                       const int32_t* context_lens, const float* pi_signs, const uint16_t* gate,
                       float* workspace, uint16_t* out, float* out_f32, int threads)
{
    if (!g || !g->tokens || !g->kv_heads || g->kv_heads > 4 || !g->heads ||
        g->heads % g->kv_heads || g->head_size != 256 || !g->block_size ||
        g->block_size % KV4_TILE || (g->block_size & (g->block_size - 1)) || !g->max_blocks ||
        !g->splits || g->splits > KV4_MAX_SPLITS || g->output_stage > 2 || g->element_type > 1)
        return -1;
    if (g->output_stage >= 1 && !pi_signs) return -1;
    if (g->output_stage == 2 && !gate) return -1;
    kv4_job j;
    memset(&j, 0, sizeof j);
    j.g = g;
    j.query = query;
    j.key = key;
    j.value = value;
    j.scales = scales;
    j.block_table = block_table;
    j.context_lens = context_lens;
    j.pi_signs = pi_signs;
    j.gate = gate;
    j.partials = workspace;
    j.out = out;
    j.out_f32 = out_f32;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tids[64];
    kv4_thread_arg args[64];
    for (int t = 0; t < threads; ++t) {
        args[t].j = &j;
        args[t].first = (uint32_t)t;
        args[t].step = (uint32_t)threads;
    }
    if (threads == 1) {
        kv4_thread(&args[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, kv4_thread, &args[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    return j.status;
}
