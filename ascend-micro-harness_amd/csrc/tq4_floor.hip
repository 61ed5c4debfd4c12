// libtq4_floor.so: compute-free copies of four launches, for measurement only
// (bench.py --floor). Nothing in libtq4.so uses them.
//
// tq4_floor_decode_launch: the configs[2] decode's memory chain without its
// arithmetic, on the decode's own grid (one 256-lane workgroup per (seq, kv
// head, split), splits fastest) and buffers. Stages, cumulative by `mode`:
//   0  each workgroup writes its output words;
//   1  + phase 0: context length, q rows, signs, the split's block-table
//      window staged in LDS, one barrier;
//   2  + each wave's two strip pairs loaded (the decode's lane layout,
//      xor-reduced so the loads cannot be dropped), a merge barrier;
//   3  + the fused combine's exchange: a ticket per split, device-coherent
//      (sc1) record stores by all but the last ticket holder, which polls
//      the K records (16 per round trip, bounded), zeroes them and writes
//      the output rows.
// tq4_floor_writer_launch: the configs[1] writer's traffic without its
// arithmetic: per (strip of 16 tokens, kv head) the slots and 16 BF16 key
// and value rows in; one 64-byte key row per token, the 1 KiB value strip
// and 32 scales out. mode 0 stores only; mode 1 loads and stores (each store
// depends on the loaded words).
//
// tq4_floor_scatter_launch: the token scatter writer's traffic without its
// arithmetic (configs[1]'s secondary row, and the configs[4] step's writer):
// per (token, kv head) the slot and the two BF16 rows in, the token's value
// strip read after the slot and written back whole, its key row and two
// scales out; mode 0 stores only, mode 1 loads and stores.
//
// tq4_floor_gather_launch: the configs[4] decode's cache reads without its
// arithmetic, queue or combine: every listed strip (one live (sequence, kv
// head, page) of 16 tokens: its 1 KiB key strip, 1 KiB value strip and two
// 64-byte scale rows) is read once, four strips in flight per wave, over a
// grid of the caller's size; the list is built on the host from the block
// tables, so the kernel reads nothing but the cache and its own index.
//
// Geometry is fixed to the rows measured and checked on the host (-1
// otherwise): decode d = 128, GQA 4, 16-token pages, K = 16, 256-page
// tables (16 pages = 8 strip pairs per split, two per wave); writers d = 128,
// 16-token pages (whole strips for the strip writer's copy).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

struct FloorDecode {
    const uint16_t* q;
    const int8_t* key_cache;
    const int8_t* value_cache;
    const float* scale_cache;
    const int32_t* block_tables;
    const int32_t* context_lens;
    const float* pi_signs;
    float* records;     // [B][Hq][K][d + 4]
    uint32_t* tickets;  // [B][Hkv] counters, 32 words apart, zero between launches
    uint16_t* out;      // [B][Hq][d]
    uint32_t B, Hq, Hkv, G, S, P, max_blocks, K, mode;
};

struct FloorWriter {
    const uint16_t* key;
    const uint16_t* value;
    const int32_t* slots;
    int8_t* key_cache;
    int8_t* value_cache;
    float* scale_cache;
    uint32_t H, D, S, P, tokens, mode;
};

struct FloorScatter {
    const uint16_t* key;
    const uint16_t* value;
    const int32_t* slots;
    int8_t* key_cache;
    int8_t* value_cache;
    float* scale_cache;
    uint32_t H, D, S, P, tokens, mode;
};

struct FloorGather {
    const int8_t* key_cache;
    const int8_t* value_cache;
    const float* scale_cache;
    const uint32_t* rows;  // first cache row ((page * Hkv + head) * 16) of each strip
    uint32_t* out;         // one word per workgroup
    uint32_t n_rows, P, Hkv;
};

constexpr int kD = 128, kRS = kD + 4;
constexpr uint32_t kMagic = 0x7FBADBADu;  // a written record word is never zero
constexpr int kSc1 = 16;                  // device-coherent cache policy
constexpr uint32_t kPollLimit = 1u << 20;
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const float* base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7fffffff,
                                             0x00020000);
}

__global__ __launch_bounds__(256) void floor_decode_kernel(FloorDecode p)
{
    __shared__ uint32_t strip[64];
    __shared__ uint32_t red[4][64];
    __shared__ int flag;
    const uint32_t item = blockIdx.x;
    const uint32_t split = item % p.K, kvh = (item / p.K) % p.Hkv, seq = item / (p.K * p.Hkv);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = p.G;
    uint32_t x = 0;
    if (p.mode >= 1) {
        const int32_t c = p.context_lens[seq];
        uint32_t qx = 0;
        for (int i = 0; i < 4; ++i) {
            const uint32_t g = min((uint32_t)wave + 4 * i, G - 1);
            const uint16_t* qr = p.q + ((size_t)seq * p.Hq + kvh * G + g) * kD + lane * 2;
            qx ^= qr[0] ^ ((uint32_t)qr[1] << 16);
        }
        const float s0 = p.pi_signs[lane * 2], s1 = p.pi_signs[lane * 2 + 1];
        const uint32_t width = (p.max_blocks + p.K - 1) / p.K;
        const uint32_t pb = split * width;
        const uint32_t pc = min(width, p.max_blocks - min(pb, p.max_blocks));
        if ((uint32_t)tid < pc && tid < 64) {
            const int32_t phys = p.block_tables[(size_t)seq * p.max_blocks + pb + tid];
            strip[tid] = ((uint32_t)phys * p.Hkv + kvh) * p.S;  // 16-token pages: one strip each
        }
        lds_barrier();
        x = qx ^ (uint32_t)c ^ __float_as_uint(s0) ^ __float_as_uint(s1);
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    uint32_t ticket = 0;
    if (p.mode >= 2) {
        const int n = lane & 15, g4 = lane >> 4, half = g4 & 1, sp = g4 >> 1;
        const size_t plane = (size_t)p.P * p.Hkv * p.S;
        uint32_t acc = 0;
        u4 kw[2][2], vw[2][2];
        float scw[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t gp = wave + 4 * j;  // 8 pairs in the 16-strip window
            const uint32_t s0 = 2 * gp;
            const uint32_t rk = strip[s0 + (n >> 3)], rv = strip[s0 + sp];
            const uint32_t t1 = 8 * ((n >> 2) & 1) + (n & 3);
            const int8_t* kb = p.key_cache + (size_t)(rk + t1) * (kD / 2) + g4 * (kD / 8);
            kw[j][0] = *(const u4*)kb;
            kw[j][1] = *(const u4*)(kb + 4 * (kD / 2));
            const int8_t* vb8 = p.value_cache + (size_t)rv * (kD / 2) + n * (kD / 2) + 16 * half;
            vw[j][0] = *(const u4*)vb8;
            vw[j][1] = *(const u4*)(vb8 + 32);
            scw[j] = p.scale_cache[(size_t)half * plane + rv + n];
        }
        if (p.mode >= 3 && tid == 0)
            ticket = __hip_atomic_fetch_add(p.tickets + ((size_t)seq * p.Hkv + kvh) * 32, 1u,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc ^= kw[j][0][e] ^ kw[j][1][e] ^ vw[j][0][e] ^ vw[j][1][e];
            acc ^= __float_as_uint(scw[j]);
        }
        red[wave][lane] = acc ^ x;
        if (p.mode >= 3 && tid == 0) {
            const int last = ticket == p.K - 1;
            if (last)
                __hip_atomic_store(p.tickets + ((size_t)seq * p.Hkv + kvh) * 32, 0u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            flag = last;
        }
        lds_barrier();
        x = red[0][lane] ^ red[1][lane] ^ red[2][lane] ^ red[3][lane];
    }
    const float val = 1.0f + (float)(x & 0xffu);
    if (p.mode >= 3) {
        if (!flag) {
            // export: G * d/4 float4 of the row values and a header per row
            const uint32_t e4 = tid;
            if (e4 < G * kD / 4) {
                const uint32_t r = e4 / (kD / 4), ch = 4 * (e4 % (kD / 4));
                const __amdgpu_buffer_rsrc_t rs =
                    rsrc_of(p.records + (((size_t)seq * p.Hq + kvh * G + r) * p.K + split) * kRS);
                const uint32_t w = __float_as_uint(val) ^ kMagic;
                __builtin_amdgcn_raw_buffer_store_b128(u4{w, w, w, w}, rs, (4 + ch) * 4u, 0, kSc1);
                if (ch == 0)
                    __builtin_amdgcn_raw_buffer_store_b128(u4{w, w, kMagic, kMagic}, rs, 0, 0, kSc1);
            }
            return;
        }
        // the last ticket holder: wave g polls row g's K records (its own
        // slot skipped), 16 per round trip, at most kPollLimit times
        const uint32_t g = wave;
        if (g >= G) return;
        const __amdgpu_buffer_rsrc_t rs =
            rsrc_of(p.records + ((size_t)seq * p.Hq + kvh * G + g) * p.K * kRS);
        const int c = lane & 31, ks = lane >> 5;
        u2 hw[8];
        u4 aw[8];
        float sum = 0.0f;
        for (uint32_t it = 0; it < kPollLimit; ++it) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t k = ks + 2 * i;  // K = 16
                hw[i] = __builtin_amdgcn_raw_buffer_load_b64(rs, k * kRS * 4u, 0, kSc1);
                aw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, k * kRS * 4u + 4u * (4 + 4 * c),
                                                              0, kSc1);
            }
            uint32_t mn = 0xffffffffu;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t k = ks + 2 * i;
                const uint32_t m = min(min(hw[i][0], hw[i][1]),
                                       min(min(aw[i][0], aw[i][1]), min(aw[i][2], aw[i][3])));
                mn = k == split ? mn : min(mn, m);
            }
            if (!__any(mn == 0u)) break;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t k = ks + 2 * i;
            __builtin_amdgcn_raw_buffer_store_b64(u2{0u, 0u}, rs, k * kRS * 4u, 0, kSc1);
            __builtin_amdgcn_raw_buffer_store_b128(u4{0u, 0u, 0u, 0u}, rs,
                                                   k * kRS * 4u + 4u * (4 + 4 * c), 0, kSc1);
            sum += __uint_as_float(aw[i][0] ^ kMagic) + __uint_as_float(hw[i][1] ^ kMagic);
        }
        sum += __shfl_xor(sum, 32, 64);
        if (lane < 32) {
            uint16_t* dst = p.out + ((size_t)seq * p.Hq + kvh * G + g) * kD + c * 4;
            const uint32_t b = __float_as_uint(sum + val) >> 16;
            *(u2*)dst = u2{b | (b << 16), b | (b << 16)};
        }
        return;
    }
    // modes 0..2: split 0 writes its rows directly
    for (uint32_t g = wave; g < G; g += 4) {
        if (lane < 32 && split == 0) {
            uint16_t* dst = p.out + ((size_t)seq * p.Hq + kvh * G + g) * kD + (lane & 31) * 4;
            const uint32_t b = __float_as_uint(val) >> 16;
            *(u2*)dst = u2{b | (b << 16), b | (b << 16)};
        }
    }
}

__global__ __launch_bounds__(256) void floor_writer_kernel(FloorWriter p)
{
    const uint32_t strip = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const int t = threadIdx.x, j = t >> 4, c = t & 15;  // token j of the strip, 16-byte chunk c
    const uint32_t tok = strip * 16 + j;
    uint32_t x = 0x11u;
    int32_t slot = (int32_t)tok;
    if (p.mode >= 1) {
        slot = p.slots[tok];
        const u4 kw = *(const u4*)(p.key + ((size_t)tok * p.H + h) * kD + c * 8);
        const u4 vw = *(const u4*)(p.value + ((size_t)tok * p.H + h) * kD + c * 8);
        x = kw[0] ^ kw[1] ^ kw[2] ^ kw[3] ^ vw[0] ^ vw[1] ^ vw[2] ^ vw[3];
    }
    const uint32_t page = (uint32_t)slot / 16u, tip = (uint32_t)slot % 16u;
    if (page >= p.P) return;  // the slots name pages of the pool
    const size_t row = ((size_t)page * p.H + h) * 16 + tip;
    *(uint32_t*)(p.key_cache + row * 64 + c * 4) = x;
    const size_t srow = ((size_t)page * p.H + h) * 16;
    *(uint32_t*)(p.value_cache + srow * 64 + (size_t)t * 4) = x;
    if (c == 0) {
        p.scale_cache[row] = (float)(x & 0xff);
        p.scale_cache[(size_t)p.P * p.H * 16 + row] = (float)(x & 0xff);
    }
}

// The token scatter's traffic without its arithmetic: per (token, kv head)
// item, a 16-lane group as in the scatter writer, sixteen items a workgroup.
// mode 0 stores only (the token's key row, its whole 1 KiB value strip and
// two scales, at a strip of its own); mode 1 adds the slot, the two BF16 rows
// and, after the slot, the value strip's read (each store depends on the
// loaded words).
__global__ __launch_bounds__(256) void floor_scatter_kernel(FloorScatter p)
{
    const int tid = threadIdx.x, l = tid & 15;
    const uint32_t item = blockIdx.x * 16 + (tid >> 4);
    if (item >= p.tokens * p.H) return;
    const uint32_t tok = item / p.H, h = item % p.H;
    uint32_t x = 0x11u;
    int32_t slot = (int32_t)(tok * 16u);
    u4 sw[4] = {u4{0u, 0u, 0u, 0u}, u4{0u, 0u, 0u, 0u}, u4{0u, 0u, 0u, 0u}, u4{0u, 0u, 0u, 0u}};
    if (p.mode >= 1) {
        slot = p.slots[tok];
        const u4 kw = *(const u4*)(p.key + ((size_t)tok * p.H + h) * kD + l * 8);
        const u4 vw = *(const u4*)(p.value + ((size_t)tok * p.H + h) * kD + l * 8);
        x = kw[0] ^ kw[1] ^ kw[2] ^ kw[3] ^ vw[0] ^ vw[1] ^ vw[2] ^ vw[3];
        const uint32_t pg = (uint32_t)slot / 16u;
        const size_t srow = ((size_t)(pg < p.P ? pg : 0u) * p.H + h) * 16;
        const u4* strip = (const u4*)(p.value_cache + srow * 64 + (size_t)l * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) sw[i] = strip[i];
    }
    const uint32_t page = (uint32_t)slot / 16u, tip = (uint32_t)slot % 16u;
    if (page >= p.P) return;  // the slots name pages of the pool
    const size_t srow = ((size_t)page * p.H + h) * 16;
    *(uint32_t*)(p.key_cache + (srow + tip) * 64 + (size_t)l * 4) = x;
    u4* dst = (u4*)(p.value_cache + srow * 64 + (size_t)l * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = sw[i] ^ u4{x, x, x, x};
    if (l == 0) {
        p.scale_cache[srow + tip] = (float)(x & 0xff);
        p.scale_cache[(size_t)p.P * p.H * 16 + srow + tip] = (float)(x & 0xff);
    }
}

__global__ __launch_bounds__(256) void floor_gather_kernel(FloorGather p)
{
    const int lane = threadIdx.x & 63;
    const uint32_t waves = gridDim.x * 4u;
    const uint32_t w = blockIdx.x * 4u + (threadIdx.x >> 6);
    const size_t plane = (size_t)p.P * p.Hkv * 16;
    uint32_t acc = 0;
    // rows of the next four strips, loaded one batch ahead (clamped indices)
    uint32_t nxt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) nxt[u] = p.rows[min(w + u * waves, p.n_rows - 1)];
    for (uint32_t i = w; i < p.n_rows; i += 4 * waves) {
        uint32_t cur[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
#pragma unroll
        for (int u = 0; u < 4; ++u) nxt[u] = p.rows[min(i + (4 + u) * waves, p.n_rows - 1)];
        u4 kw[4], vw[4];
        float sk[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            kw[u] = *(const u4*)(p.key_cache + (size_t)cur[u] * (kD / 2) + lane * 16);
            vw[u] = *(const u4*)(p.value_cache + (size_t)cur[u] * (kD / 2) + lane * 16);
            // lanes 0..15: key scales, 16..31: value scales, the rest reload the key scales
            sk[u] = p.scale_cache[((lane >> 4) == 1 ? plane : 0) + cur[u] + (lane & 15)];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool live = i + u * waves < p.n_rows;
            const uint32_t x = kw[u][0] ^ kw[u][1] ^ kw[u][2] ^ kw[u][3] ^ vw[u][0] ^ vw[u][1] ^
                               vw[u][2] ^ vw[u][3] ^ __float_as_uint(sk[u]);
            acc ^= live ? x : 0u;
        }
    }
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t a = 0;
        for (int t = 0; t < 256; ++t) a ^= red[t];
        p.out[blockIdx.x] = a;
    }
}

}  // namespace

extern "C" int tq4_floor_scatter_launch(void* stream, const FloorScatter* p)
{
    if (p == nullptr || p->D != 128 || p->S != 16 || p->tokens == 0 || p->mode > 1 ||
        (uint64_t)p->tokens * p->H > (1ull << 26))
        return -1;
    const uint32_t items = p->tokens * p->H;
    hipLaunchKernelGGL(floor_scatter_kernel, dim3((items + 15) / 16), dim3(256), 0,
                       (hipStream_t)stream, *p);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int tq4_floor_gather_launch(void* stream, const FloorGather* p, uint32_t workgroups)
{
    if (p == nullptr || p->n_rows == 0 || workgroups == 0 || workgroups > 65535) return -1;
    hipLaunchKernelGGL(floor_gather_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       *p);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int tq4_floor_decode_launch(void* stream, const FloorDecode* p)
{
    if (p == nullptr || p->G != 4 || p->S != 16 || p->K != 16 || p->max_blocks != 256 ||
        p->Hq != p->Hkv * p->G || p->mode > 3)
        return -1;
    hipLaunchKernelGGL(floor_decode_kernel, dim3(p->B * p->Hkv * p->K), dim3(256), 0,
                       (hipStream_t)stream, *p);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int tq4_floor_writer_launch(void* stream, const FloorWriter* p)
{
    if (p == nullptr || p->D != 128 || p->S != 16 || p->tokens % 16 != 0 || p->mode > 1)
        return -1;
    hipLaunchKernelGGL(floor_writer_kernel, dim3(p->tokens / 16 * p->H), dim3(256), 0,
                       (hipStream_t)stream, *p);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
