// ref_driver.cpp -- a C-ABI shim over the reference's own header-only CPU
// oracles, compiled in place from /root/reference (see oracle/Makefile) into
// oracle/_ref/libtq4_ref.so.
//
// TEST INFRASTRUCTURE ONLY. It exists so the tests and tests/golden/
// gen_golden.py can ask the reference's oracles for golden vectors and check
// the C restatement in oracle/tq4_oracle.c against them. Nothing here is on
// the product path. No reference source is copied: the headers are included
// from where they lie.
//
// Reference headers used (paths relative to the reference checkout):
//   tests/common/turboquant_oracle.hpp            tq_oracle
//   tests/common/turboquant_scatter_oracle.hpp    tq_scatter
//   tests/common/rotate_butterfly_oracle.hpp      rot_oracle
//   tests/common/l2_atomic_oracle.hpp             l2_probe_oracle
//   tests/common/aic_splitk_decode_fixture.hpp    splitk_decode_test
//   include/turboquant_splitk_contract.hpp        turboquant_splitk
//   kernels/ops/turboquant/turboquant_decode_tail.hpp  turboquant_decode_tail
//   tests/cpu/icdf_fixture.hpp                    icdf (ICDF leaf fixture + oracle)
//   tests/common/lloydmax_oracle.hpp              lloyd (Lloyd-Max / Gaussian-CDF)
//   tests/common/fused_decode_opt_fixture.hpp     fused_decode_opt_test (KV4/FP8
//                                                 NZ cache fixture, FP64 expected)

#include "tests/common/turboquant_oracle.hpp"
#include "tests/common/turboquant_scatter_oracle.hpp"
#include "tests/common/rotate_butterfly_oracle.hpp"
#include "tests/common/l2_atomic_oracle.hpp"
#include "tests/common/aic_splitk_decode_fixture.hpp"
#include "include/turboquant_splitk_contract.hpp"
#include "kernels/ops/turboquant/turboquant_decode_tail.hpp"
#include "tests/cpu/icdf_fixture.hpp"
#include "tests/common/lloydmax_oracle.hpp"
#include "tests/common/fused_decode_opt_fixture.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

namespace {

tq_oracle::Shape make_shape(int num_tokens, int heads, int head_size, int block_size,
                            int num_blocks)
{
    tq_oracle::Shape s;
    s.num_tokens = num_tokens;
    s.num_kv_heads = heads;
    s.head_size = head_size;
    s.block_size = block_size;
    s.num_blocks = num_blocks;
    return s;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- tq_oracle
int ref_tq_shape_valid(int num_tokens, int heads, int head_size, int block_size, int num_blocks)
{
    return make_shape(num_tokens, heads, head_size, block_size, num_blocks).valid() ? 1 : 0;
}

void ref_tq_build_activations(int num_tokens, int heads, int head_size, int block_size,
                              int num_blocks, int8_t* key, int8_t* value)
{
    std::vector<int8_t> k, v;
    tq_oracle::build_activations(make_shape(num_tokens, heads, head_size, block_size, num_blocks),
                                 k, v);
    std::memcpy(key, k.data(), k.size());
    std::memcpy(value, v.data(), v.size());
}

void ref_tq_build_slot_mapping(int num_tokens, int heads, int head_size, int block_size,
                               int num_blocks, int32_t* slots)
{
    const auto s = tq_oracle::build_slot_mapping(
        make_shape(num_tokens, heads, head_size, block_size, num_blocks));
    std::memcpy(slots, s.data(), s.size() * sizeof(int32_t));
}

void ref_tq_build_tables(int head_size, int8_t* tables)
{
    const auto t = tq_oracle::build_tables(make_shape(16, 1, head_size, 16, 1));
    std::memcpy(tables, t.data(), t.size());
}

long long ref_tq_audit_tables(int head_size, const int8_t* tables)
{
    return tq_oracle::audit_tables(make_shape(16, 1, head_size, 16, 1), tables);
}

// compute_oracle_reference: the full cache images (unwritten pages zero),
// page_written flags and the first strip that violated the slot contract.
int ref_tq_compute_reference(int num_tokens, int heads, int head_size, int block_size,
                             int num_blocks, const int8_t* key, const int8_t* value,
                             const int32_t* slots, int8_t* key_cache, int8_t* value_cache,
                             float* scale_cache, char* page_written, int* audit_ok)
{
    try {
        const auto shape = make_shape(num_tokens, heads, head_size, block_size, num_blocks);
        const auto ref = tq_oracle::compute_oracle_reference(shape, key, value, slots);
        std::memcpy(key_cache, ref.key_cache.data(), ref.key_cache.size());
        std::memcpy(value_cache, ref.value_cache.data(), ref.value_cache.size());
        std::memcpy(scale_cache, ref.scale_cache.data(), ref.scale_cache.size() * sizeof(float));
        std::memcpy(page_written, ref.page_written.data(), ref.page_written.size());
        if (audit_ok) *audit_ok = tq_oracle::audit_reference(ref).ok() ? 1 : 0;
        return ref.bad_slot_strip;
    } catch (const std::exception&) {
        return -2;
    }
}

long long ref_tq_rint_even_shift(long long y, int shift)
{
    return tq_oracle::rint_even_shift(y, shift);
}

int ref_tq_pi_sign(int channel) { return tq_oracle::pi_sign(channel); }

// --------------------------------------------------------------- rot_oracle
// d = 256 only (rot_oracle::kChannels).
void ref_rot_staged(int direction, const float* x, const float* signs, float scale, float* y)
{
    const auto v = rot_oracle::staged(direction ? rot_oracle::Direction::Ingress
                                                : rot_oracle::Direction::Egress,
                                      x, signs, scale);
    std::memcpy(y, v.data(), v.size() * sizeof(float));
}

void ref_rot_dense_left(const float* x, const float* signs, float* y)
{
    const auto v = rot_oracle::dense_left(x, signs);
    std::memcpy(y, v.data(), v.size() * sizeof(float));
}

void ref_rot_dense_right(const float* x, const float* signs, float* y)
{
    const auto v = rot_oracle::dense_right(x, signs);
    std::memcpy(y, v.data(), v.size() * sizeof(float));
}

// --------------------------------------------------------------- tq_scatter
// Integer-valued BF16 activation for (request, plane, head, token, channel).
float ref_scatter_activation(int request, int plane, int head, int token, int channel,
                             int zero_token)
{
    return tq_scatter::activation(request, plane, head, token, channel, zero_token);
}

// compute_reference over one token per entry of `slots` (request r owns tokens
// [cu[r], cu[r+1])), d = 256. The prior images are updated in place.
int ref_scatter_compute_reference(int num_requests, int heads, int block_size, int num_blocks,
                                  const int32_t* cu_seqlens, const int32_t* slots,
                                  const float* signs, int zero_token, int8_t* key_cache,
                                  int8_t* value_cache, float* scale_cache, int* zero_rows,
                                  int* clamped_rows)
{
    try {
        tq_scatter::Shape shape;
        shape.num_requests = num_requests;
        shape.num_kv_heads = heads;
        shape.head_size = 256;
        shape.block_size = block_size;
        shape.num_blocks = num_blocks;
        if (!shape.valid()) return -1;
        std::vector<tq_scatter::TokenPlan> plans;
        for (int r = 0; r < num_requests; ++r)
            for (int t = cu_seqlens[r]; t < cu_seqlens[r + 1]; ++t)
                plans.push_back(tq_scatter::plan_token(shape, r, t, slots[t]));
        std::vector<float> sg(signs, signs + 256);
        std::vector<int8_t> pk(key_cache, key_cache + shape.cache_bytes());
        std::vector<int8_t> pv(value_cache, value_cache + shape.cache_bytes());
        std::vector<float> ps(scale_cache, scale_cache + shape.scale_floats());
        const auto ref = tq_scatter::compute_reference(shape, plans, sg, zero_token, pk, pv, ps);
        std::memcpy(key_cache, ref.key_cache.data(), ref.key_cache.size());
        std::memcpy(value_cache, ref.value_cache.data(), ref.value_cache.size());
        std::memcpy(scale_cache, ref.scale_cache.data(), ref.scale_cache.size() * sizeof(float));
        if (zero_rows) *zero_rows = ref.zero_rows;
        if (clamped_rows) *clamped_rows = ref.clamped_rows;
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

unsigned long long ref_scatter_value_nibble(int heads, int head_size, int block_size,
                                            int num_blocks, int block, int head, int token,
                                            int channel)
{
    tq_scatter::Shape s;
    s.num_kv_heads = heads;
    s.head_size = head_size;
    s.block_size = block_size;
    s.num_blocks = num_blocks;
    return tq_scatter::value_nibble(s, block, head, token, channel);
}

unsigned long long ref_scatter_key_nibble(int heads, int head_size, int block_size,
                                          int num_blocks, int block, int head, int token,
                                          int channel)
{
    tq_scatter::Shape s;
    s.num_kv_heads = heads;
    s.head_size = head_size;
    s.block_size = block_size;
    s.num_blocks = num_blocks;
    return tq_scatter::key_nibble(s, block, head, token, channel);
}

unsigned long long ref_scatter_scale_index(int heads, int block_size, int num_blocks, int plane,
                                           int block, int head, int token)
{
    tq_scatter::Shape s;
    s.num_kv_heads = heads;
    s.block_size = block_size;
    s.num_blocks = num_blocks;
    return tq_scatter::scale_index(s, plane, block, head, token);
}

// ------------------------------------------------------------ split-K / tail
void ref_partition(unsigned pages, unsigned splits, unsigned split, unsigned* begin,
                   unsigned* count)
{
    const auto r = turboquant_splitk::Partition(pages, splits, split);
    *begin = r.begin;
    *count = r.count;
}

unsigned ref_active_in_strip(unsigned long long token_base, unsigned seq_len)
{
    return turboquant_decode_tail::ActiveInStrip(token_base, seq_len);
}

unsigned ref_live_strips_in_window(unsigned seq_len, unsigned page_begin, unsigned seq_pages,
                                   unsigned block_size, unsigned strip_begin, unsigned strips)
{
    return turboquant_decode_tail::LiveStripsInWindow(seq_len, page_begin, seq_pages, block_size,
                                                      strip_begin, strips);
}

// ---------------------------------------------------------- l2_probe_oracle
// One combine step over d = 256 records laid out [m, l, acc[256]].
void ref_l2_combine_step(const float* curr, const float* tile, float* out)
{
    l2_probe_oracle::State a, b;
    a.m = curr[0];
    a.l = curr[1];
    b.m = tile[0];
    b.l = tile[1];
    for (int c = 0; c < 256; ++c) {
        a.acc[c] = curr[2 + c];
        b.acc[c] = tile[2 + c];
    }
    const auto r = l2_probe_oracle::combine_step(a, b);
    out[0] = r.m;
    out[1] = r.l;
    for (int c = 0; c < 256; ++c) out[2 + c] = r.acc[c];
}

// tile_state for split k of a fixture (0 uniform, 1 staggered) as [m, l, acc].
void ref_l2_tile_state(int fixture, unsigned split, float* out)
{
    const auto s = l2_probe_oracle::tile_state(
        fixture ? l2_probe_oracle::Fixture::Staggered : l2_probe_oracle::Fixture::Uniform, split);
    out[0] = s.m;
    out[1] = s.l;
    for (int c = 0; c < 256; ++c) out[2 + c] = s.acc[c];
}

int ref_l2_uniform_expected(unsigned splits, unsigned reps, float* out)
{
    try {
        const auto s = l2_probe_oracle::uniform_expected(splits, reps);
        out[0] = s.m;
        out[1] = s.l;
        for (int c = 0; c < 256; ++c) out[2 + c] = s.acc[c];
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// The sequential combine of splits 0..K-1 in order, then the tail egress
// (normalise, Pi on the right with 1/16, gate_vector, no bf16 rounding).
void ref_l2_combine_and_egress(int fixture, unsigned splits, float* combined, float* egress)
{
    std::vector<std::uint32_t> order(splits);
    for (unsigned k = 0; k < splits; ++k) order[k] = k;
    const auto s = l2_probe_oracle::combine_sequence(
        fixture ? l2_probe_oracle::Fixture::Staggered : l2_probe_oracle::Fixture::Uniform, order);
    combined[0] = s.m;
    combined[1] = s.l;
    for (int c = 0; c < 256; ++c) combined[2 + c] = s.acc[c];
    const auto e = l2_probe_oracle::egress_reference(s);
    std::memcpy(egress, e.data(), 256 * sizeof(float));
}

void ref_l2_gate_vector(float* gate)
{
    const auto g = l2_probe_oracle::gate_vector();
    std::memcpy(gate, g.data(), 256 * sizeof(float));
}

// ------------------------------------------------------ splitk_decode_test
// The dynamically sized fixture, d = 256. Sizes the caller must allocate:
//   q, gate, expected: batch*heads*rows*256
//   key, value: batch*pages*heads*page*128 bytes; scales: batch*pages*heads*page*2
//   table: batch*pages; signs: 256
int ref_splitk_fixture_dims(int n, int page_size, int* pages, int* tokens)
{
    *pages = (n + page_size - 1) / page_size;
    *tokens = *pages * page_size;
    return 0;
}

int ref_splitk_fixture(int n, int batch, int heads, int rows, int page_size, int live, int fill,
                       uint16_t* q, uint8_t* key, uint8_t* value, float* scales, float* gate,
                       float* signs, uint32_t* table, float* expected)
{
    try {
        const auto tf = fill == 0   ? splitk_decode_test::TailFill::kZero
                        : fill == 1 ? splitk_decode_test::TailFill::kDirty
                                    : splitk_decode_test::TailFill::kNaN;
        splitk_decode_test::Fixture f(n, batch, heads, rows, page_size, live, tf);
        std::memcpy(q, f.q.data(), f.q.size() * 2);
        std::memcpy(key, f.key.data(), f.key.size());
        std::memcpy(value, f.value.data(), f.value.size());
        std::memcpy(scales, f.scales.data(), f.scales.size() * 4);
        std::memcpy(gate, f.gate.data(), f.gate.size() * 4);
        std::memcpy(signs, f.signs.data(), f.signs.size() * 4);
        std::memcpy(table, f.table.data(), f.table.size() * 4);
        std::memcpy(expected, f.expected.data(), f.expected.size() * 4);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

// ReferenceAicPartial for one (request, head, page window), 16 rows: FP64
// m[16], l[16], acc[16*256]. Requires a fixture built with rows == 16.
int ref_aic_partial(int n, int batch, int heads, int page_size, int live, int fill, int request,
                    int head, unsigned begin, unsigned pages, double* m, double* l, double* acc)
{
    try {
        const auto tf = fill == 0   ? splitk_decode_test::TailFill::kZero
                        : fill == 1 ? splitk_decode_test::TailFill::kDirty
                                    : splitk_decode_test::TailFill::kNaN;
        splitk_decode_test::Fixture f(n, batch, heads, splitk_decode_test::kAicRows, page_size,
                                      live, tf);
        const auto p = splitk_decode_test::ReferenceAicPartial(f, request, head, begin, pages);
        std::memcpy(m, p.m.data(), p.m.size() * 8);
        std::memcpy(l, p.l.data(), p.l.size() * 8);
        std::memcpy(acc, p.acc.data(), p.acc.size() * 8);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

// ------------------------------------------------------------- codebooks
// icdf::make_fixture(bf16, tiles): tiles*1024 input half/bf16 words and the
// oracle's tiles*512 packed bytes; -2 if the fixture's own property checks fail.
int ref_icdf_fixture(int bf16, uint32_t tiles, uint16_t* in_bits, uint8_t* packed)
{
    try {
        const icdf::Fixture fx = icdf::make_fixture(bf16 != 0, tiles);
        icdf::assert_properties(fx);
        std::memcpy(in_bits, fx.in_bits.data(), fx.in_bits.size() * 2);
        std::memcpy(packed, fx.oracle_packed.data(), fx.oracle_packed.size());
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

// lloyd::fixture(n, rows, boundaries, bits): n*rows FP32 values
void ref_lloyd_fixture(unsigned n, unsigned rows, int boundaries, unsigned bits, float* x)
{
    const auto v = lloyd::fixture(n, rows, boundaries != 0, bits);
    std::memcpy(x, v.data(), v.size() * 4);
}

unsigned ref_lloyd_code(unsigned bits, float x, int sigmoid)
{
    return lloyd::code(bits, x, sigmoid != 0);
}

float ref_lloyd_centroid(unsigned bits, unsigned q, int sigmoid)
{
    return lloyd::centroid(bits, q, sigmoid != 0);
}

float ref_lloyd_threshold(unsigned bits, unsigned i)
{
    return bits == 2 ? ascend_micro::LloydMaxCodebook<2>::thresholds[i]
                     : ascend_micro::LloydMaxCodebook<4>::thresholds[i];
}

void ref_lloyd_pack(const unsigned* q, unsigned n, unsigned bits, uint8_t* out)
{
    const std::vector<unsigned> v(q, q + n);
    const auto p = lloyd::pack(v, bits);
    std::memcpy(out, p.data(), p.size());
}

// ------------------------------------------------- fused_decode_opt_test (KV4/FP8)
// sizes[0..5]: query floats, cache bytes (key = value), scale floats, table
// ints, length ints, physical pages.
int ref_fdo_dims(int n, int b, int h, int g, int block, long long* sizes)
{
    try {
        const fused_decode_opt_test::Fixture f(n, b, h, g, block);
        sizes[0] = (long long)f.query.size();
        sizes[1] = (long long)f.key.size();
        sizes[2] = (long long)f.scales.size();
        sizes[3] = (long long)f.table.size();
        sizes[4] = (long long)f.lengths.size();
        sizes[5] = f.physical_pages;
        return f.pages;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_fdo_fixture(int n, int b, int h, int g, int block, int element, float* query, uint8_t* key,
                    uint8_t* value, float* scales, int32_t* table, int32_t* lengths,
                    float* expected, uint16_t* expected_bits)
{
    try {
        const auto e = element ? fused_decode_opt_test::Element::kBf16
                               : fused_decode_opt_test::Element::kFp16;
        const fused_decode_opt_test::Fixture f(n, b, h, g, block, e);
        std::memcpy(query, f.query.data(), f.query.size() * 4);
        std::memcpy(key, f.key.data(), f.key.size());
        std::memcpy(value, f.value.data(), f.value.size());
        std::memcpy(scales, f.scales.data(), f.scales.size() * 4);
        std::memcpy(table, f.table.data(), f.table.size() * 4);
        std::memcpy(lengths, f.lengths.data(), f.lengths.size() * 4);
        std::memcpy(expected, f.expected.data(), f.expected.size() * 4);
        for (std::size_t i = 0; i < f.expected.size(); ++i)
            expected_bits[i] = fused_decode_opt_test::reference_bits(e, f.expected[i]);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// The raw-query entry's inputs for one fixture: the original-basis query and
// the gate logits (element bits), the sign vector, and the expected rows of
// output stage `stage` (float).
int ref_fdo_raw(int n, int b, int h, int g, int block, int element, unsigned stage,
                uint16_t* raw_query, uint16_t* gate_bits, float* pi_signs, float* expected)
{
    try {
        const auto e = element ? fused_decode_opt_test::Element::kBf16
                               : fused_decode_opt_test::Element::kFp16;
        const fused_decode_opt_test::Fixture f(n, b, h, g, block, e);
        const fused_decode_opt_test::RawQueryBasis basis;
        const auto raw = f.raw_query(basis);
        std::memcpy(raw_query, raw.data(), raw.size() * 2);
        const auto gl = f.gate_logits();
        std::memcpy(gate_bits, gl.data(), gl.size() * 2);
        std::memcpy(pi_signs, basis.signs.data(), basis.signs.size() * 4);
        const std::size_t rows = f.query.size() / 256;
        for (std::size_t r = 0; r < rows; ++r) {
            const auto row = f.expected_row(basis, r, stage);
            std::memcpy(expected + r * 256, row.data(), 256 * 4);
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

float ref_fdo_gain()
{
    return vllm_ascend::turboquant::TurboQuantModeTraits<
        vllm_ascend::turboquant::TurboQuantMode::KV4_FP8>::kGain;
}

unsigned long long ref_nz_byte(unsigned long long slot, unsigned long long kv_head,
                               unsigned long long column, unsigned long long kv_heads,
                               unsigned long long packed_bytes)
{
    return vllm_ascend::turboquant::NzTiledPackedByte(slot, kv_head, column, kv_heads,
                                                       packed_bytes);
}

}  // extern "C"

