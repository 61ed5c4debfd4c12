/* kv4fp8_oracle.h -- C restatement of the reference's KV4/FP8 fused decode
 * (the 64-token NZ-tiled cache and its decode), for the tests.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it as the checker. The product path never links it.
 *
 * Reference (paths relative to the reference checkout; the integration copy
 * under kernels/ops/turboquant/vllm_integration_layer/op_kernel/ is "opk/"):
 *   cache layout       opk/common/turboquant_layout.h:81-92 (NzTiledPackedByte)
 *   levels and gain    opk/common/turboquant_mode.h:95-117 (KV4_FP8: signed
 *                      nibble + 0.5, kGain), opk/common/turboquant_codec_mx.h:
 *                      289-312,435-441 (UnpackAffine, ComputeNibbleOperands)
 *   FP8 operands       opk/common/turboquant_codec_mx.h:349-359 (CAST_RINT),
 *                      opk/vector/turboquant_vector_service.h:342-345 (448)
 *   query operand      opk/vector/turboquant_vector_service.h:1033-1058
 *   tile recurrence    opk/vector/routine_vector_cube_softmax.hpp:36-75,
 *                      opk/vector/turboquant_vector_service.h:594-679
 *   tail mask          opk/vector/turboquant_vector_service.h:541-549
 *   task / partials    opk/turboquant_fused_decode.cpp:479-568,
 *                      opk/vector/turboquant_vector_service.h:472-486,1181-1201
 *   split reduce       opk/vector/turboquant_vector_service.h:253-320
 *   normalise / cast   opk/vector/turboquant_vector_service.h:144-185
 *   output stages      opk/cube/turboquant_query_basis.h:181-208,
 *                      opk/common/turboquant_codec_950.h:115-153 (ApplyPi)
 *   task partition     kernels/ops/turboquant/vllm_integration_layer/include/
 *                      turboquant_fused_decode.hpp (build_decode_tiling)
 */
#ifndef KV4FP8_ORACLE_H
#define KV4FP8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint32_t tokens, heads, kv_heads, head_size, block_size, max_blocks, num_blocks;
    uint32_t splits, fused_context_limit;
    float scale, inv_sqrt_len;
    uint32_t output_stage;  /* 0 rotated basis, 1 Pi applied, 2 Pi then gate */
    uint32_t element_type;  /* output (and raw query / gate) format: 0 fp16, 1 bf16 */
} tq4o_kv4fp8_geom;

uint64_t tq4o_nz_byte(uint64_t slot, uint64_t kv_head, uint64_t column, uint64_t kv_heads,
                      uint64_t packed_bytes);
uint8_t tq4o_fp8_e4m3_encode(float x);
float tq4o_fp8_e4m3_decode(uint8_t b);
uint16_t tq4o_f32_to_f16(float x);
float tq4o_elem_to_f32(uint32_t element_type, uint16_t bits);
uint16_t tq4o_f32_to_elem(uint32_t element_type, float x);
void tq4o_kv4fp8_apply_pi(float* x, const float* signs, float inv_sqrt_len, uint32_t n);
void tq4o_kv4fp8_rotate_query(uint32_t element_type, const uint16_t* raw, const float* signs,
                              float inv_sqrt_len, uint64_t vectors, uint32_t n, float* out);
uint32_t tq4o_kv4fp8_partial_floats(uint32_t head_size);
int tq4o_kv4fp8_decode(const tq4o_kv4fp8_geom* g, const float* query, const uint8_t* key,
                       const uint8_t* value, const float* scales, const int32_t* block_table,
                       const int32_t* context_lens, const float* pi_signs, const uint16_t* gate,
                       float* workspace, uint16_t* out, float* out_f32, int threads);

#ifdef __cplusplus
}
#endif
#endif
