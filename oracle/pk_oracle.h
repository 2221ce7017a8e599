/*
 * pk_oracle.h -- CPU restatement of the l4-parakeet-rs quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels in libpk_linear.so.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in the product links it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Conventions: weights are [N x K] row-major ("weight_oi", linear.cu:75-77),
 * activations [M x K] row-major, fp16 values are passed as raw uint16 bits.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
uint16_t orc_f32_to_f16(float value);
float orc_f16_to_f32(uint16_t bits);
uint8_t orc_f32_to_e4m3(float value);
float orc_e4m3_to_f32(uint8_t bits);
float orc_e3m2_to_f32(uint8_t bits);
uint8_t orc_e3m2_of_int(int v);
void orc_fp6_chunks(const int8_t* codes, size_t count, uint8_t* out);
int8_t orc_quantize_i8(float value);
float orc_pattern(uint64_t index, uint64_t salt, float amplitude);
void orc_pattern_fill(float* out, size_t count, uint64_t first_index, uint64_t salt,
                      float amplitude);

/* ---- size contracts (packing.rs, exl3.rs) -------------------------------- */
int orc_estimate_linear(int format, size_t logical_in, size_t logical_out, int exl3_bits,
                        size_t* out6);
int orc_exl3_layout(size_t logical_in, size_t logical_out, int qbits, size_t* out7);

/* ---- weight packers ------------------------------------------------------ */
void orc_pack_fp8_rows(const uint16_t* w, int n, int k, uint8_t* q, float* scales);
void orc_pack_int8_rows(const uint16_t* w, int n, int k, int8_t* q, float* scales);
void orc_pack_int4_rows(const uint16_t* w, int n, int k, uint8_t* q, float* scales);
void orc_pack_int4_g128(const uint16_t* w, int n, int k, uint32_t* q, uint16_t* scales,
                        uint16_t* zeros);
void orc_pad_fp16_linear(const float* src, int logical_out, int logical_in, int padded_out,
                         int padded_in, uint16_t* dst);
void orc_q4k_encode_block(const uint16_t* src256, uint8_t* block144);
float orc_q4k_value(const uint8_t* block144, int index);
void orc_q4k_encode(const uint16_t* w, int n, int k, uint8_t* blocks);

/* ---- activation quantizers ---------------------------------------------- */
void orc_quantize_fp8_static(const uint16_t* x, size_t count, float inverse_scale,
                             uint8_t* out);
void orc_quantize_int8_static(const uint16_t* x, size_t count, float inverse_scale,
                              int8_t* out);
void orc_quantize_fp8_rows(const uint16_t* x, int rows, int valid_rows, int k, uint8_t* q,
                           float* scales);
void orc_quantize_int8_rows(const uint16_t* x, int rows, int valid_rows, int k, int8_t* q,
                            float* scales);
void orc_quantize_int4_rows(const uint16_t* x, int rows, int valid_rows, int k, uint8_t* q,
                            float* scales);
void orc_layer_norm_quantize(const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                             int rows, int valid_rows, int k, float epsilon, int int4,
                             uint8_t* q, float* scales, uint16_t* normalized);
void orc_layer_norm_pair(const uint16_t* x, const uint16_t* w1, const uint16_t* b1, const uint16_t* w2,
                         const uint16_t* b2, int rows, int valid_rows, float epsilon, float inverse_scale,
                         uint16_t* out, void* next_out);
void orc_gemm_g128_f8(const uint8_t* x, const uint32_t* q, const uint16_t* scales, const uint16_t* zeros, int m,
                      int n, int k, float* out);
void orc_compress_24(const uint8_t* x, int rows, int k, uint8_t* data, uint8_t* meta);
void orc_compress_24_i8_exact(const int8_t* x, int rows, int k, uint8_t* data, uint8_t* meta, uint32_t* counts, uint32_t* ovf);
void orc_residual_24_i8(const int8_t* x, const uint8_t* meta, int rows, int k, uint8_t* data2, uint8_t* meta2);
void orc_decompress_24(const uint8_t* data, const uint8_t* meta, int rows, int k, uint8_t* x);

/* ---- GEMM references ------------------------------------------------------ */
void orc_gemm_i8_i32(const int8_t* x, const int8_t* w, int m, int n, int k, int32_t* acc);
void orc_gemm_s4_i32(const uint8_t* x, const uint8_t* w, int m, int n, int k, int32_t* acc);
void orc_gemm_e4m3_f32(const uint8_t* x, const uint8_t* w, int m, int n, int k, float* acc);
void orc_gemm_f16_f32(const uint16_t* x, const uint16_t* w, int m, int n, int k, float* acc);
void orc_gemm_g128_a16(const uint16_t* x, const uint32_t* q, const uint16_t* scales,
                       const uint16_t* zeros, int m, int n, int k, float* out);
void orc_gemm_g128_a8(const int8_t* x, const float* x_scales, const uint32_t* q,
                      const uint16_t* scales, const uint16_t* zeros, int m, int n, int k, int parts,
                      int32_t* group_acc, float* out);
void orc_gemm_q4k_f32(const uint16_t* x, const uint8_t* blocks, int m, int n, int k, float* acc);

/* Epilogue applied to a float accumulator matrix [m x n].  See pk_oracle.c. */
void orc_epilogue(const float* acc, const float* row_scales, float in_scale,
                  const float* w_scales, const float* bias, int m, int n, int mode,
                  int valid_rows, uint16_t* out16, uint8_t* out8);
void orc_epilogue_linear(const float* acc, const float* bias, const uint16_t* residual,
                         int m, int n, float out_scale, float res_scale, int activation,
                         uint16_t* out);
void orc_epilogue_quantized(const float* acc, float in_scale, const float* w_scales,
                            const float* bias, int m, int n, int activation, uint16_t* out);

/* ---- joint ---------------------------------------------------------------- */
void orc_joint_scores_f16(const uint16_t* w, const float* bias, const uint16_t* enc,
                          const float* pred, int outputs, int hidden, float* scores);
void orc_joint_scores_i8(const int8_t* w, const float* w_scales, const float* bias,
                         const uint16_t* enc, const float* pred, int outputs, int hidden,
                         float* scores);
void orc_joint_decide(const float* scores, int token_outputs, int durations, int* token,
                      int* duration);

/* ---- threading for the CPU baseline -------------------------------------- */
int orc_threads(void);
void orc_set_threads(int threads);

/* ---- TDT decode ------------------------------------------------------------- */
void orc_lstm_step(const uint16_t* w_ih, const uint16_t* w_hh, const float* b_ih, const float* b_hh,
                   const float* x, const float* h, const float* c, int hidden, float* h_out, float* c_out);
int orc_tdt_decode(const uint16_t* enc, int frames, int enc_stride, const uint16_t* emb, const uint16_t* w_ih0,
                   const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1,
                   const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1, const uint16_t* w_proj,
                   const float* b_proj, const void* w_joint, int joint_int8, const float* joint_scales,
                   const float* b_joint, int hidden, int token_outputs, int durations, int max_symbols,
                   int32_t* tokens, int capacity, float* pred_out, int* frame_out);
float orc_det_exp(float x);
float orc_det_tanh(float v);
float orc_quantize_tensor_i8(const uint16_t* w, size_t n, int8_t* q);
void orc_lstm_long_update(const int8_t* q_hh0, const int8_t* q_hh1, const int8_t* q_ih1, const float* cq,
                          const float* bias, const uint16_t* table_row, const int8_t* qh, const float* c, int hidden,
                          int8_t* qh_out, float* c_out, float* h1_out);
int orc_tdt_decode_long(const uint16_t* enc, int frames, int enc_stride, const uint16_t* table, const uint16_t* w_hh0,
                        const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1, const uint16_t* w_hh1,
                        const float* b_ih1, const float* b_hh1, const uint16_t* w_proj, const float* b_proj,
                        const void* w_joint, int joint_int8, const float* joint_scales, const float* b_joint, int hidden,
                        int token_outputs, int durations, int max_symbols, int32_t* tokens, int capacity,
                        float* pred_out, int* frame_out);

/* ---- local relative-position attention (encoder.cu:1476-2097) ----------- */
int orc_score_vector_byte(int d);
int orc_key_int4_nibble(int d);
void orc_pack_score_vectors(const uint16_t* in, int vectors, uint8_t* out, float* scales);
void orc_pack_key_int4(const uint16_t* in, int vectors, uint8_t* out, float* scales);
void orc_quantize_value_int4(const uint16_t* vt, int rows, float inverse_scale, int edge_only, int valid_rows,
                             uint8_t* out);
void orc_local_attention(int packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                         const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output, int rows,
                         int padded_rows, int valid_rows, int left, int right, int value_stride,
                         const uint8_t* packed_key, const float* key_scales, const uint8_t* packed_position,
                         const float* position_scales, int tile_begin, int tile_end);

void orc_quantize_fp8_transpose(const uint16_t* in, int rows, float inverse_scale, uint8_t* out);
void orc_pack_position_heads(const uint16_t* in, uint16_t* out);
void orc_local_attention_short(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* pos,
                               const uint16_t* bu, const uint16_t* bv, uint16_t* out, int rows, int padded_rows,
                               int valid_rows, int left, int right);

#ifdef __cplusplus
}
#endif
#endif
