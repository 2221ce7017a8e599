// Internal launcher declarations shared by the translation units of
// libpk_linear.so.  Launchers return 0 or a negative PK_E_* status.
#pragma once

#include <stddef.h>

#include <mutex>

#include "pk_gemm.hpp"

namespace pk {

int launch_gemm(int fmt, int epi, const GemmArgs& args, hipStream_t stream);
// Tile rows the launcher picks for an m x n output (sets *cols and the
// number of LDS stages), or a negative status.
int gemm_tile_plan(int fmt, int epi, int m, int n, int* cols, int* stages);
// K split of an m x n x k launch (4: one tile per workgroup, K over its waves; else 1).
int gemm_k_split(int fmt, int epi, int m, int n, int k);
int launch_quantize_static(const void* in, void* out, float inverse_scale, size_t elements, bool int8, hipStream_t s);
int launch_quantize_rows(int kind, const void* in, void* out, float* scales, int rows, int valid_rows, int k, hipStream_t s);
// INT8 rows as 2:4 data / metadata plus per-row overflow lists (k % 128 == 0, k <= 4096),
// and, when data2 / meta2 are given, the residual 2:4 form of the positions not kept.
int launch_quantize_rows_sp24(const void* in, uint8_t* data, uint8_t* meta, float* scales, uint32_t* ovf_count, uint32_t* ovf,
                              uint8_t* data2, uint8_t* meta2, int rows, int valid_rows, int k, hipStream_t s);
int launch_pack_rows(int kind, const void* w, void* out, float* scales, int n, int k, hipStream_t s);
int launch_q4k_dequant(const uint8_t* blocks, uint16_t* out, int n, int k, hipStream_t s);
int launch_unpack_s4(const uint8_t* in, int8_t* out, size_t bytes, hipStream_t s);
int launch_unpack_s4_fp6(const uint8_t* in, uint8_t* out, size_t bytes, hipStream_t s);
int launch_expand_g128_e4m3(const uint32_t* q, const uint16_t* zeros, const uint16_t* scales, uint16_t* scales_t, uint8_t* out,
                            int n, int k, hipStream_t s);
int launch_pack_g128(const void* w, uint32_t* q, uint16_t* scales, uint16_t* zeros, int n, int k, hipStream_t s);
// mode 0: FP8, 1: INT4 nibble pairs, 2: INT4 codes as int8 bytes
int launch_layer_norm_quantize(int mode, const void* in, const void* gamma, const void* beta, void* out, float* scales,
                               void* normalized, int rows, int padded_rows, float epsilon, hipStream_t s);
int launch_layer_norm_pair(const void* in, const void* g1, const void* b1, void* out, const void* g2, const void* b2, void* next_out,
                           int rows, int padded_rows, float epsilon, float inverse_scale, hipStream_t s);
int launch_joint(const void* w, int w_int8, const float* w_scales, const float* bias, const void* enc, const float* pred,
                 float* scores, int* decision, int outputs, int hidden, int token_outputs, int durations, int steps,
                 int enc_stride, hipStream_t s);

// abort flag + 2 parities x 8 round frames x 64 workgroups of published u64 words
constexpr int kJointScanWorkspaceWords = 2304;
int launch_joint_scan(const void* w, int w_int8, const float* w_scales, const float* bias, const uint16_t* enc, const float* pred,
                      int outputs, int hidden, int token_outputs, int durations, int frames, int enc_stride, int max_symbols,
                      int* state, uint32_t* workspace, hipStream_t s);

// Device address of this device's static scan scratch (kJointScanWorkspaceWords
// words), looked up on the first call per device.
int joint_scan_scratch(uint32_t** out);

int decode_workspace_words(int hidden);
// emb set: fp16 prediction network; table set (emb unused): the long form.
int launch_tdt_decode(const uint16_t* enc, int frames, int enc_stride, const uint16_t* emb, const uint16_t* table, const uint16_t* const* w_ih,
                      const uint16_t* const* w_hh, const float* const* b_ih, const float* const* b_hh, const uint16_t* w_proj,
                      const float* b_proj, const void* w_joint, int joint_int8, const float* joint_scales, const float* b_joint,
                      int hidden, int token_outputs, int durations, int max_symbols, int32_t* tokens, int capacity, int32_t* result,
                      uint32_t* workspace, hipStream_t s);

void launch_quantize_fp8_transpose(const uint16_t* in, uint8_t* out, int rows, float inverse_scale, hipStream_t s);
void launch_pack_position_heads(const uint16_t* in, uint16_t* out, hipStream_t s);
void launch_local_attention_short(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* pos,
                                  const uint16_t* bu, const uint16_t* bv, uint16_t* out, int rows, int padded_rows,
                                  int valid_rows, int left, int right, hipStream_t s);

int launch_pack_vectors(bool int4, const uint16_t* in, uint8_t* out, float* scales, int vectors, hipStream_t s);
int launch_quantize_value_int4(const uint16_t* vt, uint8_t* out, int rows, float inverse_scale, bool edge_only, int valid_rows,
                               hipStream_t s);
int launch_local_attention(bool packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                           const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output, int rows,
                           int padded_rows, int valid_rows, int left, int right, int value_stride, const uint8_t* packed_key,
                           const float* key_scales, const uint8_t* packed_position, const float* position_scales, hipStream_t s);

int launch_sparse24_i8_contract(const uint8_t* data, const uint8_t* meta, const float* in_scales, const uint32_t* ovf_count,
                                const uint32_t* ovf, const uint8_t* data2, const uint8_t* meta2, const int8_t* w, const int8_t* wt,
                                const float* w_scales, float* out, int m, int n, int k, hipStream_t s);
int launch_transpose_i8(const int8_t* w, int8_t* wt, int n, int k, hipStream_t s);
void set_error(const char* fmt, ...);
int cu_count();
int launch_sparse24_contract(const uint8_t* data, const uint8_t* meta, const uint8_t* w, const float* w_scales, float in_scale,
                             uint16_t* out, int m, int n, int k, hipStream_t s);

}  // namespace pk
