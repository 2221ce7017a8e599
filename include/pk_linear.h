/*
 * pk_linear.h -- C ABI of libpk_linear.so, the MI355X (gfx950) quantized-weight
 * linear path of the Parakeet-TDT encoder and joint.
 *
 * Drop-in replacement for the launch surface of l4-parakeet-rs: the Rust host
 * there loads `pk_sm89_*` kernels from a cubin and launches them with cudarc's
 * positional launch_builder().arg() (src/cuda.rs:698-740,
 * src/cuda/quant_benchmark.rs:644-745, src/cuda/encoder.rs:1128-1836).  Each
 * entry point here keeps that kernel's name (prefix pk_ instead of pk_sm89_),
 * its argument order and meaning, and appends the stream.  Shape constants the
 * reference bakes into a kernel (1024 -> 4096 etc.) stay baked into the entry
 * point of the same name; the pk_gemm_* entries take explicit shapes.
 *
 * Conventions:
 *   - All pointers are device pointers unless stated; fp16 data is passed as
 *     uint16_t bits; weights are [N x K] row-major (weight_oi, linear.cu:75-77).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Calls only
 *     enqueue work; nothing synchronises and nothing allocates device memory.
 *   - Return 0 on success or a negative PK_E_* code; pk_last_error() returns a
 *     thread-local message for the last failure on the calling thread.
 *   - Shapes: K must be a multiple of the format's K-step (128 for FP8/INT8,
 *     256 for packed INT4, 64 for FP16) and N a multiple of 16; M is free
 *     (the reference pads M to 16, N to 128 and K to 128, which satisfies
 *     this).  Operand base pointers must be 16-byte aligned.
 *   - Every GEMM entry point (pk_gemm, the pk_linear_* linears and the encoder
 *     wrappers) also needs 16-byte aligned bias, weight-scale and residual
 *     pointers: the epilogue reads them as 16-byte vectors, so a slice at a
 *     4-byte offset returns PK_E_ALIGN (copy it to an aligned buffer first).
 *   - Results do not depend on M or on the GPU's CU count, with one stated
 *     exception: INT4-g128 launches on small grids that split K in four
 *     parts within a workgroup (pk_gemm_k_split reports 4) fold the group sums
 *     by parts, so their fp32 results are associated differently from the
 *     same rows' on a large grid (each part is exact; see pk_gemm_k_split).
 */
#ifndef PK_LINEAR_H
#define PK_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_OK 0
#define PK_E_SHAPE (-1)
#define PK_E_ALIGN (-2)
#define PK_E_LAUNCH (-3)
#define PK_E_ARG (-4)
#define PK_E_FORMAT (-5) /* invalid .pkl4 artifact */
#define PK_E_IO (-6)     /* artifact file could not be read */

const char* pk_last_error(void);
/* Version of this ABI (bumped on any signature change). */
int32_t pk_abi_version(void);

/* ---- size contracts (host only, no GPU) ---------------------------------- */

/* packing.rs:71-130 (estimate_linear).  format: 0 fp16, 1 fp8 e4m3, 2 int8,
 * 3 GGML Q4_K, 4 EXL3-derived.  out6 = {logical_in, logical_out, padded_in,
 * padded_out, payload_bytes, metadata_bytes}.  Returns 1 when a layout exists,
 * 0 for Q4_K with K % 256 != 0 (the reference's None), PK_E_SHAPE for empty
 * dimensions, PK_E_ARG for an unknown format or bit rate. */
int32_t pk_estimate_linear(int32_t format, size_t logical_in, size_t logical_out, int32_t exl3_bits,
                           size_t* out6);
/* exl3.rs:37-75 (Exl3Layout).  out7 = {padded_in, padded_out, trellis_shape[3],
 * trellis_bytes, scale_bytes}.  Returns 0, PK_E_SHAPE or PK_E_ARG. */
int32_t pk_exl3_layout(size_t logical_in, size_t logical_out, int32_t qbits, size_t* out7);

/* ---- .pkl4 artifact and load-time derivation (host code) -------------------
 * artifact.rs:11-157 (AotArtifactIndex::open) with the checks of
 * artifact.rs:514-650: prefix "PKL4AOT\0", schema 2, flags 0, JSON header,
 * payload at the first 4096-byte boundary, 256-byte aligned tensors, linear
 * weights as fp16 [ceil128(N) x ceil128(K)] and their biases as fp32
 * [ceil128(N)] zero padded.  Invalid files return PK_E_FORMAT with the
 * reference's message in pk_last_error(). */

typedef struct pk_artifact pk_artifact;

#define PK_STORAGE_FP16 0        /* AotStorage::Fp16 */
#define PK_STORAGE_FP32 1        /* AotStorage::Fp32 */
#define PK_STORAGE_FP16_LINEAR 2 /* AotStorage::Sm89Fp16Linear */
#define PK_STORAGE_FP32_BIAS 3   /* AotStorage::Sm89Fp32Bias */

typedef struct {
    const char* name;          /* owned by the artifact */
    int32_t storage;           /* PK_STORAGE_* */
    int32_t rank;
    uint64_t logical_shape[4];
    uint64_t physical_shape[4];
    uint64_t offset;           /* payload offset */
    uint64_t bytes;
} pk_tensor_info;

typedef struct {
    int32_t profile;           /* 0 v2-english, 1 v3-multilingual (config.rs:14-17) */
    int32_t blank_token_id;    /* 1024 or 8192 */
    int32_t tensor_count;
    int32_t vocabulary_size;
    uint64_t data_start;       /* file offset of the payload */
    uint64_t payload_bytes;
    uint64_t file_bytes;
} pk_artifact_summary;

/* Opens and validates an artifact; *out is NULL on failure. */
int32_t pk_artifact_open(const char* path, pk_artifact** out);
void pk_artifact_close(pk_artifact* artifact);
int32_t pk_artifact_info(const pk_artifact* artifact, pk_artifact_summary* out);
/* Tensor `index` (header order). */
int32_t pk_artifact_tensor(const pk_artifact* artifact, int32_t index, pk_tensor_info* out);
/* Index of the tensor called `name`, or PK_E_ARG (artifact.rs:160-167's missing tensor). */
int32_t pk_artifact_find(const pk_artifact* artifact, const char* name);
/* Vocabulary piece `index` (< blank_token_id), or NULL. */
const char* pk_artifact_vocabulary(const pk_artifact* artifact, int32_t index);
/* Copies tensor `index`'s stored bytes into host memory (capacity >= bytes). */
int32_t pk_artifact_read(const pk_artifact* artifact, int32_t index, void* host_dst, uint64_t capacity);

#define PK_DERIVE_FP16 0      /* upload only */
#define PK_DERIVE_FP8_ROWS 1  /* pk_pack_fp8_rows: packed u8 [N x K], fp32 scales [N] */
#define PK_DERIVE_INT8_ROWS 2 /* pk_pack_int8_rows: packed s8 [N x K], fp32 scales [N] */
#define PK_DERIVE_INT4_ROWS 3 /* pk_pack_int4_rows: packed [N x K/2], fp32 scales [N] */
#define PK_DERIVE_INT4_G128 4 /* pk_pack_int4_g128: u32 [N x K/8], fp16 scales and zeros [N x K/128] */

/* Load-time derivation of one sm89_fp16_linear tensor (the job of
 * QuantizedFfnWeights::load_for, encoder.rs:361-422, and of upload_aot,
 * cuda.rs:375-412, for one tensor): reads its padded fp16 [N x K] (physical
 * shape) into host_staging (staging_bytes >= its bytes; pinned memory makes the
 * copy asynchronous), uploads it to device_fp16 on `stream` and packs it on the
 * GPU into `format` (packed / scales / zeros as the packer it names; zeros only
 * for PK_DERIVE_INT4_G128).  All-zero padding rows pack with scale 1.  The
 * staging buffer must stay untouched until the stream has run the upload. */
int32_t pk_artifact_derive_linear(const pk_artifact* artifact, int32_t index, int32_t format, void* host_staging,
                                  uint64_t staging_bytes, uint16_t* device_fp16, void* packed, void* scales,
                                  uint16_t* zeros, void* stream);

/* ---- load-time weight packers (fp16 [n x k] -> packed) -------------------- */

/* encoder.rs:361-422 FP8 branch / quant_benchmark.rs:779-801: per-row
 * scale = max|w| / 448 (1 for an all-zero row), q = e4m3(w / scale). */
int32_t pk_pack_fp8_rows(const uint16_t* weight, int32_t n, int32_t k, uint8_t* packed, float* scales,
                         void* stream);
/* quant_benchmark.rs:803-829: per-row scale = max|w| / 127, q = rne clamp +-127. */
int32_t pk_pack_int8_rows(const uint16_t* weight, int32_t n, int32_t k, int8_t* packed, float* scales,
                          void* stream);
/* encoder.rs:378-407 INT4 branch: scale = max(max(w/7, -w/8)), q in [-8, 7],
 * byte j = q[2j] & 15 | q[2j+1] << 4; packed is [n x k/2]. */
int32_t pk_pack_int4_rows(const uint16_t* weight, int32_t n, int32_t k, uint8_t* packed, float* scales,
                          void* stream);
/* No reference counterpart: group-wise asymmetric INT4,
 * 128-K groups, q packed 8 per uint32 ([n x k/8]), fp16 scales and integer
 * fp16 zero-points ([n x k/128]); dequant (q - z) * s. */
int32_t pk_pack_int4_g128(const uint16_t* weight, int32_t n, int32_t k, uint32_t* packed,
                          uint16_t* scales, uint16_t* zeros, void* stream);
/* No reference counterpart: INT4-g128 weights (pk_pack_int4_g128 layout,
 * zeros [n x k/128]) as e4m3 (q - z) bytes [n x k] in k order, exact since
 * |q - z| <= 15, and their fp16 scales moved to group-major order
 * (scales_t [k/128 x n]); the weight and g_scales operands of pk_gemm format 8
 * (e4m3 activations x INT4-g128 weights), expanded per call into caller
 * buffers.  packed and expanded 16-byte aligned. */
int32_t pk_expand_int4_g128_e4m3(const uint32_t* packed, const uint16_t* zeros, const uint16_t* scales, int32_t n,
                                 int32_t k, uint8_t* expanded, uint16_t* scales_t, void* stream);
/* linear.cu:459-472 pk_sm89_q4_k_dequantize: GGUF Q4_K superblocks (144 bytes
 * per 256 values: fp16 d, fp16 dmin, 12 bytes of 6-bit scales/mins, 128 quant
 * bytes) [n x k/256] -> fp16 [n x k], value = f16(d*sc*q - dmin*mn). */
int32_t pk_q4_k_dequantize(const uint8_t* input, uint16_t* output, int32_t n, int32_t k, void* stream);

/* ---- activation quantizers ------------------------------------------------ */

/* linear.cu:537-547 pk_sm89_quantize_fp8: out = e4m3(in * inverse_scale). */
int32_t pk_quantize_fp8(const uint16_t* input, uint8_t* output, float inverse_scale, int32_t elements,
                        void* stream);
/* linear.cu:549-560 pk_sm89_quantize_int8: rne(clamp(in * inverse_scale, +-127)). */
int32_t pk_quantize_int8(const uint16_t* input, int8_t* output, float inverse_scale, int32_t elements,
                         void* stream);
/* encoder.cu:549-559 pk_sm89_quantize_fp8_fixed (note the argument order). */
int32_t pk_quantize_fp8_fixed(const uint16_t* input, uint8_t* output, int32_t elements, float inverse_scale,
                              void* stream);
/* encoder.cu:1129-1146 pk_sm89_quantize_rows1024: per-row FP8, rows of 1024. */
int32_t pk_quantize_rows1024(const uint16_t* input, uint8_t* output, float* scales, int32_t rows, void* stream);
/* encoder.cu:1148-1157 pk_sm89_quantize_rows256: per-row FP8, rows of 256. */
int32_t pk_quantize_rows256(const uint16_t* input, uint8_t* output, float* scales, int32_t rows, void* stream);
/* encoder.cu:1159-1180 pk_sm89_quantize_ffn_contract: per-row FP8 of the
 * [1024 x 4096] FF contract weight (grid = 1024 rows in the reference). */
int32_t pk_quantize_ffn_contract(const uint16_t* input, uint8_t* output, float* scales, void* stream);
/* Generalised dynamic per-row quantizers over fp16 [rows x k]; rows >=
 * valid_rows are written as zeros with scale 1.  kind: 0 FP8 (max/448),
 * 1 INT8 (max/127, per-token dynamic INT8), 2 INT4 (max(x/7, -x/8), [rows x k/2]). */
int32_t pk_quantize_rows(int32_t kind, const uint16_t* input, void* output, float* scales, int32_t rows,
                         int32_t valid_rows, int32_t k, void* stream);
/* encoder.cu:211-306 pk_sm89_layer_norm_quantize_{fp8,int4}_dynamic: LayerNorm
 * over 1024 features, fp16 rounding, per-row dynamic FP8 / INT4 (+ scales);
 * rows in [rows, padded_rows) are zero with scale 1.  input, weight and bias
 * 8-byte aligned, output 4-byte (FP8) / 2-byte (INT4) aligned (PK_E_ALIGN). */
int32_t pk_layer_norm_quantize_fp8_dynamic(const uint16_t* input, const uint16_t* weight, const uint16_t* bias,
                                           uint8_t* output, float* scales, int32_t rows, int32_t padded_rows,
                                           float epsilon, void* stream);
int32_t pk_layer_norm_quantize_int4_dynamic(const uint16_t* input, const uint16_t* weight, const uint16_t* bias,
                                            uint8_t* output, float* scales, int32_t rows, int32_t padded_rows,
                                            float epsilon, void* stream);

/* encoder.cu:128-209 pk_sm89_layer_norm_pair (launched at encoder.rs:1394-1433):
 * output = fp16(LN(input; weight, bias)) [padded_rows x 1024], then
 * LN(output; next_weight, next_bias) into next_output, as fp16 when
 * inverse_scale == 0, else as e4m3(fp16 value * inverse_scale) bytes (the
 * reference passes 56 = 448 / 8 for an FP8 next FF1).  Rows in [rows,
 * padded_rows) are zero in both outputs.  fp16 pointers 8-byte aligned,
 * next_output 4-byte (e4m3) / 8-byte (fp16) aligned (PK_E_ALIGN). */
int32_t pk_layer_norm_pair(const uint16_t* input, const uint16_t* weight, const uint16_t* bias, uint16_t* output,
                           const uint16_t* next_weight, const uint16_t* next_bias, void* next_output, int32_t rows,
                           int32_t padded_rows, float epsilon, float inverse_scale, void* stream);

/* The LayerNorm + dynamic INT4 producer above (same scales, same codes) with
 * the codes written as int8 bytes [padded_rows x 1024] instead of nibble
 * pairs: the operand form the INT8 MFMA reads (CDNA4 has no 4-bit integer
 * MFMA), consumed by pk_ffn_expand_int4_sparse_codes.  output 4-byte aligned. */
int32_t pk_layer_norm_quantize_int4_codes(const uint16_t* input, const uint16_t* weight, const uint16_t* bias,
                                          int8_t* output, float* scales, int32_t rows, int32_t padded_rows,
                                          float epsilon, void* stream);
/* No reference counterpart: the same producer (same scales, same codes) with
 * the codes written in the FP6 e3m2 chunk form: 16 codes a 16-byte chunk, code
 * j of the chunk in bits 6j..6j+5 of its first 12 bytes (little-endian), then
 * 4 zero bytes; e3m2 holds every code in -8..7 exactly.  [padded_rows x 1024]
 * bytes, the operand pk_ffn_expand_int4_sparse_fp6 reads on the f8f6f4 MFMA,
 * which multiplies FP6 at twice the FP8 / INT8 rate.  output 4-byte aligned. */
int32_t pk_layer_norm_quantize_int4_fp6(const uint16_t* input, const uint16_t* weight, const uint16_t* bias,
                                        uint8_t* output, float* scales, int32_t rows, int32_t padded_rows,
                                        float epsilon, void* stream);
/* No reference counterpart: nibble pairs (as pk_unpack_int4 reads them) -> the
 * FP6 e3m2 chunk form above, `elements` codes (a multiple of 32) into as many
 * bytes; both pointers 16-byte aligned.  The load-time derivation of the
 * per-row INT4 FF2 weights' FP6 operand form. */
int32_t pk_unpack_int4_fp6(const uint8_t* packed, uint8_t* codes, int64_t elements, void* stream);
/* Nibble pairs (byte j = q[2j] & 15 | q[2j+1] << 4, the encoder.rs:405 order of
 * pk_pack_int4_rows and of the INT4 producer) -> sign-extended int8 codes,
 * `elements` codes (a multiple of 32); both pointers 16-byte aligned.  The
 * load-time derivation of the per-row INT4 FF2 weights' operand form. */
int32_t pk_unpack_int4(const uint8_t* packed, int8_t* codes, int64_t elements, void* stream);

/* ---- linears (linear.cu) ---------------------------------------------------- */

/* linear.cu:83-171 pk_sm89_fp16_linear_epilogue (+ the _m64 variant and the
 * cuBLAS GemmEx fallback, cublas.rs:67-113): Y = act((X W^T + b) * out_scale
 * + res_scale * R), fp16 in/out, fp32 accumulate.  bias / residual may be NULL;
 * act 0 none, 1 SiLU, 2 ReLU. */
int32_t pk_linear_fp16_epilogue(const uint16_t* input, const uint16_t* weight_oi, const float* bias,
                                const uint16_t* residual, uint16_t* output, int32_t m, int32_t n, int32_t k,
                                float output_scale, float residual_scale, int32_t activation, void* stream);
/* linear.cu:176-239 pk_sm89_fp16_qkv: three projections into Q|K|V, each
 * [m x n] contiguous in `output`. */
int32_t pk_linear_fp16_qkv(const uint16_t* input, const uint16_t* query_weight, const uint16_t* key_weight,
                           const uint16_t* value_weight, uint16_t* output, int32_t m, int32_t n, int32_t k,
                           void* stream);
/* linear.cu:325-374 pk_sm89_fp8_linear_epilogue: Y = act(fma(sum e4m3*e4m3,
 * in_scale * w_scale[n], bias[n])) -> fp16.  bias may be NULL. */
int32_t pk_linear_fp8_epilogue(const uint8_t* input, const uint8_t* weight_oi, const float* weight_scales,
                               const float* bias, uint16_t* output, int32_t m, int32_t n, int32_t k,
                               float input_scale, int32_t activation, void* stream);
/* linear.cu:378-429 pk_sm89_int8_linear_epilogue: exact int32 accumulation,
 * then the same epilogue as the FP8 linear. */
int32_t pk_linear_int8_epilogue(const int8_t* input, const int8_t* weight_oi, const float* weight_scales,
                                const float* bias, uint16_t* output, int32_t m, int32_t n, int32_t k,
                                float input_scale, int32_t activation, void* stream);
/* The exact INT8 x INT8 -> INT32 accumulators of pk_linear_int8_epilogue
 * ([m x n] int32), the bit-exact parity instrument of
 * quant_benchmark.rs:872-909. */
int32_t pk_linear_int8_accumulate(const int8_t* input, const int8_t* weight_oi, int32_t* accumulators,
                                  int32_t m, int32_t n, int32_t k, void* stream);
/* Per-token dynamic INT8 activations (scales [m]) x per-channel INT8 weights:
 * Y = (acc * input_scales[row]) * weight_scales[n] (+ bias) -> fp16 or fp32. */
int32_t pk_linear_int8_dyn(const int8_t* input, const float* input_scales, const int8_t* weight_oi,
                           const float* weight_scales, const float* bias, void* output, int32_t output_fp32,
                           int32_t m, int32_t n, int32_t k, void* stream);
/* Per-row FP8 with dynamic per-row activation scales (the ffn_fp8_async
 * dynamic_scale path, encoder.cu:972-995), fp16 or fp32 output. */
int32_t pk_linear_fp8_dyn(const uint8_t* input, const float* input_scales, const uint8_t* weight_oi,
                          const float* weight_scales, const float* bias, void* output, int32_t output_fp32,
                          int32_t m, int32_t n, int32_t k, void* stream);
/* s4 x s4 -> exact int32 (the mma...s4.s4 path of encoder.cu:211-292): both
 * operands packed two per byte ([m x k/2], [n x k/2]). */
int32_t pk_linear_int4_accumulate(const uint8_t* input, const uint8_t* weight_oi, int32_t* accumulators,
                                  int32_t m, int32_t n, int32_t k, void* stream);
/* No reference counterpart.  fp16 activations x
 * group-wise INT4 weights (pk_pack_int4_g128 layout), weights dequantized to
 * fp16 in registers, fp32 accumulate; bias may be NULL; fp16 or fp32 output. */
int32_t pk_linear_int4g128(const uint16_t* input, const uint32_t* weight_q, const uint16_t* weight_scales,
                           const uint16_t* weight_zeros, const float* bias, void* output, int32_t output_fp32,
                           int32_t m, int32_t n, int32_t k, void* stream);
/* linear.cu:478-535 pk_sm89_q4_k_linear_epilogue: fp16 input [m x k] x Q4_K
 * weights [n x k/256 blocks] dequantized to fp16 in registers, fp32
 * accumulate, out = f16(act(acc + bias[n])); bias may be NULL; k % 256 == 0. */
int32_t pk_q4_k_linear_epilogue(const uint16_t* input, const uint8_t* weight_oi, const float* bias, uint16_t* output,
                                int32_t m, int32_t n, int32_t k, int32_t activation, void* stream);
/* Mixed variant: per-token dynamic INT8 activations x group-wise INT4 weights
 * on the INT8 MFMA; each 128-K group's int32 sum (exact) is scaled by its fp16
 * scale in fp32, then by the row scale. */
int32_t pk_linear_int4g128_a8(const int8_t* input, const float* input_scales, const uint32_t* weight_q,
                              const uint16_t* weight_scales, const uint16_t* weight_zeros, const float* bias,
                              void* output, int32_t output_fp32, int32_t m, int32_t n, int32_t k, void* stream);

/* ---- encoder FastConformer linears (encoder.cu ffn_fp8_async wrappers) --------
 * `rows` is the (padded) frame count; per-row fp32 scales come from the
 * quantizers above.  Widths are those of the reference kernels. */

/* encoder.cu:1063-1069 pk_sm89_ffn_expand_fp8_async: FF1 1024 -> 4096,
 * SiLU -> fp16 [rows x 4096].  dynamic_scale != 0 uses input_scales[row],
 * else input_scale. */
int32_t pk_ffn_expand_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                          const float* input_scales, uint16_t* output, int32_t rows, float input_scale,
                          int32_t dynamic_scale, void* stream);
/* encoder.cu:1071-1077 pk_sm89_ffn_expand_fp8_packed: as above, output
 * e4m3(fp16(SiLU) * 16) bytes [rows x 4096]. */
int32_t pk_ffn_expand_fp8_packed(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                 const float* input_scales, uint8_t* output, int32_t rows, float input_scale,
                                 int32_t dynamic_scale, void* stream);
/* encoder.cu:1079-1085 pk_sm89_ffn_expand_int4_sparse: s4 activations
 * [rows x 512 bytes] x s4 weights [4096 x 512 bytes], exact int32, then
 * SiLU -> fp16 -> x16 -> e4m3, 2:4 compressed: `output` receives
 * [rows x 2048] data bytes followed by [rows x 512] metadata bytes. */
int32_t pk_ffn_expand_int4_sparse(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                  const float* input_scales, uint8_t* output, int32_t rows, float input_scale,
                                  int32_t dynamic_scale, void* stream);
/* pk_ffn_expand_int4_sparse on the operand form of the same INT4 values: int8
 * codes [rows x 1024] (pk_layer_norm_quantize_int4_codes) x int8 codes [4096 x
 * 1024] (pk_unpack_int4 of the per-row INT4 weights), on the INT8 MFMA with no
 * nibble decode in the K-loop.  Same exact int32 accumulators, so the output
 * (data + metadata, same layout) is identical to pk_ffn_expand_int4_sparse's. */
int32_t pk_ffn_expand_int4_sparse_codes(const int8_t* input, const int8_t* weight, const float* weight_scales,
                                        const float* input_scales, uint8_t* output, int32_t rows, float input_scale,
                                        int32_t dynamic, void* stream);
/* pk_ffn_expand_int4_sparse on the FP6 form of the same INT4 values: FP6 chunk
 * codes [rows x 1024] (pk_layer_norm_quantize_int4_fp6) x FP6 chunk codes
 * [4096 x 1024] (pk_unpack_int4_fp6 of the per-row INT4 weights), on the
 * f8f6f4 MFMA at the FP6 rate.  Products of codes are exact in FP6 x FP6 and
 * the fp32 sums of K = 1024 of them (|sum| <= 2^16) are exact, so the output
 * (data + metadata, same layout) is identical to pk_ffn_expand_int4_sparse's. */
int32_t pk_ffn_expand_int4_sparse_fp6(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                      const float* input_scales, uint8_t* output, int32_t rows, float input_scale,
                                      int32_t dynamic, void* stream);
/* encoder.cu:1095-1103 pk_sm89_ffn_contract_fp8: FF contract 4096 -> 1024 on
 * FP8 input at scale 1/16; output (fp16 [rows x 1024]) += 0.5 * Y in place. */
int32_t pk_ffn_contract_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                            uint16_t* output, int32_t rows, void* stream);
/* encoder.cu:1087-1093 pk_sm89_ffn_contract_fp8_sparse: FF2 contract on 2:4
 * compressed FP8 activations on the sparse MFMA (v_smfmac_f32_16x16x128_fp8_fp8).
 * `input` holds [rows x inner_width/2] data bytes followed by [rows x
 * inner_width/8] metadata bytes (the layout pk_ffn_expand_int4_sparse writes);
 * weight FP8 [1024 x inner_width]; output (fp16 [rows x 1024]) += 0.5 * Y at
 * input scale 1/16.  The metadata block must be 16-byte aligned. */
int32_t pk_ffn_contract_fp8_sparse(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                   uint16_t* output, int32_t rows, int32_t inner_width, void* stream);
/* encoder.cu:1313-1319 pk_sm89_conv_residual_fp8: pointwise2 1024 -> 1024,
 * dynamic per-row input scales, output += Y in place. */
int32_t pk_conv_residual_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                             const float* input_scales, uint16_t* output, int32_t rows, void* stream);
/* encoder.cu:2099-2107 pk_sm89_attention_output_fp8: o_proj 1024 -> 1024,
 * input scale 1/28, output += Y in place. */
int32_t pk_attention_output_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                uint16_t* output, int32_t rows, void* stream);

/* encoder.cu:1121-1127 pk_sm89_conv_glu_fp8: pointwise1 1024 -> 2048 (weight
 * [2048 x 1024] natural row order, scales [2048]) with dynamic per-row input
 * scales, then GLU: out[r, c] = fp16(v) / (1 + exp(-fp16(g))) with v, g the
 * scaled fp16-rounded outputs c and c + 1024; rows >= valid_rows are written
 * as 0.  output is fp16 [rows x 1024]. */
int32_t pk_conv_glu_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                        const float* input_scales, uint16_t* output, int32_t rows, int32_t valid_rows, void* stream);
/* encoder.cu:1105-1111 pk_sm89_subsample_projection_fp8: 4096 -> 1024 + bias,
 * dynamic per-row input scales, fp16 out (subsampling.rs:436-806 caller). */
int32_t pk_subsample_projection_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                    const float* input_scales, const float* bias, uint16_t* output, int32_t rows,
                                    void* stream);
/* encoder.cu:1113-1119 pk_sm89_subsample_pointwise_fp8: 256 -> 256 + bias, ReLU. */
int32_t pk_subsample_pointwise_fp8(const uint8_t* input, const uint8_t* weight, const float* weight_scales,
                                   const float* input_scales, const float* bias, uint16_t* output, int32_t rows,
                                   void* stream);

/* Activation-sparse FF2 contract (the reference's sparse
 * FF2 is the 2:4 path, encoder.cu:1087-1095): INT8 activations [rows x 4096]
 * with per-row scales (zeros where the frame's activations were dropped) x
 * per-row INT8 weights [1024 x 4096] -> fp32 [rows x 1024],
 * out = (acc * input_scale[r]) * weight_scale[n].  Every 16-row x 128-K
 * activation block whose bytes are all zero skips its MFMAs (wave ballot),
 * which is exact.  skip_counts (device uint32[2], may be NULL) accumulates
 * {skipped blocks, total blocks}; the caller clears it. */
int32_t pk_ffn_contract_int8_rowskip(const int8_t* input, const float* input_scales, const int8_t* weight,
                                     const float* weight_scales, float* output, int32_t rows, uint32_t* skip_counts,
                                     void* stream);

/* Exact 2:4 form of the activation-sparse FF2.  The
 * reference's sparse FF2 (encoder.cu:685-704 selection, :1037-1095 contract)
 * keeps the two largest magnitudes of every quartet and drops the rest; here
 * the dropped nonzeros are kept in a per-row overflow list, so the contract
 * is exact.
 *
 * pk_quantize_rows_int8_sparse24: the INT8 per-row dynamic quantization of
 * pk_quantize_rows kind 1 (same scales and bytes), written as 2:4 data
 * [rows x k/2] and metadata [rows x k/8] (quartet p: idx0 | idx1 << 2 at bits
 * 4 (p % 2) of byte p / 2, the reference's layout) plus, per row,
 * overflow_counts[row] entries at overflow[row * k/2 ...], each
 * (element << 8) | int8 byte, in ascending element order (at most k/2).
 * residual_data [rows x k/2] / residual_meta [rows x k/8] (both or neither,
 * no counterpart in the reference): the residual 2:4 form, per quartet the
 * two positions the selection did not keep, ascending, with their bytes, in
 * the layout of data / meta.  k % 128 == 0, k <= 4096; input 16-byte
 * aligned, data / residual_data / overflow / overflow_counts 4-byte aligned.
 * Rows >= valid_rows are zero, scale 1.  Other k are for other consumers:
 * pk_ffn_contract_int8_sparse24 reads only k = 4096 buffers. */
int32_t pk_quantize_rows_int8_sparse24(const uint16_t* input, uint8_t* data, uint8_t* meta, float* scales,
                                       uint32_t* overflow_counts, uint32_t* overflow, uint8_t* residual_data,
                                       uint8_t* residual_meta, int32_t rows, int32_t valid_rows, int32_t k, void* stream);
/* Load-time derivation: weight_t [k x n] = transpose of the INT8 weight [n x k]
 * (the overflow pass of the contract below reads weight columns). */
int32_t pk_transpose_int8(const int8_t* weight, int8_t* weight_t, int32_t n, int32_t k, void* stream);
/* The FF2 contract 4096 -> 1024 on that form: fp32 output [rows x 1024] equal
 * bit for bit to pk_ffn_contract_int8_rowskip's on the dense INT8 rows,
 * out = (acc * input_scale[r]) * weight_scale[n].  With residual_data /
 * residual_meta (both or neither, from the quantizer above), row tiles
 * whose rows hold more than 8 overflow entries each on average add the
 * residual 2:4 form in a second sparse pass instead of walking the lists.
 * data, meta, residual data / meta, weight, weight_t, weight_scales and
 * output 16-byte aligned.  The contract is the FF2 shape only (n = 1024,
 * k = 4096): data / metadata / overflow / residual buffers must come from
 * pk_quantize_rows_int8_sparse24 with k = 4096. */
int32_t pk_ffn_contract_int8_sparse24(const uint8_t* data, const uint8_t* meta, const float* input_scales,
                                      const uint32_t* overflow_counts, const uint32_t* overflow, const uint8_t* residual_data,
                                      const uint8_t* residual_meta, const int8_t* weight, const int8_t* weight_t,
                                      const float* weight_scales, float* output, int32_t rows, void* stream);

/* ---- generic fused GEMM ------------------------------------------------------
 * format: 0 FP8, 1 INT8, 2 INT4 (s4 x s4), 3 INT4-g128 x INT8, 4 FP16,
 * 5 INT4-g128 x FP16, 6 INT8 with zero-block skip, 7 Q4_K x FP16 (epilogues
 * 0 and 3 only), 8 e4m3 activations x INT4-g128 weights given as e4m3 (q - z)
 * bytes (b from pk_expand_int4_g128_e4m3; g_scales required, group-major
 * [k/128 x n] as that call writes them, 16-byte aligned; g_zeros unused;
 * each 128-K group summed in fp32 by one MFMA, then folded in K order with
 * one fma by its fp16 scale; epilogues 0, 1 and 3), 9 INT4 codes as FP6 e3m2
 * chunks on both operands (pk_layer_norm_quantize_int4_fp6 /
 * pk_unpack_int4_fp6; k a multiple of 128; f8f6f4 MFMA, exact integer sums in
 * fp32; epilogues 2 and 3).  epilogue: 0 fp16 (act(v [+bias]) * out_scale
 * [+ res_scale * residual]), 1 e4m3(fp16(SiLU(v)) * 16), 2 as 1 + 2:4
 * compression (metadata to out_meta), 3 fp32 v [+bias], 4 raw int32.
 * v = acc * row_scale * w_scale with row_scale = row_scales[r] or in_scale. */
int32_t pk_gemm(int32_t format, int32_t epilogue, const void* a, const void* b, int32_t m, int32_t n, int32_t k,
                const float* w_scales, const float* row_scales, float in_scale, const float* bias,
                const uint16_t* residual, float out_scale, float res_scale, int32_t activation,
                const uint16_t* g_scales, const uint16_t* g_zeros, void* out, uint8_t* out_meta, int32_t ldo,
                void* stream);

/* Tile shape pk_gemm launches for an m x n output of `format` / `epilogue`
 * (host only, no GPU work): returns the tile rows (32, 64, 128 or 256) and
 * sets *tile_cols (128, or 256 for the one-workgroup 256 x 256 engine) and
 * *stages (2 for the double-buffered engines; more for the one-tile-per-
 * workgroup ring used when the tiles do not outnumber the CUs), or returns a
 * negative PK_E_* status.  Either pointer may be NULL.  No counterpart in the
 * reference (its kernels have one tile shape); it lets callers and tests see
 * which kernel variant a shape runs. */
int32_t pk_gemm_tile(int32_t format, int32_t epilogue, int32_t m, int32_t n, int32_t* tile_cols, int32_t* stages);
/* K split of pk_gemm's launch for an m x n x k output (host only): 4 when each
 * 32-row tile's K-steps are divided in four K-ordered parts within its
 * workgroup (16 waves, each part's LDS ring shared by four of them) and the
 * partial tiles summed in K order (INT4-g128 formats on grids that take
 * 32-row tiles, k >= 1024; *stages of pk_gemm_tile is the plain ring's), else
 * 1; or a negative PK_E_* status.
 * No counterpart in the reference. */
int32_t pk_gemm_k_split(int32_t format, int32_t epilogue, int32_t m, int32_t n, int32_t k);

/* ---- TDT joint (decoder.cu:690-759) ------------------------------------------ */

/* Batch-1 joint GEMV for `steps` consecutive frames:
 *   score[o] = bias[o] + w_scale[o] * sum_k W[o,k] * relu(enc[t,k] + pred[k])
 * for o < outputs, then decision[2t] = argmax over the first token_outputs
 * scores (ties to the lower id) and decision[2t+1] = the duration argmax over
 * the next `durations` scores (first maximum wins).  weight is fp16
 * (weight_int8 = 0, w_scales ignored, may be NULL) or int8 with per-row fp32
 * scales.  enc is fp16 [steps x enc_stride], pred fp32 [hidden]; scores
 * (optional, fp32 [steps x outputs]) and decision (int32 [steps x 2]). */
int32_t pk_joint_gemv(const void* weight, int32_t weight_int8, const float* w_scales, const float* bias,
                      const uint16_t* enc, const float* pred, float* scores, int32_t* decision,
                      int32_t outputs, int32_t hidden, int32_t token_outputs, int32_t durations,
                      int32_t steps, int32_t enc_stride, void* stream);

/* The greedy TDT loop's joint steps between two emitted tokens
 * (decoder.cu:690-783 with the prediction vector fixed), in one persistent
 * launch: from frame state[0] with state[1] symbols already added at it,
 * repeat { scores of frame t; token / duration decision as pk_joint_gemv;
 * symbols += 1; t += duration; if duration != 0 or symbols == max_symbols
 * { if duration == 0, t += 1; symbols = 0 } } until a token other than the
 * blank (id token_outputs - 1) is chosen or t >= frames.  state (device
 * int32[4]) returns {t, symbols, token or -1 when the frames ran out, joint
 * steps run}; state[2] = -2 if the workgroups failed to meet at a barrier
 * (not co-resident).  The weights stay in registers for the whole scan:
 * hidden % 128 == 0, hidden <= 1024, durations <= 8, token_outputs +
 * durations <= 2048.  workspace is a device uint32[2304] the call overwrites
 * (the decision words the workgroups exchange: per round of 8 frames one
 * word per workgroup and frame, two rounds' worth). */
int32_t pk_joint_scan(const void* weight, int32_t weight_int8, const float* w_scales, const float* bias,
                      const uint16_t* enc, const float* pred, int32_t outputs, int32_t hidden,
                      int32_t token_outputs, int32_t durations, int32_t frames, int32_t enc_stride,
                      int32_t max_symbols, int32_t* state, uint32_t* workspace, void* stream);

/* pk_joint_scan without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * 2304 words (9 KiB) of scratch are a static device array of the library (one copy
 * per GPU, held until the process ends; its address is looked up once per
 * device), cleared by a fill kernel at the start of every call.  Same
 * arguments, limits and results as pk_joint_scan; token_outputs + durations
 * above 2048 return PK_E_SHAPE.  Calls on one GPU share the scratch: calls
 * on one stream are ordered and independent, calls that overlap on one GPU
 * (different streams) race.  Allocates nothing. */
int32_t pk_joint_scan_noalloc(const void* weight, int32_t weight_int8, const float* w_scales, const float* bias,
                              const uint16_t* enc, const float* pred, int32_t outputs, int32_t hidden,
                              int32_t token_outputs, int32_t durations, int32_t frames, int32_t enc_stride,
                              int32_t max_symbols, int32_t* state, void* stream);

/* ---- TDT greedy decode (decoder.cu:146-445, fp16 prediction network) --------
 * The whole batch-1 greedy decode of one utterance in one persistent launch:
 * 2-layer LSTM prediction network (weights [4H x H] fp16 with gate rows
 * i, f, g, o; fp32 biases [4H]) on the last emitted token's embedding (zeros
 * before the first token), projection [H x H] fp16 + fp32 bias, joint as
 * pk_joint_gemv (fp16 weights, or INT8 with per-row scales), token / duration
 * decision and the frame / symbol rules (decoder.cu:773-783).  The prediction
 * is recomputed, and its LSTM state committed, after each emitted token.
 * tokens (device int32[capacity]) receive the emitted ids; result (device
 * int32[4]) = {tokens emitted (may exceed capacity), final frame, status
 * (0, or -2 if the persistent workgroups failed to meet), joint steps}.
 * hidden % 128 == 0, hidden <= 1024, durations <= 8; workspace = device
 * memory of pk_tdt_decode_workspace_bytes(hidden) bytes, overwritten. */
int32_t pk_tdt_decode_workspace_bytes(int32_t hidden);
int32_t pk_tdt_decode(const uint16_t* enc, int32_t frames, int32_t enc_stride, const uint16_t* embedding,
                      const uint16_t* w_ih0, const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0,
                      const uint16_t* w_ih1, const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1,
                      const uint16_t* w_proj, const float* b_proj, const void* w_joint, int32_t joint_int8,
                      const float* joint_scales, const float* b_joint, int32_t hidden, int32_t token_outputs,
                      int32_t durations, int32_t max_symbols, int32_t* tokens, int32_t capacity, int32_t* result,
                      void* workspace, uint64_t workspace_bytes, void* stream);
/* decoder.cu:452-784 tdt_persistent_fp8 (kernel pk_sm89_tdt_persistent_fp8_ih,
 * decoder.cu:805-824; chosen by decoder.rs:86-92 for frames >= 1024): the same
 * decode with the long-request prediction network.  Inside the launch, W_hh0,
 * W_hh1 and W_ih1 become per-tensor symmetric INT8 (scale = max|w| / 127, 1 for
 * an all-zero matrix; q = clamp(rint(w / scale), +-127)); hidden states are
 * also carried as INT8 at scale 1/127 (clamp(rint(127 h))), which feed the
 * recurrent and layer-1 input products; gate = int dot * scale / 127 + b_ih + b_hh
 * (+ layer 0's input_table[token][gate row], fp16, zero before the first
 * token).  input_table = [token_outputs - 1 x 4H] fp16, embedding x W_ih0^T, as
 * decoder.rs:355-377 derives it per request with the fp16 linear
 * (pk_linear_fp16_epilogue, m = tokens, n = 4H, k = H, no bias, scale 1).
 * Cell states, the layer-1 output feeding the projection and the projection
 * are fp32; projection and joint as pk_tdt_decode.  Workspace as
 * pk_tdt_decode_workspace_bytes; W_hh0, W_hh1, W_ih1 16-byte aligned. */
int32_t pk_tdt_decode_long(const uint16_t* enc, int32_t frames, int32_t enc_stride, const uint16_t* input_table,
                           const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1,
                           const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1, const uint16_t* w_proj,
                           const float* b_proj, const void* w_joint, int32_t joint_int8, const float* joint_scales,
                           const float* b_joint, int32_t hidden, int32_t token_outputs, int32_t durations,
                           int32_t max_symbols, int32_t* tokens, int32_t capacity, int32_t* result, void* workspace,
                           uint64_t workspace_bytes, void* stream);

/* ---- long-form local relative-position attention (encoder.cu:1476-2097) ----
 * Model constants: width 1024 = 8 heads x 128, window 128 left / 128 right,
 * position table [8 x 272 x 128] fp16 (rows 257..271 padding).  Query and
 * key are [padded_rows x 1024] fp16 row-major.  value_fp8 is the buffer
 * written by pk_quantize_value_int4{,_register} with value_stride =
 * padded_rows: FP8 V [1024 x stride] (v * 56), S4 V [1024 x stride / 2],
 * 1024 float per-feature scales.  Tiles of 16 queries whose window lies in
 * [0, valid_rows) take the quantized tile path; all other queries the FP32
 * per-query path; rows >= min(rows, valid_rows) are written as zero.
 * Requirements: padded_rows % 16 == 0, rows and valid_rows in (0, padded_rows],
 * value_stride >= padded_rows and % 16 == 0, attention_left = attention_right
 * = 128, 16-byte aligned operands.  `value` (fp16 V) is not read. */

/* encoder.cu:2054-2074 pk_sm89_pack_score_vectors: per 128-value fp16 vector,
 * scale = max|v|/127 (1 if zero), bytes rn(v/scale) in MMA fragment order. */
int32_t pk_pack_score_vectors(const uint16_t* input, uint8_t* output, float* scales, int32_t vectors,
                              void* stream);
/* encoder.cu:2076-2097 pk_sm89_pack_key_int4: scale = max|v|/7, 64 bytes of
 * nibbles rn(v/scale) & 15 per vector in MMA fragment order. */
int32_t pk_pack_key_int4(const uint16_t* input, uint8_t* output, float* scales, int32_t vectors, void* stream);
/* encoder.cu:561-595 pk_sm89_quantize_value_int4: feature-major fp16 V
 * [1024 x elements/1024] -> FP8 V, S4 V (clamp +-7, per-feature max/7),
 * scales.  elements % (1024*16) == 0. */
int32_t pk_quantize_value_int4(const uint16_t* input, uint8_t* output, int32_t elements, float inverse_scale,
                               void* stream);
/* encoder.cu:597-634 pk_sm89_quantize_value_int4_register: as above, but FP8 V
 * is written only for row pairs (2i, 2i+1) with 2i < 272 or 2i + 1 >=
 * valid_rows - 272 (the keys the per-query boundary path reads). */
int32_t pk_quantize_value_int4_register(const uint16_t* input, uint8_t* output, int32_t elements,
                                        float inverse_scale, int32_t valid_rows, void* stream);
/* encoder.cu:2024-2036 pk_sm89_local_relpos_attention_tc_scores: fp16 scores,
 * e4m3 probabilities and V, fp16 output [padded_rows x 1024]. */
int32_t pk_local_relpos_attention_tc_scores(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                                            const uint8_t* value_fp8, const uint16_t* position,
                                            const uint16_t* bias_u, const uint16_t* bias_v, uint16_t* output,
                                            int32_t rows, int32_t padded_rows, int32_t valid_rows,
                                            int32_t attention_left, int32_t attention_right,
                                            int32_t value_stride, void* stream);
/* encoder.cu:2038-2052 pk_sm89_local_relpos_attention_packed: INT4 content
 * scores against pk_pack_key_int4 keys (vectors row*8 + head), INT8 position
 * scores against pk_pack_score_vectors of the position table (vectors
 * head*272 + row), U4 probabilities x S4 V; output e4m3(fp16(context) * 28)
 * bytes [padded_rows x 1024], the input of pk_attention_output_fp8. */
int32_t pk_local_relpos_attention_packed(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                                         const uint8_t* value_fp8, const uint16_t* position,
                                         const uint16_t* bias_u, const uint16_t* bias_v, uint8_t* output,
                                         int32_t rows, int32_t padded_rows, int32_t valid_rows,
                                         int32_t attention_left, int32_t attention_right, int32_t value_stride,
                                         const uint8_t* packed_key, const float* key_scales,
                                         const uint8_t* packed_position, const float* position_scales,
                                         void* stream);
/* encoder.cu:1338-1461 pk_sm89_local_relpos_attention (the reference's kernel
 * for padded_rows < 512, encoder.rs:619,850-858): fp16 Q, K, V [padded_rows x
 * 1024], packed position table [8 x 272 x 128] (pk_pack_position_heads), fp32
 * scores (q + u).k + (q + v).p over 128 dimensions times 1/sqrt(128), softmax,
 * fp16 output [padded_rows x 1024]; rows at or beyond min(rows, valid_rows)
 * are zero.  attention_left, attention_right <= 128. */
int32_t pk_local_relpos_attention(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                                  const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v,
                                  uint16_t* output, int32_t rows, int32_t padded_rows, int32_t valid_rows,
                                  int32_t attention_left, int32_t attention_right, void* stream);
/* encoder.cu:644-671 pk_sm89_quantize_fp8_fixed_transpose (encoder.rs:1293-1320):
 * row-major fp16 V [rows x 1024] -> feature-major e4m3 [1024 x rows],
 * out[f * rows + r] = e4m3(in[r * 1024 + f] * inverse_scale). */
int32_t pk_quantize_fp8_fixed_transpose(const uint16_t* input, uint8_t* output, int32_t rows, float inverse_scale,
                                        void* stream);
/* encoder.cu:1321-1336 pk_sm89_pack_position_heads (encoder.rs:442-480): a
 * position projection [272 x 1024] fp16 -> [8 heads x 272 x 128], the layout
 * every attention kernel reads. */
int32_t pk_pack_position_heads(const uint16_t* input, uint16_t* output, void* stream);

#ifdef __cplusplus
}
#endif
#endif
