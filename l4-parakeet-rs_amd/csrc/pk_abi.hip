// extern "C" boundary of libpk_linear.so (declared in include/pk_linear.h).
// Each entry point validates shapes and pointers on the host, fills a
// GemmArgs or calls a launcher, and reports failures through pk_last_error().
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../../include/pk_linear.h"
#include "pk_kernels.hpp"

namespace pk {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
}

static int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return PK_E_LAUNCH;
    }
    return PK_OK;
}

static GemmArgs base_args(const void* a, const void* b, int m, int n, int k, void* out, int ldo) {
    GemmArgs g{};
    g.a = (const uint8_t*)a;
    g.b = (const uint8_t*)b;
    g.m = m;
    g.n = n;
    g.k = k;
    g.in_scale = 1.0f;
    g.out_scale = 1.0f;
    g.out = out;
    g.ldo = ldo;
    g.valid_rows = m;
    return g;
}

static bool need(const void* p, const char* name) {
    if (!p) set_error("%s must not be NULL", name);
    return p != nullptr;
}

}  // namespace pk

using namespace pk;

#define STREAM ((hipStream_t)stream)

extern "C" {

const char* pk_last_error(void) { return g_error.c_str(); }
int32_t pk_abi_version(void) { return 1; }

// ---- size contracts ---------------------------------------------------------

static size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

int32_t pk_exl3_layout(size_t logical_in, size_t logical_out, int32_t qbits, size_t* out7) {
    if (logical_in == 0 || logical_out == 0) { set_error("linear dimensions must be nonzero"); return PK_E_SHAPE; }
    if (qbits < 1 || qbits > 8) { set_error("EXL3 supports integer rates from 1 through 8 bpw, got %d", qbits); return PK_E_ARG; }
    const size_t pin = round_up(logical_in, 128), pout = round_up(logical_out, 128);
    out7[0] = pin;
    out7[1] = pout;
    out7[2] = pin / 16;
    out7[3] = pout / 16;
    out7[4] = 16 * (size_t)qbits;
    out7[5] = pin * pout * (size_t)qbits / 8;
    out7[6] = 2 * (pin + pout);
    return PK_OK;
}

int32_t pk_estimate_linear(int32_t format, size_t logical_in, size_t logical_out, int32_t exl3_bits, size_t* out6) {
    if (logical_in == 0 || logical_out == 0) { set_error("linear dimensions must be nonzero"); return PK_E_SHAPE; }
    out6[0] = logical_in;
    out6[1] = logical_out;
    switch (format) {
    case 0: case 1: case 2: {
        const size_t pin = round_up(logical_in, 128), pout = round_up(logical_out, 128);
        out6[2] = pin;
        out6[3] = pout;
        out6[4] = pin * pout * (format == 0 ? 2 : 1);
        out6[5] = format == 0 ? 0 : pout * 4;
        return 1;
    }
    case 3:
        if (logical_in % 256 != 0) return 0;
        out6[2] = logical_in;
        out6[3] = logical_out;
        out6[4] = logical_out * (logical_in / 256) * 144;
        out6[5] = 0;
        return 1;
    case 4: {
        size_t e[7];
        const int32_t st = pk_exl3_layout(logical_in, logical_out, exl3_bits, e);
        if (st != PK_OK) return st;
        out6[2] = e[0];
        out6[3] = e[1];
        out6[4] = e[5];
        out6[5] = e[6];
        return 1;
    }
    default:
        set_error("unknown linear format %d", format);
        return PK_E_ARG;
    }
}

// ---- packers ------------------------------------------------------------------

static int32_t pack_rows(int kind, const uint16_t* w, int32_t n, int32_t k, void* q, float* s, void* stream) {
    if (n < 0 || k <= 0 || (kind == 2 && k % 2)) { set_error("invalid packer shape n=%d k=%d", n, k); return PK_E_SHAPE; }
    if (!need(w, "weight") || !need(q, "packed") || !need(s, "scales")) return PK_E_ARG;
    launch_pack_rows(kind, w, q, s, n, k, STREAM);
    return check_launch("pack_rows");
}

int32_t pk_pack_fp8_rows(const uint16_t* w, int32_t n, int32_t k, uint8_t* q, float* s, void* stream) { return pack_rows(0, w, n, k, q, s, stream); }
int32_t pk_pack_int8_rows(const uint16_t* w, int32_t n, int32_t k, int8_t* q, float* s, void* stream) { return pack_rows(1, w, n, k, q, s, stream); }
int32_t pk_pack_int4_rows(const uint16_t* w, int32_t n, int32_t k, uint8_t* q, float* s, void* stream) { return pack_rows(2, w, n, k, q, s, stream); }

int32_t pk_pack_int4_g128(const uint16_t* w, int32_t n, int32_t k, uint32_t* q, uint16_t* s, uint16_t* z, void* stream) {
    if (n < 0 || k <= 0 || k % 128) { set_error("g128 packer needs k %% 128 == 0 (k=%d)", k); return PK_E_SHAPE; }
    if (!need(w, "weight") || !need(q, "packed") || !need(s, "scales") || !need(z, "zeros")) return PK_E_ARG;
    launch_pack_g128(w, q, s, z, n, k, STREAM);
    return check_launch("pack_int4_g128");
}

int32_t pk_expand_int4_g128_e4m3(const uint32_t* q, const uint16_t* z, const uint16_t* scales, int32_t n, int32_t k,
                                 uint8_t* out, uint16_t* scales_t, void* stream) {
    if (n < 0 || k <= 0 || k % 128) { set_error("g128 expansion needs k %% 128 == 0 (k=%d)", k); return PK_E_SHAPE; }
    if (n == 0) return 0;
    if (!need(q, "packed") || !need(z, "zeros") || !need(scales, "scales") || !need(out, "expanded") ||
        !need(scales_t, "scales_t"))
        return PK_E_ARG;
    if (((uintptr_t)q | (uintptr_t)out) & 15) { set_error("packed and expanded must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_expand_g128_e4m3(q, z, scales, scales_t, out, n, k, STREAM);
    return check_launch("expand_int4_g128_e4m3");
}

int32_t pk_q4_k_dequantize(const uint8_t* input, uint16_t* output, int32_t n, int32_t k, void* stream) {
    if (n < 0 || k <= 0 || k % 256) { set_error("Q4_K needs k %% 256 == 0 (k=%d)", k); return PK_E_SHAPE; }
    if (!need(input, "input") || !need(output, "output")) return PK_E_ARG;
    if (((uintptr_t)input | (uintptr_t)output) & 15) { set_error("Q4_K blocks and output must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_q4k_dequant(input, output, n, k, STREAM);
    return check_launch("q4_k_dequantize");
}

// ---- activation quantizers ------------------------------------------------------

int32_t pk_quantize_fp8(const uint16_t* in, uint8_t* out, float inverse_scale, int32_t elements, void* stream) {
    if (elements < 0) { set_error("negative element count"); return PK_E_SHAPE; }
    if (elements && (!need(in, "input") || !need(out, "output"))) return PK_E_ARG;
    launch_quantize_static(in, out, inverse_scale, (size_t)elements, false, STREAM);
    return check_launch("quantize_fp8");
}

int32_t pk_quantize_int8(const uint16_t* in, int8_t* out, float inverse_scale, int32_t elements, void* stream) {
    if (elements < 0) { set_error("negative element count"); return PK_E_SHAPE; }
    if (elements && (!need(in, "input") || !need(out, "output"))) return PK_E_ARG;
    launch_quantize_static(in, out, inverse_scale, (size_t)elements, true, STREAM);
    return check_launch("quantize_int8");
}

int32_t pk_quantize_fp8_fixed(const uint16_t* in, uint8_t* out, int32_t elements, float inverse_scale, void* stream) {
    return pk_quantize_fp8(in, out, inverse_scale, elements, stream);
}

int32_t pk_quantize_rows(int32_t kind, const uint16_t* in, void* out, float* scales, int32_t rows, int32_t valid_rows,
                         int32_t k, void* stream) {
    if (kind < 0 || kind > 2) { set_error("quantize kind must be 0 (fp8), 1 (int8) or 2 (int4)"); return PK_E_ARG; }
    if (rows < 0 || k <= 0 || k % 8) { set_error("quantize_rows needs k %% 8 == 0 (k=%d)", k); return PK_E_SHAPE; }
    if (rows && (!need(in, "input") || !need(out, "output") || !need(scales, "scales"))) return PK_E_ARG;
    if (((uintptr_t)in | (uintptr_t)out) & 15) { set_error("quantize_rows pointers must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_quantize_rows(kind, in, out, scales, rows, valid_rows < 0 ? 0 : valid_rows, k, STREAM);
    return check_launch("quantize_rows");
}

int32_t pk_quantize_rows1024(const uint16_t* in, uint8_t* out, float* scales, int32_t rows, void* stream) {
    return pk_quantize_rows(0, in, out, scales, rows, rows, 1024, stream);
}
int32_t pk_quantize_rows256(const uint16_t* in, uint8_t* out, float* scales, int32_t rows, void* stream) {
    return pk_quantize_rows(0, in, out, scales, rows, rows, 256, stream);
}
int32_t pk_quantize_ffn_contract(const uint16_t* in, uint8_t* out, float* scales, void* stream) {
    return pk_quantize_rows(0, in, out, scales, 1024, 1024, 4096, stream);
}

static int32_t ln_quantize(int mode, const uint16_t* in, const uint16_t* w, const uint16_t* b, uint8_t* out, float* scales,
                           int32_t rows, int32_t padded_rows, float eps, void* stream) {
    const bool int4 = mode == 1;
    if (rows < 0 || padded_rows < rows) { set_error("need 0 <= rows <= padded_rows"); return PK_E_SHAPE; }
    if (padded_rows && (!need(in, "input") || !need(w, "weight") || !need(b, "bias") || !need(out, "output") || !need(scales, "scales")))
        return PK_E_ARG;
    if (((uintptr_t)in | (uintptr_t)w | (uintptr_t)b) & 7 || (uintptr_t)out & (int4 ? 1 : 3)) {
        set_error("layer_norm_quantize needs 8-byte aligned input, weight and bias and a %d-byte aligned output", int4 ? 2 : 4);
        return PK_E_ALIGN;
    }
    launch_layer_norm_quantize(mode, in, w, b, out, scales, nullptr, rows, padded_rows, eps, STREAM);
    return check_launch("layer_norm_quantize");
}

int32_t pk_layer_norm_quantize_fp8_dynamic(const uint16_t* in, const uint16_t* w, const uint16_t* b, uint8_t* out, float* scales,
                                           int32_t rows, int32_t padded_rows, float eps, void* stream) {
    return ln_quantize(0, in, w, b, out, scales, rows, padded_rows, eps, stream);
}
int32_t pk_layer_norm_quantize_int4_dynamic(const uint16_t* in, const uint16_t* w, const uint16_t* b, uint8_t* out, float* scales,
                                            int32_t rows, int32_t padded_rows, float eps, void* stream) {
    return ln_quantize(1, in, w, b, out, scales, rows, padded_rows, eps, stream);
}
int32_t pk_layer_norm_quantize_int4_codes(const uint16_t* in, const uint16_t* w, const uint16_t* b, int8_t* out, float* scales,
                                          int32_t rows, int32_t padded_rows, float eps, void* stream) {
    return ln_quantize(2, in, w, b, (uint8_t*)out, scales, rows, padded_rows, eps, stream);
}

int32_t pk_layer_norm_quantize_int4_fp6(const uint16_t* in, const uint16_t* w, const uint16_t* b, uint8_t* out, float* scales,
                                        int32_t rows, int32_t padded_rows, float eps, void* stream) {
    return ln_quantize(3, in, w, b, out, scales, rows, padded_rows, eps, stream);
}

int32_t pk_unpack_int4_fp6(const uint8_t* packed, uint8_t* codes, int64_t elements, void* stream) {
    if (elements < 0 || elements % 32) { set_error("unpack_int4_fp6 needs a multiple of 32 elements (got %lld)", (long long)elements); return PK_E_SHAPE; }
    if (elements == 0) return 0;
    if (!need(packed, "packed") || !need(codes, "codes")) return PK_E_ARG;
    if (((uintptr_t)packed | (uintptr_t)codes) & 15) { set_error("packed and codes must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_unpack_s4_fp6(packed, codes, (size_t)elements / 2, STREAM);
    return check_launch("unpack_int4_fp6");
}

int32_t pk_unpack_int4(const uint8_t* packed, int8_t* codes, int64_t elements, void* stream) {
    if (elements < 0 || elements % 32) { set_error("unpack_int4 needs a multiple of 32 elements (got %lld)", (long long)elements); return PK_E_SHAPE; }
    if (elements == 0) return 0;
    if (!need(packed, "packed") || !need(codes, "codes")) return PK_E_ARG;
    if (((uintptr_t)packed | (uintptr_t)codes) & 15) { set_error("packed and codes must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_unpack_s4(packed, codes, (size_t)elements / 2, STREAM);
    return check_launch("unpack_int4");
}

int32_t pk_layer_norm_pair(const uint16_t* in, const uint16_t* w, const uint16_t* b, uint16_t* out, const uint16_t* next_w,
                           const uint16_t* next_b, void* next_out, int32_t rows, int32_t padded_rows, float eps, float inverse_scale,
                           void* stream) {
    if (rows < 0 || padded_rows < rows) { set_error("need 0 <= rows <= padded_rows"); return PK_E_SHAPE; }
    if (padded_rows && (!need(in, "input") || !need(w, "weight") || !need(b, "bias") || !need(out, "output") ||
                        !need(next_w, "next_weight") || !need(next_b, "next_bias") || !need(next_out, "next_output")))
        return PK_E_ARG;
    const uintptr_t a8 = (uintptr_t)in | (uintptr_t)w | (uintptr_t)b | (uintptr_t)out | (uintptr_t)next_w | (uintptr_t)next_b;
    if (a8 & 7 || (uintptr_t)next_out & (inverse_scale != 0.0f ? 3 : 7)) {
        set_error("layer_norm_pair needs 8-byte aligned fp16 vectors and a %d-byte aligned next_output",
                  inverse_scale != 0.0f ? 4 : 8);
        return PK_E_ALIGN;
    }
    launch_layer_norm_pair(in, w, b, out, next_w, next_b, next_out, rows, padded_rows, eps, inverse_scale, STREAM);
    return check_launch("layer_norm_pair");
}

// ---- linears ---------------------------------------------------------------------

int32_t pk_gemm(int32_t format, int32_t epilogue, const void* a, const void* b, int32_t m, int32_t n, int32_t k,
                const float* w_scales, const float* row_scales, float in_scale, const float* bias, const uint16_t* residual,
                float out_scale, float res_scale, int32_t activation, const uint16_t* g_scales, const uint16_t* g_zeros,
                void* out, uint8_t* out_meta, int32_t ldo, void* stream) {
    if (!need(a, "a") || !need(b, "b") || !need(out, "out")) return PK_E_ARG;
    if ((format == FMT_G128A8 || format == FMT_G128A16) && (!need(g_scales, "g_scales") || !need(g_zeros, "g_zeros"))) return PK_E_ARG;
    if (format == FMT_G128F8 && !need(g_scales, "g_scales")) return PK_E_ARG;
    if (format == FMT_G128F8 && ((uintptr_t)g_scales & 15)) {
        set_error("format 8 reads its group-major scales as 16-byte vectors: g_scales must be 16-byte aligned");
        return PK_E_ALIGN;
    }
    if (epilogue == EPI_F8_24 && !need(out_meta, "out_meta")) return PK_E_ARG;
    if (activation < 0 || activation > 2) { set_error("activation must be 0, 1 or 2"); return PK_E_ARG; }
    GemmArgs g = base_args(a, b, m, n, k, out, ldo);
    g.w_scales = w_scales;
    g.row_scales = row_scales;
    g.in_scale = in_scale;
    g.bias = bias;
    g.residual = residual;
    g.out_scale = out_scale;
    g.res_scale = res_scale;
    g.act = activation;
    g.g_scales = g_scales;
    g.g_zeros = g_zeros;
    g.out_meta = out_meta;
    return launch_gemm(format, epilogue, g, STREAM);
}

int32_t pk_gemm_tile(int32_t format, int32_t epilogue, int32_t m, int32_t n, int32_t* tile_cols, int32_t* stages) {
    int cols = 0, st = 0;
    const int r = gemm_tile_plan(format, epilogue, m, n, &cols, &st);
    if (r < 0) {
        set_error(r == PK_E_ARG ? "unknown format %d" : "PK_GEMM_TILE_ROWS must be 64, 128 or 256", format);
        return r;
    }
    if (tile_cols) *tile_cols = cols;
    if (stages) *stages = st;
    return r;
}

int32_t pk_gemm_k_split(int32_t format, int32_t epilogue, int32_t m, int32_t n, int32_t k) {
    if (m < 0 || n <= 0 || k <= 0) { set_error("invalid GEMM shape m=%d n=%d k=%d", m, n, k); return PK_E_SHAPE; }
    const int r = gemm_k_split(format, epilogue, m, n, k);
    if (r < 0) set_error(r == PK_E_ARG ? "unknown format %d" : "PK_GEMM_TILE_ROWS must be 64, 128 or 256", format);
    return r;
}

int32_t pk_linear_fp16_epilogue(const uint16_t* in, const uint16_t* w, const float* bias, const uint16_t* residual, uint16_t* out,
                                int32_t m, int32_t n, int32_t k, float out_scale, float res_scale, int32_t act, void* stream) {
    return pk_gemm(FMT_F16, EPI_F16, in, w, m, n, k, nullptr, nullptr, 1.0f, bias, residual, out_scale, res_scale, act, nullptr,
                   nullptr, out, nullptr, n, stream);
}

int32_t pk_q4_k_linear_epilogue(const uint16_t* in, const uint8_t* w, const float* bias, uint16_t* out, int32_t m, int32_t n, int32_t k,
                                int32_t act, void* stream) {
    if (!need(in, "input") || !need(w, "weight_oi") || !need(out, "output")) return PK_E_ARG;
    if (act < 0 || act > 2) { set_error("activation must be 0, 1 or 2"); return PK_E_ARG; }
    GemmArgs g = base_args(in, w, m, n, k, out, n);
    g.in_scale = 1.0f;
    g.bias = bias;
    g.out_scale = 1.0f;
    g.res_scale = 0.0f;
    g.act = act;
    return launch_gemm(FMT_Q4K, EPI_F16, g, STREAM);
}

int32_t pk_linear_fp16_qkv(const uint16_t* in, const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, uint16_t* out, int32_t m,
                           int32_t n, int32_t k, void* stream) {
    const uint16_t* ws[3] = {wq, wk, wv};
    for (int i = 0; i < 3; ++i) {
        const int32_t st = pk_linear_fp16_epilogue(in, ws[i], nullptr, nullptr, out + (size_t)i * m * n, m, n, k, 1.0f, 0.0f, 0, stream);
        if (st != PK_OK) return st;
    }
    return PK_OK;
}

static int32_t scaled_linear(int fmt, int epi, const void* in, const float* row_scales, float in_scale, int fused,
                             const void* w, const float* w_scales, const float* bias, const uint16_t* residual,
                             float out_scale, int32_t act, void* out, int32_t m, int32_t n, int32_t k, void* stream) {
    if (!need(in, "input") || !need(w, "weight_oi") || !need(out, "output")) return PK_E_ARG;
    if (act < 0 || act > 2) { set_error("activation must be 0, 1 or 2"); return PK_E_ARG; }
    GemmArgs g = base_args(in, w, m, n, k, out, n);
    g.w_scales = w_scales;
    g.row_scales = row_scales;
    g.in_scale = in_scale;
    g.fused_scale = fused;
    g.bias = bias;
    g.residual = residual;
    g.out_scale = out_scale;
    g.res_scale = 1.0f;
    g.act = act;
    return launch_gemm(fmt, epi, g, STREAM);
}

int32_t pk_linear_fp8_epilogue(const uint8_t* in, const uint8_t* w, const float* ws, const float* bias, uint16_t* out, int32_t m,
                               int32_t n, int32_t k, float in_scale, int32_t act, void* stream) {
    if (!need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, nullptr, in_scale, 1, w, ws, bias, nullptr, 1.0f, act, out, m, n, k, stream);
}

int32_t pk_linear_int8_epilogue(const int8_t* in, const int8_t* w, const float* ws, const float* bias, uint16_t* out, int32_t m,
                                int32_t n, int32_t k, float in_scale, int32_t act, void* stream) {
    if (!need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_I8, EPI_F16, in, nullptr, in_scale, 1, w, ws, bias, nullptr, 1.0f, act, out, m, n, k, stream);
}

int32_t pk_linear_int8_accumulate(const int8_t* in, const int8_t* w, int32_t* acc, int32_t m, int32_t n, int32_t k, void* stream) {
    return scaled_linear(FMT_I8, EPI_I32, in, nullptr, 1.0f, 0, w, nullptr, nullptr, nullptr, 1.0f, 0, acc, m, n, k, stream);
}

int32_t pk_linear_int4_accumulate(const uint8_t* in, const uint8_t* w, int32_t* acc, int32_t m, int32_t n, int32_t k, void* stream) {
    return scaled_linear(FMT_S4, EPI_I32, in, nullptr, 1.0f, 0, w, nullptr, nullptr, nullptr, 1.0f, 0, acc, m, n, k, stream);
}

int32_t pk_linear_int8_dyn(const int8_t* in, const float* in_scales, const int8_t* w, const float* ws, const float* bias, void* out,
                           int32_t out_fp32, int32_t m, int32_t n, int32_t k, void* stream) {
    if (!need(in_scales, "input_scales") || !need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_I8, out_fp32 ? EPI_F32 : EPI_F16, in, in_scales, 1.0f, 0, w, ws, bias, nullptr, 1.0f, 0, out, m, n, k,
                         stream);
}

int32_t pk_linear_fp8_dyn(const uint8_t* in, const float* in_scales, const uint8_t* w, const float* ws, const float* bias, void* out,
                          int32_t out_fp32, int32_t m, int32_t n, int32_t k, void* stream) {
    if (!need(in_scales, "input_scales") || !need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, out_fp32 ? EPI_F32 : EPI_F16, in, in_scales, 1.0f, 0, w, ws, bias, nullptr, 1.0f, 0, out, m, n, k,
                         stream);
}

int32_t pk_linear_int4g128(const uint16_t* in, const uint32_t* q, const uint16_t* s, const uint16_t* z, const float* bias, void* out,
                           int32_t out_fp32, int32_t m, int32_t n, int32_t k, void* stream) {
    return pk_gemm(FMT_G128A16, out_fp32 ? EPI_F32 : EPI_F16, in, q, m, n, k, nullptr, nullptr, 1.0f, bias, nullptr, 1.0f, 0.0f, 0, s, z,
                   out, nullptr, n, stream);
}

int32_t pk_linear_int4g128_a8(const int8_t* in, const float* in_scales, const uint32_t* q, const uint16_t* s, const uint16_t* z,
                              const float* bias, void* out, int32_t out_fp32, int32_t m, int32_t n, int32_t k, void* stream) {
    if (!need(in_scales, "input_scales")) return PK_E_ARG;
    return pk_gemm(FMT_G128A8, out_fp32 ? EPI_F32 : EPI_F16, in, q, m, n, k, nullptr, in_scales, 1.0f, bias, nullptr, 1.0f, 0.0f, 0, s,
                   z, out, nullptr, n, stream);
}

// ---- encoder wrappers (fixed widths of the reference kernels) -------------------

int32_t pk_ffn_expand_fp8(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint16_t* out, int32_t rows,
                          float in_scale, int32_t dynamic, void* stream) {
    if (!need(ws, "weight_scales") || (dynamic && !need(in_scales, "input_scales"))) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, dynamic ? in_scales : nullptr, in_scale, 0, w, ws, nullptr, nullptr, 1.0f, 1, out, rows,
                         4096, 1024, stream);
}

int32_t pk_ffn_expand_fp8_packed(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint8_t* out,
                                 int32_t rows, float in_scale, int32_t dynamic, void* stream) {
    if (!need(ws, "weight_scales") || (dynamic && !need(in_scales, "input_scales"))) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F8, in, dynamic ? in_scales : nullptr, in_scale, 0, w, ws, nullptr, nullptr, 1.0f, 0, out, rows,
                         4096, 1024, stream);
}

int32_t pk_ffn_expand_int4_sparse(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint8_t* out,
                                  int32_t rows, float in_scale, int32_t dynamic, void* stream) {
    if (!need(in, "input") || !need(w, "weight") || !need(out, "output") || !need(ws, "weight_scales") ||
        (dynamic && !need(in_scales, "input_scales")))
        return PK_E_ARG;
    if (rows < 0) { set_error("negative rows"); return PK_E_SHAPE; }
    GemmArgs g = base_args(in, w, rows, 4096, 1024, out, 4096);
    g.w_scales = ws;
    g.row_scales = dynamic ? in_scales : nullptr;
    g.in_scale = in_scale;
    g.out_meta = out + (size_t)rows * 2048;
    return launch_gemm(FMT_S4, EPI_F8_24, g, STREAM);
}

int32_t pk_ffn_expand_int4_sparse_codes(const int8_t* in, const int8_t* w, const float* ws, const float* in_scales, uint8_t* out,
                                        int32_t rows, float in_scale, int32_t dynamic, void* stream) {
    if (!need(in, "input") || !need(w, "weight") || !need(out, "output") || !need(ws, "weight_scales") ||
        (dynamic && !need(in_scales, "input_scales")))
        return PK_E_ARG;
    if (rows < 0) { set_error("negative rows"); return PK_E_SHAPE; }
    GemmArgs g = base_args(in, w, rows, 4096, 1024, out, 4096);
    g.w_scales = ws;
    g.row_scales = dynamic ? in_scales : nullptr;
    g.in_scale = in_scale;
    g.out_meta = out + (size_t)rows * 2048;
    return launch_gemm(FMT_I8, EPI_F8_24, g, STREAM);
}

int32_t pk_ffn_expand_int4_sparse_fp6(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint8_t* out,
                                      int32_t rows, float in_scale, int32_t dynamic, void* stream) {
    if (!need(in, "input") || !need(w, "weight") || !need(out, "output") || !need(ws, "weight_scales") ||
        (dynamic && !need(in_scales, "input_scales")))
        return PK_E_ARG;
    if (rows < 0) { set_error("negative rows"); return PK_E_SHAPE; }
    GemmArgs g = base_args(in, w, rows, 4096, 1024, out, 4096);
    g.w_scales = ws;
    g.row_scales = dynamic ? in_scales : nullptr;
    g.in_scale = in_scale;
    g.out_meta = out + (size_t)rows * 2048;
    return launch_gemm(FMT_S4F6, EPI_F8_24, g, STREAM);
}

int32_t pk_ffn_contract_fp8(const uint8_t* in, const uint8_t* w, const float* ws, uint16_t* out, int32_t rows, void* stream) {
    if (!need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, nullptr, 1.0f / 16.0f, 0, w, ws, nullptr, out, 0.5f, 0, out, rows, 1024, 4096, stream);
}

int32_t pk_ffn_contract_fp8_sparse(const uint8_t* in, const uint8_t* w, const float* ws, uint16_t* out, int32_t rows,
                                   int32_t inner_width, void* stream) {
    if (!need(in, "input") || !need(w, "weight") || !need(ws, "weight_scales") || !need(out, "output")) return PK_E_ARG;
    if (rows < 0 || inner_width <= 0 || inner_width % 128) {
        set_error("sparse contract needs rows >= 0 and inner_width %% 128 == 0 (got %d)", inner_width);
        return PK_E_SHAPE;
    }
    if (((uintptr_t)in | (uintptr_t)w | (uintptr_t)out) & 15) { set_error("pointers must be 16-byte aligned"); return PK_E_ALIGN; }
    const uint8_t* meta = in + (size_t)rows * (inner_width / 2);
    if (((uintptr_t)meta) & 15) { set_error("metadata (input + rows * inner_width / 2) must be 16-byte aligned"); return PK_E_ALIGN; }
    return launch_sparse24_contract(in, meta, w, ws, 1.0f / 16.0f, out, rows, 1024, inner_width, STREAM);
}

int32_t pk_conv_residual_fp8(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint16_t* out, int32_t rows,
                             void* stream) {
    if (!need(ws, "weight_scales") || !need(in_scales, "input_scales")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, in_scales, 1.0f, 0, w, ws, nullptr, out, 1.0f, 0, out, rows, 1024, 1024, stream);
}

int32_t pk_attention_output_fp8(const uint8_t* in, const uint8_t* w, const float* ws, uint16_t* out, int32_t rows, void* stream) {
    if (!need(ws, "weight_scales")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, nullptr, 1.0f / 28.0f, 0, w, ws, nullptr, out, 1.0f, 0, out, rows, 1024, 1024, stream);
}

int32_t pk_conv_glu_fp8(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, uint16_t* out, int32_t rows,
                        int32_t valid_rows, void* stream) {
    if (!need(in, "input") || !need(w, "weight") || !need(ws, "weight_scales") || !need(in_scales, "input_scales") ||
        !need(out, "output"))
        return PK_E_ARG;
    if (rows < 0 || valid_rows < 0 || valid_rows > rows) { set_error("need 0 <= valid_rows <= rows"); return PK_E_SHAPE; }
    GemmArgs g = base_args(in, w, rows, 2048, 1024, out, 1024);
    g.w_scales = ws;
    g.row_scales = in_scales;
    g.valid_rows = valid_rows;
    return launch_gemm(FMT_FP8, EPI_GLU, g, STREAM);
}

static int32_t subsample_linear(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, const float* bias,
                                uint16_t* out, int32_t rows, int32_t n, int32_t k, int32_t act, void* stream) {
    if (!need(ws, "weight_scales") || !need(in_scales, "input_scales") || !need(bias, "bias")) return PK_E_ARG;
    return scaled_linear(FMT_FP8, EPI_F16, in, in_scales, 1.0f, 0, w, ws, bias, nullptr, 1.0f, act, out, rows, n, k, stream);
}

int32_t pk_subsample_projection_fp8(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, const float* bias,
                                    uint16_t* out, int32_t rows, void* stream) {
    return subsample_linear(in, w, ws, in_scales, bias, out, rows, 1024, 4096, 0, stream);
}

int32_t pk_subsample_pointwise_fp8(const uint8_t* in, const uint8_t* w, const float* ws, const float* in_scales, const float* bias,
                                   uint16_t* out, int32_t rows, void* stream) {
    return subsample_linear(in, w, ws, in_scales, bias, out, rows, 256, 256, 2, stream);
}

int32_t pk_ffn_contract_int8_rowskip(const int8_t* in, const float* in_scales, const int8_t* w, const float* ws, float* out,
                                     int32_t rows, uint32_t* skip_counts, void* stream) {
    if (!need(in, "input") || !need(in_scales, "input_scales") || !need(w, "weight") || !need(ws, "weight_scales") ||
        !need(out, "output"))
        return PK_E_ARG;
    if (rows < 0) { set_error("negative rows"); return PK_E_SHAPE; }
    GemmArgs g = base_args(in, w, rows, 1024, 4096, out, 1024);
    g.w_scales = ws;
    g.row_scales = in_scales;
    g.skip_count = skip_counts;
    return launch_gemm(FMT_I8_SKIP, EPI_F32, g, STREAM);
}

int32_t pk_quantize_rows_int8_sparse24(const uint16_t* in, uint8_t* data, uint8_t* meta, float* scales, uint32_t* overflow_counts,
                                       uint32_t* overflow, uint8_t* residual_data, uint8_t* residual_meta, int32_t rows,
                                       int32_t valid_rows, int32_t k, void* stream) {
    if (rows < 0 || k <= 0 || k % 128 || k > 4096) {
        set_error("sparse24 quantizer needs rows >= 0 and k %% 128 == 0, k <= 4096 (k=%d)", k);
        return PK_E_SHAPE;
    }
    if (rows && (!need(in, "input") || !need(data, "data") || !need(meta, "meta") || !need(scales, "scales") ||
                 !need(overflow_counts, "overflow_counts") || !need(overflow, "overflow")))
        return PK_E_ARG;
    if ((residual_data == nullptr) != (residual_meta == nullptr)) {
        set_error("sparse24 quantizer: residual_data and residual_meta go together");
        return PK_E_ARG;
    }
    if (((uintptr_t)in & 15) || ((uintptr_t)data & 3) || ((uintptr_t)residual_data & 3) || ((uintptr_t)overflow & 3) ||
        ((uintptr_t)overflow_counts & 3)) {
        set_error("sparse24 quantizer: input must be 16-byte aligned, data / residual_data / overflow / overflow_counts 4-byte aligned");
        return PK_E_ALIGN;
    }
    launch_quantize_rows_sp24(in, data, meta, scales, overflow_counts, overflow, residual_data, residual_meta, rows,
                              valid_rows < 0 ? 0 : valid_rows, k, STREAM);
    return check_launch("quantize_rows_int8_sparse24");
}

int32_t pk_transpose_int8(const int8_t* w, int8_t* wt, int32_t n, int32_t k, void* stream) {
    if (n < 0 || k < 0) { set_error("negative transpose shape"); return PK_E_SHAPE; }
    if (n && k && (!need(w, "weight") || !need(wt, "weight_t"))) return PK_E_ARG;
    return launch_transpose_i8(w, wt, n, k, STREAM);
}

int32_t pk_ffn_contract_int8_sparse24(const uint8_t* data, const uint8_t* meta, const float* in_scales, const uint32_t* overflow_counts,
                                      const uint32_t* overflow, const uint8_t* residual_data, const uint8_t* residual_meta,
                                      const int8_t* w, const int8_t* wt, const float* ws, float* out, int32_t rows, void* stream) {
    if (rows < 0) { set_error("negative rows"); return PK_E_SHAPE; }
    if (rows == 0) return PK_OK;
    if (!need(data, "data") || !need(meta, "meta") || !need(in_scales, "input_scales") || !need(overflow_counts, "overflow_counts") ||
        !need(overflow, "overflow") || !need(w, "weight") || !need(wt, "weight_t") || !need(ws, "weight_scales") || !need(out, "output"))
        return PK_E_ARG;
    if ((residual_data == nullptr) != (residual_meta == nullptr)) {
        set_error("sparse INT8 contract: residual_data and residual_meta go together");
        return PK_E_ARG;
    }
    return launch_sparse24_i8_contract(data, meta, in_scales, overflow_counts, overflow, residual_data, residual_meta, w, wt, ws, out,
                                       rows, 1024, 4096, STREAM);
}

// ---- joint ------------------------------------------------------------------------

int32_t pk_joint_gemv(const void* w, int32_t w_int8, const float* w_scales, const float* bias, const uint16_t* enc, const float* pred,
                      float* scores, int32_t* decision, int32_t outputs, int32_t hidden, int32_t token_outputs, int32_t durations,
                      int32_t steps, int32_t enc_stride, void* stream) {
    if (outputs <= 0 || hidden <= 0 || hidden > 1024 || hidden % 16 || steps < 0 || enc_stride < hidden || token_outputs <= 0 ||
        durations < 0 || token_outputs + durations > outputs) {
        set_error("invalid joint shape outputs=%d hidden=%d tokens=%d durations=%d steps=%d stride=%d", outputs, hidden, token_outputs,
                  durations, steps, enc_stride);
        return PK_E_SHAPE;
    }
    if (!need(w, "weight") || !need(enc, "enc") || !need(pred, "pred") || !need(scores, "scores")) return PK_E_ARG;
    if (w_int8 && !need(w_scales, "w_scales")) return PK_E_ARG;
    if ((uintptr_t)w & 15) { set_error("joint weight must be 16-byte aligned"); return PK_E_ALIGN; }
    if ((uintptr_t)enc & 1) { set_error("joint enc must be 2-byte aligned (fp16)"); return PK_E_ALIGN; }
    launch_joint(w, w_int8, w_scales, bias, enc, pred, scores, decision, outputs, hidden, token_outputs, durations, steps, enc_stride,
                 STREAM);
    return check_launch("joint_gemv");
}

static int32_t joint_scan_checks(const void* w, int32_t w_int8, const float* w_scales, const uint16_t* enc, const float* pred,
                                 int32_t outputs, int32_t hidden, int32_t token_outputs, int32_t durations, int32_t frames,
                                 int32_t enc_stride, int32_t max_symbols, int32_t* state) {
    if (outputs <= 0 || hidden <= 0 || hidden > 1024 || hidden % 128 || token_outputs <= 0 || durations <= 0 || durations > 8 ||
        token_outputs + durations > outputs || token_outputs + durations > 2048 || token_outputs > 65535 || frames < 0 ||
        enc_stride < hidden || max_symbols <= 0) {
        set_error("invalid joint scan shape outputs=%d hidden=%d tokens=%d durations=%d frames=%d stride=%d max_symbols=%d", outputs,
                  hidden, token_outputs, durations, frames, enc_stride, max_symbols);
        return PK_E_SHAPE;
    }
    if (!need(w, "weight") || !need(enc, "enc") || !need(pred, "pred") || !need(state, "state")) return PK_E_ARG;
    if (w_int8 && !need(w_scales, "w_scales")) return PK_E_ARG;
    if (((uintptr_t)w | (uintptr_t)enc) & 7 || enc_stride % 2) {
        set_error("joint scan weight and enc must be 8-byte aligned, enc_stride even");
        return PK_E_ALIGN;
    }
    return PK_OK;
}

int32_t pk_joint_scan(const void* w, int32_t w_int8, const float* w_scales, const float* bias, const uint16_t* enc, const float* pred,
                      int32_t outputs, int32_t hidden, int32_t token_outputs, int32_t durations, int32_t frames, int32_t enc_stride,
                      int32_t max_symbols, int32_t* state, uint32_t* workspace, void* stream) {
    const int32_t st = joint_scan_checks(w, w_int8, w_scales, enc, pred, outputs, hidden, token_outputs, durations, frames, enc_stride,
                                         max_symbols, state);
    if (st != PK_OK) return st;
    if (!need(workspace, "workspace")) return PK_E_ARG;
    if ((uintptr_t)workspace & 7) {
        set_error("joint scan workspace must be 8-byte aligned");
        return PK_E_ALIGN;
    }
    launch_joint_scan(w, w_int8, w_scales, bias, enc, pred, outputs, hidden, token_outputs, durations, frames, enc_stride, max_symbols,
                      state, workspace, STREAM);
    return check_launch("joint_scan");
}

int32_t pk_joint_scan_noalloc(const void* w, int32_t w_int8, const float* w_scales, const float* bias, const uint16_t* enc,
                              const float* pred, int32_t outputs, int32_t hidden, int32_t token_outputs, int32_t durations,
                              int32_t frames, int32_t enc_stride, int32_t max_symbols, int32_t* state, void* stream) {
    // The static scratch holds the published words of at most 64 workgroups
    // of 32 joint rows: token_outputs + durations <= 2048.
    if (token_outputs > 0 && durations > 0 && token_outputs + durations > 2048) {
        set_error("joint scan without workspace: token_outputs + durations = %d exceeds the 2048 rows its %d-word static "
                  "scratch serves", token_outputs + durations, kJointScanWorkspaceWords);
        return PK_E_SHAPE;
    }
    const int32_t st = joint_scan_checks(w, w_int8, w_scales, enc, pred, outputs, hidden, token_outputs, durations, frames, enc_stride,
                                         max_symbols, state);
    if (st != PK_OK) return st;
    uint32_t* scratch = nullptr;
    const int r = joint_scan_scratch(&scratch);
    if (r < 0) return r;
    launch_joint_scan(w, w_int8, w_scales, bias, enc, pred, outputs, hidden, token_outputs, durations, frames, enc_stride, max_symbols,
                      state, scratch, STREAM);
    return check_launch("joint_scan_noalloc");
}

int32_t pk_tdt_decode_workspace_bytes(int32_t hidden) { return hidden > 0 ? 4 * decode_workspace_words(hidden) : PK_E_SHAPE; }

static int32_t tdt_decode(bool long_form, const uint16_t* enc, int32_t frames, int32_t enc_stride, const uint16_t* embedding,
                          const uint16_t* table, const uint16_t* w_ih0, const uint16_t* w_hh0, const float* b_ih0,
                          const float* b_hh0, const uint16_t* w_ih1, const uint16_t* w_hh1, const float* b_ih1,
                          const float* b_hh1, const uint16_t* w_proj, const float* b_proj, const void* w_joint,
                          int32_t joint_int8, const float* joint_scales, const float* b_joint, int32_t hidden,
                          int32_t token_outputs, int32_t durations, int32_t max_symbols, int32_t* tokens, int32_t capacity,
                          int32_t* result, void* workspace, uint64_t workspace_bytes, void* stream) {
    if (frames < 0 || hidden <= 0 || hidden > 1024 || hidden % 128 || enc_stride < hidden || token_outputs <= 1 ||
        token_outputs > 65535 || durations <= 0 || durations > 8 || max_symbols <= 0 || capacity < 0) {
        set_error("invalid decode shape frames=%d hidden=%d stride=%d tokens=%d durations=%d max_symbols=%d", frames, hidden,
                  enc_stride, token_outputs, durations, max_symbols);
        return PK_E_SHAPE;
    }
    if (!need(enc, "enc") || (long_form ? !need(table, "input_table") : (!need(embedding, "embedding") || !need(w_ih0, "w_ih0"))) ||
        !need(w_hh0, "w_hh0") ||
        !need(b_ih0, "b_ih0") || !need(b_hh0, "b_hh0") || !need(w_ih1, "w_ih1") || !need(w_hh1, "w_hh1") ||
        !need(b_ih1, "b_ih1") || !need(b_hh1, "b_hh1") || !need(w_proj, "w_proj") || !need(b_proj, "b_proj") ||
        !need(w_joint, "w_joint") || !need(b_joint, "b_joint") || !need(result, "result") || !need(workspace, "workspace") ||
        (capacity > 0 && !need(tokens, "tokens")))
        return PK_E_ARG;
    if (joint_int8 && !need(joint_scales, "joint_scales")) return PK_E_ARG;
    if (workspace_bytes < (uint64_t)4 * decode_workspace_words(hidden)) {
        set_error("decode workspace needs %d bytes", 4 * decode_workspace_words(hidden));
        return PK_E_SHAPE;
    }
    if (((uintptr_t)enc | (uintptr_t)embedding | (uintptr_t)w_ih0 | (uintptr_t)w_hh0 | (uintptr_t)w_ih1 | (uintptr_t)w_hh1 |
         (uintptr_t)w_proj | (uintptr_t)w_joint | (uintptr_t)workspace) & 7 || enc_stride % 2 ||
        (long_form && ((uintptr_t)w_hh0 | (uintptr_t)w_hh1 | (uintptr_t)w_ih1) & 15)) {
        set_error("decode weights, enc and workspace must be 8-byte aligned (long form: W_hh0, W_hh1, W_ih1 16-byte), "
                  "enc_stride even");
        return PK_E_ALIGN;
    }
    const uint16_t* w_ih[2] = {w_ih0, w_ih1};
    const uint16_t* w_hh[2] = {w_hh0, w_hh1};
    const float* b_ih[2] = {b_ih0, b_ih1};
    const float* b_hh[2] = {b_hh0, b_hh1};
    const int st = launch_tdt_decode(enc, frames, enc_stride, long_form ? nullptr : embedding, long_form ? table : nullptr, w_ih, w_hh,
                                     b_ih, b_hh, w_proj, b_proj, w_joint, joint_int8, joint_scales, b_joint, hidden, token_outputs,
                                     durations, max_symbols, tokens, capacity, result, (uint32_t*)workspace, STREAM);
    if (st != 0) return PK_E_SHAPE;
    return check_launch(long_form ? "tdt_decode_long" : "tdt_decode");
}

int32_t pk_tdt_decode(const uint16_t* enc, int32_t frames, int32_t enc_stride, const uint16_t* embedding,
                      const uint16_t* w_ih0, const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0,
                      const uint16_t* w_ih1, const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1,
                      const uint16_t* w_proj, const float* b_proj, const void* w_joint, int32_t joint_int8,
                      const float* joint_scales, const float* b_joint, int32_t hidden, int32_t token_outputs,
                      int32_t durations, int32_t max_symbols, int32_t* tokens, int32_t capacity, int32_t* result,
                      void* workspace, uint64_t workspace_bytes, void* stream) {
    return tdt_decode(false, enc, frames, enc_stride, embedding, nullptr, w_ih0, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1, b_hh1,
                      w_proj, b_proj, w_joint, joint_int8, joint_scales, b_joint, hidden, token_outputs, durations, max_symbols,
                      tokens, capacity, result, workspace, workspace_bytes, stream);
}

int32_t pk_tdt_decode_long(const uint16_t* enc, int32_t frames, int32_t enc_stride, const uint16_t* input_table,
                           const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1,
                           const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1, const uint16_t* w_proj,
                           const float* b_proj, const void* w_joint, int32_t joint_int8, const float* joint_scales,
                           const float* b_joint, int32_t hidden, int32_t token_outputs, int32_t durations,
                           int32_t max_symbols, int32_t* tokens, int32_t capacity, int32_t* result, void* workspace,
                           uint64_t workspace_bytes, void* stream) {
    return tdt_decode(true, enc, frames, enc_stride, nullptr, input_table, nullptr, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1,
                      b_hh1, w_proj, b_proj, w_joint, joint_int8, joint_scales, b_joint, hidden, token_outputs, durations,
                      max_symbols, tokens, capacity, result, workspace, workspace_bytes, stream);
}

// ---- local attention and its producers ---------------------------------------

static bool misaligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) != 0; }

static int32_t pack_vectors(bool int4, const uint16_t* input, uint8_t* output, float* scales, int32_t vectors, void* stream) {
    if (vectors < 0) { set_error("vectors must be >= 0, got %d", vectors); return PK_E_SHAPE; }
    if (vectors == 0) return PK_OK;
    if (!need(input, "input") || !need(output, "output") || !need(scales, "scales")) return PK_E_ARG;
    if (misaligned(input, 16) || misaligned(output, 4)) { set_error("input must be 16-byte, output 4-byte aligned"); return PK_E_ALIGN; }
    launch_pack_vectors(int4, input, output, scales, vectors, STREAM);
    return check_launch(int4 ? "pack_key_int4" : "pack_score_vectors");
}

int32_t pk_pack_score_vectors(const uint16_t* input, uint8_t* output, float* scales, int32_t vectors, void* stream) {
    return pack_vectors(false, input, output, scales, vectors, stream);
}

int32_t pk_pack_key_int4(const uint16_t* input, uint8_t* output, float* scales, int32_t vectors, void* stream) {
    return pack_vectors(true, input, output, scales, vectors, stream);
}

static int32_t quantize_value(const uint16_t* input, uint8_t* output, int32_t elements, float inverse_scale, bool edge_only,
                              int32_t valid_rows, void* stream) {
    if (elements <= 0 || elements % (1024 * 16)) {
        set_error("value elements must be a positive multiple of 1024*16, got %d", elements);
        return PK_E_SHAPE;
    }
    if (edge_only && (valid_rows < 0 || valid_rows > elements / 1024)) {
        set_error("valid_rows %d outside [0, %d]", valid_rows, elements / 1024);
        return PK_E_SHAPE;
    }
    if (!need(input, "input") || !need(output, "output")) return PK_E_ARG;
    if (misaligned(input, 16) || misaligned(output, 8)) { set_error("input must be 16-byte, output 8-byte aligned"); return PK_E_ALIGN; }
    launch_quantize_value_int4(input, output, elements / 1024, inverse_scale, edge_only, valid_rows, STREAM);
    return check_launch("quantize_value_int4");
}

int32_t pk_quantize_value_int4(const uint16_t* input, uint8_t* output, int32_t elements, float inverse_scale, void* stream) {
    return quantize_value(input, output, elements, inverse_scale, false, 0, stream);
}

int32_t pk_quantize_value_int4_register(const uint16_t* input, uint8_t* output, int32_t elements, float inverse_scale,
                                        int32_t valid_rows, void* stream) {
    return quantize_value(input, output, elements, inverse_scale, true, valid_rows, stream);
}

static int32_t local_attention(bool packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                               const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output,
                               int32_t rows, int32_t padded_rows, int32_t valid_rows, int32_t attention_left,
                               int32_t attention_right, int32_t value_stride, const uint8_t* packed_key, const float* key_scales,
                               const uint8_t* packed_position, const float* position_scales, void* stream) {
    if (padded_rows <= 0 || padded_rows % 16 || padded_rows > (1 << 21) || rows <= 0 || rows > padded_rows || valid_rows <= 0 ||
        valid_rows > padded_rows || value_stride < padded_rows || value_stride % 16) {
        set_error("invalid attention shape rows=%d padded_rows=%d valid_rows=%d value_stride=%d", rows, padded_rows, valid_rows,
                  value_stride);
        return PK_E_SHAPE;
    }
    if (attention_left != 128 || attention_right != 128) {
        set_error("the long-form attention kernels are built for a 128/128 window, got %d/%d", attention_left, attention_right);
        return PK_E_SHAPE;
    }
    if (!need(query, "query") || !need(key, "key") || !need(value_fp8, "value_fp8") || !need(position, "position") ||
        !need(bias_u, "bias_u") || !need(bias_v, "bias_v") || !need(output, "output"))
        return PK_E_ARG;
    if (packed && (!need(packed_key, "packed_key") || !need(key_scales, "key_scales") || !need(packed_position, "packed_position") ||
                   !need(position_scales, "position_scales")))
        return PK_E_ARG;
    if (misaligned(query, 16) || misaligned(key, 16) || misaligned(position, 16) || misaligned(bias_u, 16) ||
        misaligned(bias_v, 16) || misaligned(value_fp8, 16) || misaligned(output, 16) || misaligned(packed_key, 8) ||
        misaligned(packed_position, 16) || misaligned(key_scales, 4) || misaligned(position_scales, 4)) {
        set_error("attention operands must be 16-byte aligned (packed keys 8-byte, scales 4-byte)");
        return PK_E_ALIGN;
    }
    launch_local_attention(packed, query, key, value_fp8, position, bias_u, bias_v, output, rows, padded_rows, valid_rows,
                           attention_left, attention_right, value_stride, packed_key, key_scales, packed_position, position_scales,
                           STREAM);
    return check_launch(packed ? "local_relpos_attention_packed" : "local_relpos_attention_tc_scores");
}

int32_t pk_local_relpos_attention_tc_scores(const uint16_t* query, const uint16_t* key, const uint16_t* value, const uint8_t* value_fp8,
                                            const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v,
                                            uint16_t* output, int32_t rows, int32_t padded_rows, int32_t valid_rows,
                                            int32_t attention_left, int32_t attention_right, int32_t value_stride, void* stream) {
    (void)value;
    return local_attention(false, query, key, value_fp8, position, bias_u, bias_v, output, rows, padded_rows, valid_rows,
                           attention_left, attention_right, value_stride, nullptr, nullptr, nullptr, nullptr, stream);
}

int32_t pk_local_relpos_attention_packed(const uint16_t* query, const uint16_t* key, const uint16_t* value, const uint8_t* value_fp8,
                                         const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, uint8_t* output,
                                         int32_t rows, int32_t padded_rows, int32_t valid_rows, int32_t attention_left,
                                         int32_t attention_right, int32_t value_stride, const uint8_t* packed_key,
                                         const float* key_scales, const uint8_t* packed_position, const float* position_scales,
                                         void* stream) {
    (void)value;
    return local_attention(true, query, key, value_fp8, position, bias_u, bias_v, output, rows, padded_rows, valid_rows,
                           attention_left, attention_right, value_stride, packed_key, key_scales, packed_position,
                           position_scales, stream);
}

int32_t pk_local_relpos_attention(const uint16_t* query, const uint16_t* key, const uint16_t* value, const uint16_t* position,
                                  const uint16_t* bias_u, const uint16_t* bias_v, uint16_t* output, int32_t rows,
                                  int32_t padded_rows, int32_t valid_rows, int32_t attention_left, int32_t attention_right,
                                  void* stream) {
    if (padded_rows < 0 || rows < 0 || valid_rows < 0 || attention_left < 0 || attention_right < 0 ||
        attention_left > 128 || attention_right > 128) {
        set_error("invalid short attention shape rows=%d padded=%d valid=%d left=%d right=%d", rows, padded_rows, valid_rows,
                  attention_left, attention_right);
        return PK_E_SHAPE;
    }
    if (padded_rows == 0) return PK_OK;
    if (!need(query, "query") || !need(key, "key") || !need(value, "value") || !need(position, "position") ||
        !need(bias_u, "bias_u") || !need(bias_v, "bias_v") || !need(output, "output"))
        return PK_E_ARG;
    if (misaligned(query, 16) || misaligned(key, 16) || misaligned(position, 16) || misaligned(bias_u, 16) ||
        misaligned(bias_v, 16) || misaligned(value, 4) || misaligned(output, 4)) {
        set_error("query, key, position and biases must be 16-byte aligned, value and output 4-byte");
        return PK_E_ALIGN;
    }
    launch_local_attention_short(query, key, value, position, bias_u, bias_v, output, rows, padded_rows, valid_rows,
                                 attention_left, attention_right, STREAM);
    return check_launch("local_relpos_attention");
}

int32_t pk_quantize_fp8_fixed_transpose(const uint16_t* input, uint8_t* output, int32_t rows, float inverse_scale, void* stream) {
    if (rows < 0) { set_error("rows must be >= 0, got %d", rows); return PK_E_SHAPE; }
    if (rows == 0) return PK_OK;
    if (!need(input, "input") || !need(output, "output")) return PK_E_ARG;
    if (misaligned(input, 16) || (rows % 16 == 0 && misaligned(output, 16))) {
        set_error("input must be 16-byte aligned (and output too when rows %% 16 == 0)");
        return PK_E_ALIGN;
    }
    launch_quantize_fp8_transpose(input, output, rows, inverse_scale, STREAM);
    return check_launch("quantize_fp8_fixed_transpose");
}

int32_t pk_pack_position_heads(const uint16_t* input, uint16_t* output, void* stream) {
    if (!need(input, "input") || !need(output, "output")) return PK_E_ARG;
    if (misaligned(input, 16) || misaligned(output, 16)) { set_error("input and output must be 16-byte aligned"); return PK_E_ALIGN; }
    launch_pack_position_heads(input, output, STREAM);
    return check_launch("pack_position_heads");
}

}  // extern "C"
