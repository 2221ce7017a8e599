/*
 * pk_oracle.c -- CPU restatement of the l4-parakeet-rs quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for libpk_linear.so.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * The reference is Rust + CUDA and cannot be built in this image (no cargo,
 * no crates, no nvcc), so each function below restates the reference's
 * arithmetic from its source, citing file:line.  How each function is pinned
 * (known answers from the reference's own tests, an independent library, a
 * closed form or brute force) is recorded in tests/test_oracle_*.py; the
 * functions without such a pin say "parity unpinned" in their comment.
 */
#include "pk_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

int orc_threads(void) { return g_threads; }

void orc_set_threads(int threads) {
    g_threads = threads < 1 ? 1 : threads;
#ifdef _OPENMP
    omp_set_num_threads(g_threads);
#endif
}

static uint32_t f32_bits(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    return bits;
}

static float bits_f32(uint32_t bits) {
    float value;
    memcpy(&value, &bits, 4);
    return value;
}

/* IEEE binary16, round-to-nearest-even (the `half` 2.7.1 crate's f16::from_f32,
 * used by every reference packer, e.g. artifact.rs:421-423).  Written from the
 * IEEE 754 definition; pinned against numpy.float16 exhaustively in tests. */
uint16_t orc_f32_to_f16(float value) {
    uint32_t x = f32_bits(value);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    }
    if (a >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a < 0x38800000u) { /* below 2^-14: subnormal half, units of 2^-24 */
        float q = nearbyintf(bits_f32(a) * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)q);
    }
    uint32_t r = a - (112u << 23); /* rebias 127 -> 15 */
    r = r + 0x0fffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)(r >> 13));
}

float orc_f16_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t mantissa = bits & 0x3ffu;
    if (exponent == 0) {
        float magnitude = (float)mantissa * (1.0f / 16777216.0f);
        return sign ? -magnitude : magnitude;
    }
    if (exponent == 31) {
        return bits_f32(sign | 0x7f800000u | (mantissa << 13));
    }
    return bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* OCP FP8 E4M3 ("e4m3fn": bias 7, no infinities, 0x7f/0xff NaN, max 448).
 * The reference encodes with the float8 0.7.0 crate, F8E4M3::from_f32
 * (quant_benchmark.rs:797, encoder.rs:410), and on device with the
 * saturating __nv_fp8_e4m3 constructor (encoder.cu:557, linear.cu:544).
 * Restated from the OCP 8-bit floating point specification: round to nearest
 * even, finite overflow and +-inf saturate to +-448, NaN -> 0x7f.  Known
 * answers 1.0->0x38, -1.0->0xb8, 448->0x7e (quant_benchmark.rs:962-966); the
 * NaN encoding is parity unpinned (no reference test covers it). */
uint8_t orc_f32_to_e4m3(float value) {
    if (isnan(value)) {
        return 0x7f;
    }
    uint8_t sign = signbit(value) ? 0x80 : 0x00;
    float a = fabsf(value);
    if (a >= 448.0f) {
        return (uint8_t)(sign | 0x7e);
    }
    if (a < 0.015625f) { /* subnormal range: multiples of 2^-9 */
        float q = nearbyintf(a * 512.0f);
        return (uint8_t)(sign | (uint8_t)q);
    }
    int e;
    float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    int exponent = e - 1;
    int mantissa = (int)nearbyintf((2.0f * m - 1.0f) * 8.0f);
    if (mantissa == 8) {
        mantissa = 0;
        exponent += 1;
    }
    return (uint8_t)(sign | (uint8_t)(((exponent + 7) << 3) | mantissa));
}

float orc_e4m3_to_f32(uint8_t bits) {
    int sign = bits & 0x80;
    int exponent = (bits >> 3) & 15;
    int mantissa = bits & 7;
    float magnitude;
    if (exponent == 15 && mantissa == 7) {
        return NAN;
    }
    if (exponent == 0) {
        magnitude = ldexpf((float)mantissa, -9);
    } else {
        magnitude = ldexpf(1.0f + (float)mantissa / 8.0f, exponent - 7);
    }
    return sign ? -magnitude : magnitude;
}

/* FP6 e3m2 (OCP MX formats: sign bit 5, exponent bits 4..2 with bias 3,
 * mantissa bits 1..0, subnormals at exponent 0, no infinity or NaN).  No
 * reference counterpart: the operand form of INT4 codes for the f8f6f4 MFMA. */
float orc_e3m2_to_f32(uint8_t bits) {
    const int exponent = (bits >> 2) & 7, mantissa = bits & 3;
    const float magnitude = exponent == 0 ? ldexpf((float)mantissa / 4.0f, -2) : ldexpf(1.0f + (float)mantissa / 4.0f, exponent - 3);
    return (bits & 0x20) ? -magnitude : magnitude;
}

/* The e3m2 bits of an integer in -8..8, found by searching the 32 positive
 * encodings for the exact value (255 when none holds it). */
uint8_t orc_e3m2_of_int(int v) {
    const int a = v < 0 ? -v : v;
    for (int bits = 0; bits < 32; ++bits)
        if (orc_e3m2_to_f32((uint8_t)bits) == (float)a) return (uint8_t)(bits | (v < 0 ? 0x20 : 0));
    return 255;
}

/* int8 codes [count] (count a multiple of 16) -> the FP6 chunk form: each 16
 * codes one 16-byte chunk, code j's e3m2 bits at bits 6j..6j+5 of the chunk's
 * first 12 bytes read as a little-endian 96-bit number, then 4 zero bytes. */
void orc_fp6_chunks(const int8_t* codes, size_t count, uint8_t* out) {
    for (size_t c = 0; c < count / 16; ++c) {
        uint8_t* o = out + 16 * c;
        memset(o, 0, 16);
        for (int j = 0; j < 16; ++j) {
            const unsigned f = orc_e3m2_of_int(codes[16 * c + j]);
            for (int b = 0; b < 6; ++b)
                if ((f >> b) & 1u) o[(6 * j + b) >> 3] |= (uint8_t)(1u << ((6 * j + b) & 7));
        }
    }
}

/* quant_benchmark.rs:827-829: round half to even, then clamp to +-127. */
int8_t orc_quantize_i8(float value) {
    float r = nearbyintf(value);
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    if (isnan(r)) return 0;
    return (int8_t)r;
}

/* cuda.rs:809-818: splitmix64 finalizer mapped to [-amplitude, amplitude]. */
float orc_pattern(uint64_t index, uint64_t salt, float amplitude) {
    uint64_t value = index + salt * 0x9e3779b97f4a7c15ull;
    value ^= value >> 30;
    value *= 0xbf58476d1ce4e5b9ull;
    value ^= value >> 27;
    value *= 0x94d049bb133111ebull;
    value ^= value >> 31;
    float unit = (float)(value & 0xffffu) / 65535.0f;
    return (unit * 2.0f - 1.0f) * amplitude;
}

void orc_pattern_fill(float* out, size_t count, uint64_t first_index, uint64_t salt,
                      float amplitude) {
    for (size_t i = 0; i < count; ++i) {
        out[i] = orc_pattern(first_index + i, salt, amplitude);
    }
}

/* ---- size contracts ----------------------------------------------------- */

static size_t round_up(size_t value, size_t multiple) {
    return (value + multiple - 1) / multiple * multiple;
}

/* exl3.rs:37-75.  out7 = {padded_in, padded_out, trellis0, trellis1,
 * trellis2, trellis_bytes, scale_bytes}.  Returns 0, or -1 for empty / -2
 * for an invalid bit rate (Exl3LayoutError). */
int orc_exl3_layout(size_t logical_in, size_t logical_out, int qbits, size_t* out7) {
    if (logical_in == 0 || logical_out == 0) return -1;
    if (qbits < 1 || qbits > 8) return -2;
    size_t pin = round_up(logical_in, 128);
    size_t pout = round_up(logical_out, 128);
    out7[0] = pin;
    out7[1] = pout;
    out7[2] = pin / 16;
    out7[3] = pout / 16;
    out7[4] = 16 * (size_t)qbits;
    out7[5] = pin * pout * (size_t)qbits / 8;
    out7[6] = 2 * (pin + pout);
    return 0;
}

/* packing.rs:71-130.  format: 0 fp16, 1 fp8 e4m3, 2 int8, 3 Q4_K, 4 EXL3.
 * out6 = {logical_in, logical_out, padded_in, padded_out, payload, metadata}.
 * Returns 1 when a layout exists, 0 for Q4_K's "None", -1 for Empty. */
int orc_estimate_linear(int format, size_t logical_in, size_t logical_out, int exl3_bits,
                        size_t* out6) {
    if (logical_in == 0 || logical_out == 0) return -1;
    out6[0] = logical_in;
    out6[1] = logical_out;
    switch (format) {
    case 0:
    case 1:
    case 2: {
        size_t pin = round_up(logical_in, 128);
        size_t pout = round_up(logical_out, 128);
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
        int status = orc_exl3_layout(logical_in, logical_out, exl3_bits, e);
        if (status != 0) return status == -1 ? -1 : -2;
        out6[2] = e[0];
        out6[3] = e[1];
        out6[4] = e[5];
        out6[5] = e[6];
        return 1;
    }
    default:
        return -3;
    }
}

/* ---- weight packers ----------------------------------------------------- */

/* Per-row FP8: quant_benchmark.rs:779-801 and encoder.rs:367-412 (FP8
 * branch): scale = max|w| / 448, byte = e4m3(w / scale).  An all-zero row
 * gets scale 1 as in the request-time packer (encoder.cu:1141); the host
 * packers would divide by zero there. */
void orc_pack_fp8_rows(const uint16_t* w, int n, int k, uint8_t* q, float* scales) {
    for (int row = 0; row < n; ++row) {
        const uint16_t* values = w + (size_t)row * k;
        float maximum = 0.0f;
        for (int i = 0; i < k; ++i) maximum = fmaxf(maximum, fabsf(orc_f16_to_f32(values[i])));
        float scale = maximum > 0.0f ? maximum / 448.0f : 1.0f;
        scales[row] = scale;
        for (int i = 0; i < k; ++i) {
            q[(size_t)row * k + i] = orc_f32_to_e4m3(orc_f16_to_f32(values[i]) / scale);
        }
    }
}

/* Per-row INT8: quant_benchmark.rs:803-829: scale = max|w| / 127,
 * q = clamp(rne(w / scale), +-127).  Zero rows get scale 1 (see above). */
void orc_pack_int8_rows(const uint16_t* w, int n, int k, int8_t* q, float* scales) {
    for (int row = 0; row < n; ++row) {
        const uint16_t* values = w + (size_t)row * k;
        float maximum = 0.0f;
        for (int i = 0; i < k; ++i) maximum = fmaxf(maximum, fabsf(orc_f16_to_f32(values[i])));
        float scale = maximum > 0.0f ? maximum / 127.0f : 1.0f;
        scales[row] = scale;
        for (int i = 0; i < k; ++i) {
            q[(size_t)row * k + i] = orc_quantize_i8(orc_f16_to_f32(values[i]) / scale);
        }
    }
}

static int clamp_rne(float value, int lo, int hi) {
    if (isnan(value)) return 0; /* Rust `NaN as i8` is 0 (encoder.rs:396-404) */
    float r = nearbyintf(value);
    if (r < (float)lo) r = (float)lo;
    if (r > (float)hi) r = (float)hi;
    return (int)r;
}

/* Per-row symmetric INT4: encoder.rs:378-407 (INT4 branch):
 * scale = max over the row of max(w/7, -w/8) (folded from 0), q = clamp(rne(w /
 * scale), -8, 7), byte j = q[2j] & 15 | (q[2j+1] & 15) << 4.  An all-zero row
 * keeps scale 0 and packs to zero bytes (0/0 is NaN and `NaN as i8` is 0). */
void orc_pack_int4_rows(const uint16_t* w, int n, int k, uint8_t* q, float* scales) {
    for (int row = 0; row < n; ++row) {
        const uint16_t* values = w + (size_t)row * k;
        float scale = 0.0f;
        for (int i = 0; i < k; ++i) {
            float v = orc_f16_to_f32(values[i]);
            scale = fmaxf(scale, fmaxf(v / 7.0f, -v / 8.0f));
        }
        scales[row] = scale;
        for (int j = 0; j < k / 2; ++j) {
            int a = clamp_rne(orc_f16_to_f32(values[2 * j]) / scale, -8, 7);
            int b = clamp_rne(orc_f16_to_f32(values[2 * j + 1]) / scale, -8, 7);
            q[(size_t)row * (k / 2) + j] = (uint8_t)((a & 15) | ((b & 15) << 4));
        }
    }
}

/* Group-wise asymmetric INT4, groups of 128 along K.  This format has no
 * counterpart in the reference (its INT4 formats are the per-row symmetric one
 * above and GGUF Q4_K); parity unpinned against the reference, pinned by its
 * closed form.  Per (row, group): lo = min(0, min w), hi = max(0, max w),
 * s = fp16((hi - lo) / 15) (1 if that is 0), z = clamp(rne(-lo / s), 0, 15),
 * q = clamp(rne(w / s) + z, 0, 15); dequant (q - z) * s.  q is packed eight
 * per uint32 along K: word j holds k = 8j .. 8j+7, k = 8j+i sitting at bit
 * 8*(i%4) + 4*(i/4) (byte b carries k 8j+b low and 8j+4+b high), so two masks
 * give the levels in k order on the GPU.  scales and zeros are fp16
 * [n x k/128]; zeros are integers in [0, 15]. */
static int g128_shift(int i) { return 8 * (i & 3) + 4 * (i >> 2); }

void orc_pack_int4_g128(const uint16_t* w, int n, int k, uint32_t* q, uint16_t* scales,
                        uint16_t* zeros) {
    int groups = k / 128;
    for (int row = 0; row < n; ++row) {
        for (int g = 0; g < groups; ++g) {
            const uint16_t* values = w + (size_t)row * k + g * 128;
            float lo = 0.0f, hi = 0.0f;
            for (int i = 0; i < 128; ++i) {
                float v = orc_f16_to_f32(values[i]);
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            float s = orc_f16_to_f32(orc_f32_to_f16((hi - lo) / 15.0f));
            if (!(s > 0.0f)) s = 1.0f;
            int z = clamp_rne(-lo / s, 0, 15);
            scales[(size_t)row * groups + g] = orc_f32_to_f16(s);
            zeros[(size_t)row * groups + g] = orc_f32_to_f16((float)z);
            for (int j = 0; j < 16; ++j) {
                uint32_t word = 0;
                for (int i = 0; i < 8; ++i) {
                    float v = orc_f16_to_f32(values[8 * j + i]);
                    int level = clamp_rne(v / s, -64, 64) + z;
                    level = level < 0 ? 0 : (level > 15 ? 15 : level);
                    word |= (uint32_t)level << g128_shift(i);
                }
                q[(size_t)row * (k / 8) + g * 16 + j] = word;
            }
        }
    }
}

/* artifact.rs:430-465 (encode_fp16_linear): f32 [out x in] -> fp16
 * [padded_out x padded_in], zero padding. */
void orc_pad_fp16_linear(const float* src, int logical_out, int logical_in, int padded_out,
                         int padded_in, uint16_t* dst) {
    memset(dst, 0, (size_t)padded_out * padded_in * 2);
    for (int row = 0; row < logical_out; ++row) {
        for (int col = 0; col < logical_in; ++col) {
            dst[(size_t)row * padded_in + col] = orc_f32_to_f16(src[(size_t)row * logical_in + col]);
        }
    }
}

/* ---- GGUF Q4_K (q4k_benchmark.rs:403-597, linear.cu:431-456) ------------ */

static int nearest_int(float value) { return (int)nearbyintf(value); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void q4k_scale_min(const uint8_t* packed, int group, int* scale, int* minimum) {
    if (group < 4) {
        *scale = packed[group] & 63;
        *minimum = packed[group + 4] & 63;
    } else {
        *scale = (packed[group + 4] & 0x0f) | ((packed[group - 4] >> 6) << 4);
        *minimum = (packed[group + 4] >> 4) | ((packed[group] >> 6) << 4);
    }
}

/* q4k_benchmark.rs:488-562 (make_qkx2_quants: nmax 15, rmin -1, rdelta 0.1,
 * 20 steps). */
static void make_qkx2_quants(const float* x, const float* weights, uint8_t* levels,
                             float* out_scale, float* out_min) {
    float minimum = x[0], maximum = x[0];
    float sum_w = weights[0], sum_x = weights[0] * x[0];
    for (int i = 1; i < 32; ++i) {
        minimum = fminf(minimum, x[i]);
        maximum = fmaxf(maximum, x[i]);
        sum_w += weights[i];
        sum_x += weights[i] * x[i];
    }
    minimum = fminf(minimum, 0.0f);
    if (maximum == minimum) {
        memset(levels, 0, 32);
        *out_scale = 0.0f;
        *out_min = -minimum;
        return;
    }
    float iscale = 15.0f / (maximum - minimum);
    float scale = 1.0f / iscale;
    float best_error = 0.0f;
    for (int i = 0; i < 32; ++i) {
        int l = clampi(nearest_int(iscale * (x[i] - minimum)), 0, 15);
        levels[i] = (uint8_t)l;
        float diff = scale * (float)l + minimum - x[i];
        best_error += weights[i] * diff * diff;
    }
    uint8_t aux[32];
    for (int step = 0; step <= 20; ++step) {
        iscale = (-1.0f + 0.1f * (float)step + 15.0f) / (maximum - minimum);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < 32; ++i) {
            int l = clampi(nearest_int(iscale * (x[i] - minimum)), 0, 15);
            aux[i] = (uint8_t)l;
            sum_l += weights[i] * (float)l;
            sum_l2 += weights[i] * (float)(l * l);
            sum_xl += weights[i] * (float)l * x[i];
        }
        float det = sum_w * sum_l2 - sum_l * sum_l;
        if (det <= 0.0f) continue;
        float this_scale = (sum_w * sum_xl - sum_x * sum_l) / det;
        float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / det;
        if (this_min > 0.0f) {
            this_min = 0.0f;
            this_scale = sum_xl / sum_l2;
        }
        float error = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float diff = this_scale * (float)aux[i] + this_min - x[i];
            error += weights[i] * diff * diff;
        }
        if (error < best_error) {
            memcpy(levels, aux, 32);
            best_error = error;
            scale = this_scale;
            minimum = this_min;
        }
    }
    *out_scale = scale;
    *out_min = -minimum;
}

/* q4k_benchmark.rs:403-486 (encode_q4_k_block). */
void orc_q4k_encode_block(const uint16_t* src256, uint8_t* block) {
    memset(block, 0, 144);
    float x[256];
    for (int i = 0; i < 256; ++i) x[i] = orc_f16_to_f32(src256[i]);
    uint8_t levels[256];
    float scales[8], minimums[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int g = 0; g < 8; ++g) {
        const float* v = x + g * 32;
        float sum_sq = 0.0f;
        for (int i = 0; i < 32; ++i) sum_sq += v[i] * v[i];
        float rms = sqrtf(sum_sq / 32.0f);
        float weights[32];
        for (int i = 0; i < 32; ++i) weights[i] = rms + fabsf(v[i]);
        make_qkx2_quants(v, weights, levels + g * 32, &scales[g], &minimums[g]);
        max_scale = fmaxf(max_scale, scales[g]);
        max_min = fmaxf(max_min, minimums[g]);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t packed[12];
    memset(packed, 0, 12);
    for (int g = 0; g < 8; ++g) {
        int ls = clampi(nearest_int(inv_scale * scales[g]), 0, 63);
        int lm = clampi(nearest_int(inv_min * minimums[g]), 0, 63);
        if (g < 4) {
            packed[g] = (uint8_t)ls;
            packed[g + 4] = (uint8_t)lm;
        } else {
            packed[g + 4] = (uint8_t)((ls & 0x0f) | ((lm & 0x0f) << 4));
            packed[g - 4] |= (uint8_t)((ls >> 4) << 6);
            packed[g] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    uint16_t d = orc_f32_to_f16(max_scale / 63.0f);
    uint16_t dmin = orc_f32_to_f16(max_min / 63.0f);
    block[0] = (uint8_t)(d & 0xff);
    block[1] = (uint8_t)(d >> 8);
    block[2] = (uint8_t)(dmin & 0xff);
    block[3] = (uint8_t)(dmin >> 8);
    memcpy(block + 4, packed, 12);
    for (int g = 0; g < 8; ++g) {
        int sc, mn;
        q4k_scale_min(packed, g, &sc, &mn);
        float scale = orc_f16_to_f32(d) * (float)sc;
        if (scale == 0.0f) continue;
        float minimum = orc_f16_to_f32(dmin) * (float)mn;
        for (int i = 0; i < 32; ++i) {
            levels[g * 32 + i] = (uint8_t)clampi(nearest_int((x[g * 32 + i] + minimum) / scale), 0, 15);
        }
    }
    for (int pair = 0; pair < 4; ++pair) {
        for (int i = 0; i < 32; ++i) {
            block[16 + pair * 32 + i] =
                (uint8_t)(levels[pair * 64 + i] | (levels[pair * 64 + 32 + i] << 4));
        }
    }
}

/* q4k_benchmark.rs:579-597 / linear.cu:445-456: d*sc*q - dmin*m. */
float orc_q4k_value(const uint8_t* block, int index) {
    float d = orc_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    float dmin = orc_f16_to_f32((uint16_t)(block[2] | (block[3] << 8)));
    int group = index / 32;
    uint8_t packed = block[16 + (group / 2) * 32 + (index % 32)];
    int quant = (group % 2 == 0) ? (packed & 0x0f) : (packed >> 4);
    int sc, mn;
    q4k_scale_min(block + 4, group, &sc, &mn);
    return d * (float)sc * (float)quant - dmin * (float)mn;
}

/* q4k_benchmark.rs:385-401. */
void orc_q4k_encode(const uint16_t* w, int n, int k, uint8_t* blocks) {
    int per_row = k / 256;
    for (int row = 0; row < n; ++row) {
        for (int b = 0; b < per_row; ++b) {
            orc_q4k_encode_block(w + (size_t)row * k + b * 256,
                                 blocks + ((size_t)row * per_row + b) * 144);
        }
    }
}

/* ---- activation quantizers ---------------------------------------------- */

/* linear.cu:537-547 / encoder.cu:549-559: e4m3(f16 * inverse_scale). */
void orc_quantize_fp8_static(const uint16_t* x, size_t count, float inverse_scale,
                             uint8_t* out) {
    for (size_t i = 0; i < count; ++i) out[i] = orc_f32_to_e4m3(orc_f16_to_f32(x[i]) * inverse_scale);
}

/* linear.cu:549-560: rne(clamp(f16 * inverse_scale, +-127)). */
void orc_quantize_int8_static(const uint16_t* x, size_t count, float inverse_scale,
                              int8_t* out) {
    for (size_t i = 0; i < count; ++i) {
        float s = orc_f16_to_f32(x[i]) * inverse_scale;
        s = fminf(127.0f, fmaxf(-127.0f, s));
        out[i] = (int8_t)nearbyintf(s);
    }
}

/* Dynamic per-row FP8 (encoder.cu:264-292 without the norm, and the
 * request-time row packers encoder.cu:1129-1180): scale = max|x| / 448, 1 for
 * all-zero rows and for padding rows >= valid_rows (which quantize to 0). */
void orc_quantize_fp8_rows(const uint16_t* x, int rows, int valid_rows, int k, uint8_t* q,
                           float* scales) {
    for (int r = 0; r < rows; ++r) {
        uint8_t* out = q + (size_t)r * k;
        if (r >= valid_rows) {
            memset(out, 0, (size_t)k);
            scales[r] = 1.0f;
            continue;
        }
        float maximum = 0.0f;
        for (int i = 0; i < k; ++i) maximum = fmaxf(maximum, fabsf(orc_f16_to_f32(x[(size_t)r * k + i])));
        float scale = maximum > 0.0f ? maximum / 448.0f : 1.0f;
        scales[r] = scale;
        for (int i = 0; i < k; ++i) out[i] = orc_f32_to_e4m3(orc_f16_to_f32(x[(size_t)r * k + i]) / scale);
    }
}

/* Dynamic per-token INT8 (BASELINE config 3 "mixed variant"; no reference
 * counterpart, pinned by closed form): scale = max|x| / 127 (1 if zero),
 * q = clamp(rne(x / scale), +-127). */
void orc_quantize_int8_rows(const uint16_t* x, int rows, int valid_rows, int k, int8_t* q,
                            float* scales) {
    for (int r = 0; r < rows; ++r) {
        int8_t* out = q + (size_t)r * k;
        if (r >= valid_rows) {
            memset(out, 0, (size_t)k);
            scales[r] = 1.0f;
            continue;
        }
        float maximum = 0.0f;
        for (int i = 0; i < k; ++i) maximum = fmaxf(maximum, fabsf(orc_f16_to_f32(x[(size_t)r * k + i])));
        float scale = maximum > 0.0f ? maximum / 127.0f : 1.0f;
        scales[r] = scale;
        for (int i = 0; i < k; ++i) out[i] = (int8_t)clamp_rne(orc_f16_to_f32(x[(size_t)r * k + i]) / scale, -127, 127);
    }
}

/* Dynamic per-row INT4 (encoder.cu:264-290, kInt4): scale = max(max(x/7,
 * -x/8)) (1 if not positive), q = clamp(rne(x / scale), -8, 7), nibble pairs
 * with the even column low. */
void orc_quantize_int4_rows(const uint16_t* x, int rows, int valid_rows, int k, uint8_t* q,
                            float* scales) {
    for (int r = 0; r < rows; ++r) {
        uint8_t* out = q + (size_t)r * (k / 2);
        if (r >= valid_rows) {
            memset(out, 0, (size_t)k / 2);
            scales[r] = 1.0f;
            continue;
        }
        float maximum = 0.0f;
        for (int i = 0; i < k; ++i) {
            float v = orc_f16_to_f32(x[(size_t)r * k + i]);
            maximum = fmaxf(maximum, fmaxf(v / 7.0f, -v / 8.0f));
        }
        float scale = maximum > 0.0f ? maximum : 1.0f;
        scales[r] = scale;
        for (int j = 0; j < k / 2; ++j) {
            int a = clamp_rne(orc_f16_to_f32(x[(size_t)r * k + 2 * j]) / scale, -8, 7);
            int b = clamp_rne(orc_f16_to_f32(x[(size_t)r * k + 2 * j + 1]) / scale, -8, 7);
            out[j] = (uint8_t)((a & 15) | ((b & 15) << 4));
        }
    }
}

/* LayerNorm then dynamic per-row quantization (encoder.cu:211-306).  The
 * statistics use the reference's reduction shape: 256 partial sums (thread t
 * adds x[t], x[t+256], x[t+512], x[t+768] in that order), folded by
 * block_sum_tree_tail (encoder.cu:36-54) -- pairs (t, t+128), (t+64, t+192),
 * (t+32, t+160), (t+96, t+224), then ((s0+s1)+(s2+s3)), then a 32-lane
 * shuffle-down tree.  The reference uses the approximate rsqrtf; this
 * restatement (and the HIP kernel) uses the correctly rounded 1/sqrtf, a
 * deviation of at most 2 ulp in inverse_std.  Requires k == 1024. */
static float tree_sum_256(const float* partial) {
    float lanes[32];
    for (int lane = 0; lane < 32; ++lane) {
        float s0 = partial[lane] + partial[lane + 128];
        float s1 = partial[lane + 64] + partial[lane + 192];
        float s2 = partial[lane + 32] + partial[lane + 160];
        float s3 = partial[lane + 96] + partial[lane + 224];
        lanes[lane] = (s0 + s1) + (s2 + s3);
    }
    for (int offset = 16; offset > 0; offset /= 2) {
        for (int lane = 0; lane < 32; ++lane) {
            if (lane + offset < 32) lanes[lane] += lanes[lane + offset];
        }
    }
    return lanes[0];
}

void orc_layer_norm_quantize(const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                             int rows, int valid_rows, int k, float epsilon, int int4,
                             uint8_t* q, float* scales, uint16_t* normalized) {
    (void)k; /* fixed at 1024 (kModelWidth) */
    const int width = 1024;
    for (int r = 0; r < rows; ++r) {
        const uint16_t* in = x + (size_t)r * width;
        if (r >= valid_rows) {
            if (int4) memset(q + (size_t)r * width / 2, 0, width / 2);
            else memset(q + (size_t)r * width, 0, width);
            scales[r] = 1.0f;
            if (normalized) memset(normalized + (size_t)r * width, 0, width * 2);
            continue;
        }
        float partial[256];
        float values[1024];
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int item = 0; item < 4; ++item) {
                values[t + item * 256] = orc_f16_to_f32(in[t + item * 256]);
                s += values[t + item * 256];
            }
            partial[t] = s;
        }
        float mean = tree_sum_256(partial) / 1024.0f;
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int item = 0; item < 4; ++item) {
                float d = values[t + item * 256] - mean;
                s += d * d;
            }
            partial[t] = s;
        }
        float inverse_std = 1.0f / sqrtf(tree_sum_256(partial) / 1024.0f + epsilon);
        float maximum = 0.0f;
        for (int i = 0; i < width; ++i) {
            float y = (values[i] - mean) * inverse_std * orc_f16_to_f32(gamma[i]) + orc_f16_to_f32(beta[i]);
            uint16_t h = orc_f32_to_f16(y);
            if (normalized) normalized[(size_t)r * width + i] = h;
            values[i] = orc_f16_to_f32(h);
            if (int4) maximum = fmaxf(maximum, fmaxf(values[i] / 7.0f, -values[i] / 8.0f));
            else maximum = fmaxf(maximum, fabsf(values[i]));
        }
        float scale = maximum > 0.0f ? (int4 ? maximum : maximum / 448.0f) : 1.0f;
        scales[r] = scale;
        if (int4) {
            for (int j = 0; j < width / 2; ++j) {
                int a = clamp_rne(values[2 * j] / scale, -8, 7);
                int b = clamp_rne(values[2 * j + 1] / scale, -8, 7);
                q[(size_t)r * width / 2 + j] = (uint8_t)((a & 15) | ((b & 15) << 4));
            }
        } else {
            for (int i = 0; i < width; ++i) q[(size_t)r * width + i] = orc_f32_to_e4m3(values[i] / scale);
        }
    }
}

/* LayerNorm pair (encoder.cu:128-209): first = f16(LN(x; w1, b1)) into out;
 * second = f16(LN(first; w2, b2)) into next_out as fp16 (inverse_scale == 0)
 * or as e4m3(second * inverse_scale) bytes.  Both statistics in the
 * reduction shape of orc_layer_norm_quantize (the reference's second LN sums
 * a thread's four rounded first values in feature order, :181-184).  Rows >=
 * valid_rows are zeros in both outputs.  next_out holds rows x 1024 uint16
 * (fp16) or uint8 (e4m3) codes. */
static void ln_row(const float* x, const uint16_t* gamma, const uint16_t* beta, float epsilon, uint16_t* h) {
    float partial[256];
    for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int item = 0; item < 4; ++item) s += x[t + item * 256];
        partial[t] = s;
    }
    const float mean = tree_sum_256(partial) / 1024.0f;
    for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int item = 0; item < 4; ++item) {
            const float d = x[t + item * 256] - mean;
            s += d * d;
        }
        partial[t] = s;
    }
    const float inverse_std = 1.0f / sqrtf(tree_sum_256(partial) / 1024.0f + epsilon);
    for (int i = 0; i < 1024; ++i)
        h[i] = orc_f32_to_f16((x[i] - mean) * inverse_std * orc_f16_to_f32(gamma[i]) + orc_f16_to_f32(beta[i]));
}

void orc_layer_norm_pair(const uint16_t* x, const uint16_t* w1, const uint16_t* b1, const uint16_t* w2,
                         const uint16_t* b2, int rows, int valid_rows, float epsilon, float inverse_scale,
                         uint16_t* out, void* next_out) {
    for (int r = 0; r < rows; ++r) {
        uint16_t* first = out + (size_t)r * 1024;
        if (r >= valid_rows) {
            memset(first, 0, 2048);
            memset((uint8_t*)next_out + (size_t)r * (inverse_scale != 0.0f ? 1024 : 2048), 0,
                   inverse_scale != 0.0f ? 1024 : 2048);
            continue;
        }
        float v[1024];
        uint16_t second[1024];
        for (int i = 0; i < 1024; ++i) v[i] = orc_f16_to_f32(x[(size_t)r * 1024 + i]);
        ln_row(v, w1, b1, epsilon, first);
        for (int i = 0; i < 1024; ++i) v[i] = orc_f16_to_f32(first[i]);
        ln_row(v, w2, b2, epsilon, second);
        if (inverse_scale != 0.0f) {
            uint8_t* q = (uint8_t*)next_out + (size_t)r * 1024;
            for (int i = 0; i < 1024; ++i) q[i] = orc_f32_to_e4m3(orc_f16_to_f32(second[i]) * inverse_scale);
        } else {
            memcpy((uint16_t*)next_out + (size_t)r * 1024, second, 2048);
        }
    }
}

/* 2:4 compression of FP8 activations (encoder.cu:685-704, epilogue 7 at
 * :1037-1053): in each quartet keep the two largest |e4m3| (bits & 127), ties
 * to the lower index, in index order.  data is [rows x k/2]; meta is
 * [rows x k/8] bytes, quartet p's 4-bit field idx0 | idx1 << 2 at bits
 * 4*(p%2) of byte p/2. */
void orc_compress_24(const uint8_t* x, int rows, int k, uint8_t* data, uint8_t* meta) {
    memset(meta, 0, (size_t)rows * k / 8);
    for (int r = 0; r < rows; ++r) {
        for (int p = 0; p < k / 4; ++p) {
            const uint8_t* v = x + (size_t)r * k + 4 * p;
            int count = 0;
            int nibble = 0;
            for (int i = 0; i < 4; ++i) {
                int rank = 0;
                for (int j = 0; j < 4; ++j) {
                    int mi = v[i] & 127, mj = v[j] & 127;
                    rank += mj > mi || (mj == mi && j < i);
                }
                if (rank < 2) {
                    data[(size_t)r * k / 2 + 2 * p + count] = v[i];
                    nibble |= i << (2 * count);
                    ++count;
                }
            }
            meta[(size_t)r * k / 8 + p / 2] |= (uint8_t)(nibble << (4 * (p % 2)));
        }
    }
}

/* Exact 2:4 form of INT8 rows (the activation-sparse FF2 of BASELINE config
 * 4): per quartet the selection of orc_compress_24 on int8 magnitudes |v|
 * (encoder.cu:685-704 keeps the two largest, ties to the lower index, in index
 * order), and every nonzero it drops goes to the row's overflow list as
 * (element << 8) | byte in ascending element order.  counts[r] entries at
 * ovf[r * k/2 ...]. */
void orc_compress_24_i8_exact(const int8_t* x, int rows, int k, uint8_t* data, uint8_t* meta, uint32_t* counts, uint32_t* ovf) {
    memset(meta, 0, (size_t)rows * k / 8);
    for (int r = 0; r < rows; ++r) {
        uint32_t n = 0;
        for (int p = 0; p < k / 4; ++p) {
            const int8_t* v = x + (size_t)r * k + 4 * p;
            int count = 0, nibble = 0;
            for (int i = 0; i < 4; ++i) {
                int rank = 0;
                const int mi = abs((int)v[i]);
                for (int j = 0; j < 4; ++j) {
                    const int mj = abs((int)v[j]);
                    rank += j != i && (mj > mi || (mj == mi && j < i));
                }
                if (rank < 2) {
                    data[(size_t)r * k / 2 + 2 * p + count] = (uint8_t)v[i];
                    nibble |= i << (2 * count);
                    ++count;
                } else if (v[i] != 0) {
                    ovf[(size_t)r * (k / 2) + n++] = ((uint32_t)(4 * p + i) << 8) | (uint8_t)v[i];
                }
            }
            meta[(size_t)r * k / 8 + p / 2] |= (uint8_t)(nibble << (4 * (p % 2)));
        }
        counts[r] = n;
    }
}

/* Residual 2:4 form of the same INT8 rows (no counterpart in the reference;
 * this build's alternative to the overflow lists for rows with many dropped
 * nonzeros): per quartet the two positions the selection in `meta` (above)
 * did not keep, in ascending order, with their bytes (zero or not), so that
 * decompressing (data, meta) and (data2, meta2) gives disjoint parts whose
 * union is the row. */
void orc_residual_24_i8(const int8_t* x, const uint8_t* meta, int rows, int k, uint8_t* data2, uint8_t* meta2) {
    memset(meta2, 0, (size_t)rows * k / 8);
    for (int r = 0; r < rows; ++r) {
        for (int p = 0; p < k / 4; ++p) {
            const int nibble = (meta[(size_t)r * k / 8 + p / 2] >> (4 * (p % 2))) & 15;
            const int kept = (1 << (nibble & 3)) | (1 << ((nibble >> 2) & 3));
            int count = 0, out = 0;
            for (int i = 0; i < 4; ++i) {
                if (kept & (1 << i)) continue;
                if (count < 2) {
                    data2[(size_t)r * k / 2 + 2 * p + count] = (uint8_t)x[(size_t)r * k + 4 * p + i];
                    out |= i << (2 * count);
                }
                ++count;
            }
            meta2[(size_t)r * k / 8 + p / 2] |= (uint8_t)(out << (4 * (p % 2)));
        }
    }
}

void orc_decompress_24(const uint8_t* data, const uint8_t* meta, int rows, int k, uint8_t* x) {
    memset(x, 0, (size_t)rows * k);
    for (int r = 0; r < rows; ++r) {
        for (int p = 0; p < k / 4; ++p) {
            int nibble = (meta[(size_t)r * k / 8 + p / 2] >> (4 * (p % 2))) & 15;
            x[(size_t)r * k + 4 * p + (nibble & 3)] = data[(size_t)r * k / 2 + 2 * p];
            x[(size_t)r * k + 4 * p + ((nibble >> 2) & 3)] = data[(size_t)r * k / 2 + 2 * p + 1];
        }
    }
}

/* ---- GEMM references ---------------------------------------------------- */

/* Exact i32 dot products (quant_benchmark.rs:872-909). */
void orc_gemm_i8_i32(const int8_t* x, const int8_t* w, int m, int n, int k, int32_t* acc) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            const int8_t* a = x + (size_t)i * k;
            const int8_t* b = w + (size_t)j * k;
            int32_t s = 0;
            for (int t = 0; t < k; ++t) s += (int32_t)a[t] * (int32_t)b[t];
            acc[(size_t)i * n + j] = s;
        }
    }
}

static int s4(uint8_t byte, int high) {
    int v = high ? (byte >> 4) : (byte & 15);
    return v >= 8 ? v - 16 : v;
}

/* s4 x s4 -> exact s32 (the mma...s4.s4 path, encoder.cu:775-782); both
 * operands packed two per byte, even k in the low nibble. */
void orc_gemm_s4_i32(const uint8_t* x, const uint8_t* w, int m, int n, int k, int32_t* acc) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            const uint8_t* a = x + (size_t)i * k / 2;
            const uint8_t* b = w + (size_t)j * k / 2;
            int32_t s = 0;
            for (int t = 0; t < k / 2; ++t) {
                s += s4(a[t], 0) * s4(b[t], 0) + s4(a[t], 1) * s4(b[t], 1);
            }
            acc[(size_t)i * n + j] = s;
        }
    }
}

static float e4m3_table[256];
static int e4m3_table_ready = 0;

static void init_e4m3_table(void) {
    if (!e4m3_table_ready) {
        for (int i = 0; i < 256; ++i) e4m3_table[i] = orc_e4m3_to_f32((uint8_t)i);
        e4m3_table_ready = 1;
    }
}

/* Dequantize-then-fp32 dot products in index order (quant_benchmark.rs:
 * 832-869: fold over k of f32(x) * f32(w)).  Products of two e4m3 values are
 * exact in fp32; only the summation rounds. */
void orc_gemm_e4m3_f32(const uint8_t* x, const uint8_t* w, int m, int n, int k, float* acc) {
    init_e4m3_table();
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        float* a = (float*)malloc((size_t)k * sizeof(float));
        for (int t = 0; t < k; ++t) a[t] = e4m3_table[x[(size_t)i * k + t]];
        for (int j = 0; j < n; ++j) {
            const uint8_t* b = w + (size_t)j * k;
            float s = 0.0f;
            for (int t = 0; t < k; ++t) s += a[t] * e4m3_table[b[t]];
            acc[(size_t)i * n + j] = s;
        }
        free(a);
    }
}

/* cuda.rs:821-861: fp16 operands, fp32 fold. */
void orc_gemm_f16_f32(const uint16_t* x, const uint16_t* w, int m, int n, int k, float* acc) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        float* a = (float*)malloc((size_t)k * sizeof(float));
        for (int t = 0; t < k; ++t) a[t] = orc_f16_to_f32(x[(size_t)i * k + t]);
        for (int j = 0; j < n; ++j) {
            const uint16_t* b = w + (size_t)j * k;
            float s = 0.0f;
            for (int t = 0; t < k; ++t) s += a[t] * orc_f16_to_f32(b[t]);
            acc[(size_t)i * n + j] = s;
        }
        free(a);
    }
}

static int g128_level(const uint32_t* q, int k, int row, int t) {
    return (int)((q[(size_t)row * (k / 8) + t / 8] >> g128_shift(t % 8)) & 15u);
}

/* W4A16 with group-wise asymmetric INT4 weights: out = sum over groups of
 * s_g * (sum over the group of x * (q - z)).  Products x * (q - z) are exact
 * in fp32 (11-bit x 5-bit significands); the group sums fold in k order. */
void orc_gemm_g128_a16(const uint16_t* x, const uint32_t* q, const uint16_t* scales,
                       const uint16_t* zeros, int m, int n, int k, float* out) {
    int groups = k / 128;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float total = 0.0f;
            for (int g = 0; g < groups; ++g) {
                float z = orc_f16_to_f32(zeros[(size_t)j * groups + g]);
                float s = orc_f16_to_f32(scales[(size_t)j * groups + g]);
                float part = 0.0f;
                for (int t = g * 128; t < g * 128 + 128; ++t) {
                    part += orc_f16_to_f32(x[(size_t)i * k + t]) * ((float)g128_level(q, k, j, t) - z);
                }
                total = fmaf(part, s, total);
            }
            out[(size_t)i * n + j] = total;
        }
    }
}

/* W4A8: exact i32 per-group accumulators acc_g = sum x_i8 * (q - z) (z is an
 * integer), then out = x_scale * (sum over g in order of fmaf(acc_g, s_g, .)).
 * parts > 1: the groups are split into `parts` contiguous runs (run p: groups
 * [groups p / parts, groups (p + 1) / parts)), each summed in order from 0,
 * and the run sums added in order -- the association of the kernel that
 * splits a tile's K-steps over its waves. */
void orc_gemm_g128_a8(const int8_t* x, const float* x_scales, const uint32_t* q,
                      const uint16_t* scales, const uint16_t* zeros, int m, int n, int k, int parts,
                      int32_t* group_acc, float* out) {
    int groups = k / 128;
    if (parts < 1) parts = 1;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float total = 0.0f;
            for (int p = 0; p < parts; ++p) {
                float part = 0.0f;
                for (int g = groups * p / parts; g < groups * (p + 1) / parts; ++g) {
                    int z = (int)orc_f16_to_f32(zeros[(size_t)j * groups + g]);
                    int32_t a = 0;
                    for (int t = g * 128; t < g * 128 + 128; ++t) {
                        a += (int32_t)x[(size_t)i * k + t] * (g128_level(q, k, j, t) - z);
                    }
                    if (group_acc) group_acc[((size_t)i * n + j) * groups + g] = a;
                    part = fmaf((float)a, orc_f16_to_f32(scales[(size_t)j * groups + g]), part);
                }
                total = p == 0 ? part : total + part;
            }
            out[(size_t)i * n + j] = total * x_scales[i];
        }
    }
}

/* e4m3 activations x INT4-g128 weights (no reference counterpart; the
 * weights' dequant is (q - z) * s, pk_pack_int4_g128 layout): per output, each
 * 128-K group's sum of e4m3(x) * (q - z) -- every product exact in fp32 --
 * accumulated in double and rounded once to fp32 (the device's MFMA sums a
 * group in fp32 in its own order, so device results agree within a
 * tolerance, not bit for bit), then folded in K order as fmaf(sum, s, acc).
 * out is the accumulator before the epilogue's activation scale. */
void orc_gemm_g128_f8(const uint8_t* x, const uint32_t* q, const uint16_t* scales, const uint16_t* zeros, int m,
                      int n, int k, float* out) {
    const int groups = k / 128;
    float table[256];
    for (int c = 0; c < 256; ++c) table[c] = orc_e4m3_to_f32((uint8_t)c);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int g = 0; g < groups; ++g) {
                const int z = (int)orc_f16_to_f32(zeros[(size_t)j * groups + g]);
                double sum = 0.0;
                for (int t = g * 128; t < g * 128 + 128; ++t)
                    sum += (double)table[x[(size_t)i * k + t]] * (double)(g128_level(q, k, j, t) - z);
                acc = fmaf((float)sum, orc_f16_to_f32(scales[(size_t)j * groups + g]), acc);
            }
            out[(size_t)i * n + j] = acc;
        }
    }
}

/* q4k_benchmark.rs:910-945: fp16 activations times f16(dequant(Q4_K)). */
void orc_gemm_q4k_f32(const uint16_t* x, const uint8_t* blocks, int m, int n, int k, float* acc) {
    int per_row = k / 256;
    float* wd = (float*)malloc((size_t)n * k * sizeof(float));
    for (int j = 0; j < n; ++j) {
        for (int t = 0; t < k; ++t) {
            const uint8_t* block = blocks + ((size_t)j * per_row + t / 256) * 144;
            wd[(size_t)j * k + t] = orc_f16_to_f32(orc_f32_to_f16(orc_q4k_value(block, t % 256)));
        }
    }
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int t = 0; t < k; ++t) s += orc_f16_to_f32(x[(size_t)i * k + t]) * wd[(size_t)j * k + t];
            acc[(size_t)i * n + j] = s;
        }
    }
    free(wd);
}

/* ---- epilogues ------------------------------------------------------------ */

static float silu(float v) { return v / (1.0f + expf(-v)); }

static float round_f16(float v) { return orc_f16_to_f32(orc_f32_to_f16(v)); }

/* ffn_fp8_async epilogues (encoder.cu:911-1058).  value = acc * row_scale *
 * w_scale, row_scale = row_scales[r] when given, else in_scale.
 *   0: SiLU -> fp16                     1: SiLU -> fp16 -> x16 -> e4m3 (out8)
 *   2: out16 = fp16(fmaf(0.5, value, out16))     (FF contract, residual)
 *   3: + bias -> fp16                   4: + bias, ReLU -> fp16
 *   5: GLU over n = 2 * width columns: fp16(v) / (1 + exp(-fp16(g))) with
 *      v = column c, g = column c + width; rows >= valid_rows write 0
 *      (out16 is [m x width])
 *   6: out16 = fp16(value + out16)      (residual, scale 1)
 *   7: as 1 (the 2:4 compression is orc_compress_24 on its output)
 *   8: as 2 (sparse-input contract)
 *   9: SiLU -> fp16 -> x16 -> static INT8 (out8 as int8 bytes): the FF
 *      hidden at the scale of mode 1 through the static INT8 quantizer of
 *      linear.cu:549-560, rne(clamp(v, -127, 127)) */
void orc_epilogue(const float* acc, const float* row_scales, float in_scale,
                  const float* w_scales, const float* bias, int m, int n, int mode,
                  int valid_rows, uint16_t* out16, uint8_t* out8) {
    if (mode == 5) {
        int width = n / 2;
        for (int r = 0; r < m; ++r) {
            float rs = row_scales ? row_scales[r] : in_scale;
            for (int c = 0; c < width; ++c) {
                float v = round_f16(acc[(size_t)r * n + c] * rs * w_scales[c]);
                float g = round_f16(acc[(size_t)r * n + c + width] * rs * w_scales[c + width]);
                out16[(size_t)r * width + c] = r < valid_rows ? orc_f32_to_f16(v / (1.0f + expf(-g))) : 0;
            }
        }
        return;
    }
    for (int r = 0; r < m; ++r) {
        float rs = row_scales ? row_scales[r] : in_scale;
        for (int c = 0; c < n; ++c) {
            size_t idx = (size_t)r * n + c;
            float value = acc[idx] * rs * w_scales[c];
            switch (mode) {
            case 0:
                out16[idx] = orc_f32_to_f16(silu(value));
                break;
            case 1:
            case 7:
                out8[idx] = orc_f32_to_e4m3(round_f16(silu(value)) * 16.0f);
                break;
            case 2:
            case 8:
                out16[idx] = orc_f32_to_f16(fmaf(0.5f, value, orc_f16_to_f32(out16[idx])));
                break;
            case 9: {
                float h = round_f16(silu(value)) * 16.0f;
                h = fminf(fmaxf(h, -127.0f), 127.0f);
                out8[idx] = (uint8_t)(int8_t)rintf(h);
                break;
            }
            case 3:
                out16[idx] = orc_f32_to_f16(value + bias[c]);
                break;
            case 4:
                out16[idx] = orc_f32_to_f16(fmaxf(value + bias[c], 0.0f));
                break;
            case 6:
                out16[idx] = orc_f32_to_f16(fmaf(1.0f, value, orc_f16_to_f32(out16[idx])));
                break;
            default:
                break;
            }
        }
    }
}

static float activate(float v, int activation) {
    if (activation == 1) return silu(v);
    if (activation == 2) return fmaxf(v, 0.0f);
    return v;
}

/* FP16 linear epilogue (linear.cu:137-156): v = (acc + bias) * out_scale;
 * v = fmaf(res_scale, residual, v); act; fp16.  bias/residual may be NULL. */
void orc_epilogue_linear(const float* acc, const float* bias, const uint16_t* residual,
                         int m, int n, float out_scale, float res_scale, int activation,
                         uint16_t* out) {
    for (int r = 0; r < m; ++r) {
        for (int c = 0; c < n; ++c) {
            size_t idx = (size_t)r * n + c;
            float v = acc[idx];
            if (bias) v += bias[c];
            v *= out_scale;
            if (residual) v = fmaf(res_scale, orc_f16_to_f32(residual[idx]), v);
            out[idx] = orc_f32_to_f16(activate(v, activation));
        }
    }
}

/* FP8 / INT8 linear epilogue (linear.cu:362-373, 417-428):
 * act(fmaf(acc, in_scale * w_scale[c], bias[c])) -> fp16.  bias may be NULL. */
void orc_epilogue_quantized(const float* acc, float in_scale, const float* w_scales,
                            const float* bias, int m, int n, int activation, uint16_t* out) {
    for (int r = 0; r < m; ++r) {
        for (int c = 0; c < n; ++c) {
            size_t idx = (size_t)r * n + c;
            float v = fmaf(acc[idx], in_scale * w_scales[c], bias ? bias[c] : 0.0f);
            out[idx] = orc_f32_to_f16(activate(v, activation));
        }
    }
}

/* ---- joint (decoder.cu:690-759) ----------------------------------------- */

/* score[o] = bias[o] + sum_k W[o,k] * relu(enc[k] + pred[k]).  fp32 products
 * folded in k order (the reference folds 32 interleaved lanes; the order is
 * not reproducible, so parity is by tolerance). */
void orc_joint_scores_f16(const uint16_t* w, const float* bias, const uint16_t* enc,
                          const float* pred, int outputs, int hidden, float* scores) {
    for (int o = 0; o < outputs; ++o) {
        double s = 0.0;
        for (int t = 0; t < hidden; ++t) {
            float in = fmaxf(orc_f16_to_f32(enc[t]) + pred[t], 0.0f);
            s += (double)orc_f16_to_f32(w[(size_t)o * hidden + t]) * (double)in;
        }
        scores[o] = (float)(s + (double)bias[o]);
    }
}

/* INT8 joint head (a new format; the reference's joint is FP16,
 * decoder.cu:596-601): score[o] = bias[o] + w_scale[o] * sum_k q[o,k] * in[k]. */
void orc_joint_scores_i8(const int8_t* w, const float* w_scales, const float* bias,
                         const uint16_t* enc, const float* pred, int outputs, int hidden,
                         float* scores) {
    for (int o = 0; o < outputs; ++o) {
        double s = 0.0;
        for (int t = 0; t < hidden; ++t) {
            float in = fmaxf(orc_f16_to_f32(enc[t]) + pred[t], 0.0f);
            s += (double)w[(size_t)o * hidden + t] * (double)in;
        }
        scores[o] = (float)((double)w_scales[o] * s + (double)bias[o]);
    }
}

/* Greedy TDT decision (decoder.cu:34-46, 728-759): token = argmax over the
 * first token_outputs scores, ties to the lower id; duration = argmax over the
 * next `durations` scores with strict '>' (first maximum wins). */
void orc_joint_decide(const float* scores, int token_outputs, int durations, int* token,
                      int* duration) {
    int best = 0;
    for (int o = 1; o < token_outputs; ++o) {
        if (scores[o] > scores[best]) best = o;
    }
    int d = 0;
    for (int i = 1; i < durations; ++i) {
        if (scores[token_outputs + i] > scores[token_outputs + d]) d = i;
    }
    *token = best;
    *duration = d;
}

/* ---- TDT greedy decode (prediction network + joint) ------------------------ */

/* One LSTM layer step (decoder.cu:116-129 lstm_cell, gate rows i, f, g, o of
 * 4*hidden): gates = b_ih + b_hh + W_ih x + W_hh h (x NULL = zeros),
 * c' = sigmoid(f) c + sigmoid(i) tanh(g), h' = sigmoid(o) tanh(c'). */
void orc_lstm_step(const uint16_t* w_ih, const uint16_t* w_hh, const float* b_ih, const float* b_hh,
                   const float* x, const float* h, const float* c, int hidden, float* h_out, float* c_out) {
    for (int u = 0; u < hidden; ++u) {
        float g[4];
        for (int gate = 0; gate < 4; ++gate) {
            const size_t row = (size_t)(gate * hidden + u);
            double s = (double)b_ih[row] + (double)b_hh[row];
            for (int k = 0; k < hidden; ++k) {
                if (x) s += (double)orc_f16_to_f32(w_ih[row * hidden + k]) * (double)x[k];
                s += (double)orc_f16_to_f32(w_hh[row * hidden + k]) * (double)h[k];
            }
            g[gate] = (float)s;
        }
        const float ig = 1.0f / (1.0f + expf(-g[0]));
        const float fg = 1.0f / (1.0f + expf(-g[1]));
        const float cg = tanhf(g[2]);
        const float og = 1.0f / (1.0f + expf(-g[3]));
        const float cell = fg * c[u] + ig * cg;
        c_out[u] = cell;
        h_out[u] = og * tanhf(cell);
    }
}

/* decoder.cu:146-445 (tdt_persistent_fp16): greedy TDT decode.  The prediction
 * (2-layer LSTM on the last emitted token's embedding, zero input before the
 * first token, then projection + bias) is recomputed after each emitted token
 * and its state committed; blanks leave it unchanged.  Joint and frame rules
 * as orc_joint_scores_* / orc_joint_decide and decoder.cu:773-783.  Returns
 * the number of tokens (at most capacity are stored); pred_out = the final
 * prediction vector, *frame_out = the final frame index. */
int orc_tdt_decode(const uint16_t* enc, int frames, int enc_stride, const uint16_t* emb, const uint16_t* w_ih0,
                   const uint16_t* w_hh0, const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1,
                   const uint16_t* w_hh1, const float* b_ih1, const float* b_hh1, const uint16_t* w_proj,
                   const float* b_proj, const void* w_joint, int joint_int8, const float* joint_scales,
                   const float* b_joint, int hidden, int token_outputs, int durations, int max_symbols,
                   int32_t* tokens, int capacity, float* pred_out, int* frame_out) {
    const int outputs = token_outputs + durations, blank = token_outputs - 1;
    float* h = (float*)calloc((size_t)4 * hidden, sizeof(float));  /* committed h0, h1, c0, c1 */
    float* cand = (float*)calloc((size_t)4 * hidden, sizeof(float));
    float* x = (float*)malloc((size_t)hidden * sizeof(float));
    float* pred = (float*)calloc((size_t)hidden, sizeof(float));
    float* scores = (float*)malloc((size_t)outputs * sizeof(float));
    int frame = 0, symbols = 0, last = blank, emitted = 0, valid = 0, count = 0;
    while (frame < frames) {
        if (!valid) {
            if (emitted)
                for (int k = 0; k < hidden; ++k) x[k] = orc_f16_to_f32(emb[(size_t)last * hidden + k]);
            orc_lstm_step(w_ih0, w_hh0, b_ih0, b_hh0, emitted ? x : NULL, h, h + 2 * hidden, hidden, cand,
                          cand + 2 * hidden);
            orc_lstm_step(w_ih1, w_hh1, b_ih1, b_hh1, cand, h + hidden, h + 3 * hidden, hidden, cand + hidden,
                          cand + 3 * hidden);
            for (int o = 0; o < hidden; ++o) {
                double s = (double)b_proj[o];
                for (int k = 0; k < hidden; ++k)
                    s += (double)orc_f16_to_f32(w_proj[(size_t)o * hidden + k]) * (double)cand[hidden + k];
                pred[o] = (float)s;
            }
            valid = 1;
        }
        const uint16_t* e = enc + (size_t)frame * enc_stride;
        if (joint_int8)
            orc_joint_scores_i8((const int8_t*)w_joint, joint_scales, b_joint, e, pred, outputs, hidden, scores);
        else
            orc_joint_scores_f16((const uint16_t*)w_joint, b_joint, e, pred, outputs, hidden, scores);
        int tok, dur;
        orc_joint_decide(scores, token_outputs, durations, &tok, &dur);
        if (tok != blank) {
            if (count < capacity) tokens[count] = tok;
            ++count;
            last = tok;
            emitted = 1;
            valid = 0;
            memcpy(h, cand, (size_t)4 * hidden * sizeof(float));
        }
        ++symbols;
        frame += dur;
        if (dur != 0 || symbols == max_symbols) {
            if (dur == 0) ++frame;
            symbols = 0;
        }
    }
    memcpy(pred_out, pred, (size_t)hidden * sizeof(float));
    *frame_out = frame;
    free(h);
    free(cand);
    free(x);
    free(pred);
    free(scores);
    return count;
}

/* ---- long-request TDT decode (decoder.cu:452-784, tdt_persistent_fp8) ----- */

/* decoder.cu:95-97 quantize_i8: round to nearest even, clamp to +-127. */
static int orc_quant_i8(float v) {
    int q = (int)rintf(v);
    return q < -127 ? -127 : (q > 127 ? 127 : q);
}

/* decoder.cu:520-575: per-tensor symmetric INT8 of an fp16 matrix of n
 * elements: scale = max|w| / 127 (1 when every element is zero), q =
 * quantize_i8(w / scale).  Returns the scale. */
float orc_quantize_tensor_i8(const uint16_t* w, size_t n, int8_t* q) {
    float m = 0.0f;
    for (size_t i = 0; i < n; ++i) m = fmaxf(m, fabsf(orc_f16_to_f32(w[i])));
    const float scale = m > 0.0f ? m / 127.0f : 1.0f;
    for (size_t i = 0; i < n; ++i) q[i] = (int8_t)orc_quant_i8(orc_f16_to_f32(w[i]) / scale);
    return scale;
}

/* Integer dot product of INT8 row r of a [4H x H] matrix with an INT8 vector. */
static int orc_dot_i8(const int8_t* q, int row, const int8_t* x, int hidden) {
    int acc = 0;
    for (int k = 0; k < hidden; ++k) acc += (int)q[(size_t)row * hidden + k] * (int)x[k];
    return acc;
}

/* exp(x) from IEEE basic operations (the long form's cell arithmetic, which
 * the GPU evaluates operation for operation): Cody-Waite reduction x = n ln2
 * + r with ln2 split into a 16-bit head and a tail, e^r by its degree-7
 * Taylor polynomial, times 2^n.  Within 0.82 ulp of exp on [-87, 88]. */
float orc_det_exp(float x) {
    if (x != x) return x;
    x = fminf(fmaxf(x, -104.0f), 89.0f);
    const float n = rintf(x * 1.44269504f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.428606765330187e-06f, r);
    float q = 1.98412698e-04f;
    q = fmaf(q, r, 1.38888889e-03f);
    q = fmaf(q, r, 8.33333333e-03f);
    q = fmaf(q, r, 4.16666667e-02f);
    q = fmaf(q, r, 1.66666667e-01f);
    q = fmaf(q, r, 0.5f);
    q = fmaf(q, r, 1.0f);
    q = fmaf(q, r, 1.0f);
    return ldexpf(q, (int)n);
}

/* tanh(x) = sign(x) (1 - e^-2|x|) / (1 + e^-2|x|). */
float orc_det_tanh(float v) {
    const float t = orc_det_exp(-2.0f * fabsf(v));
    return copysignf((1.0f - t) / (1.0f + t), v);
}

/* decoder.cu:116-129 lstm_cell with orc_det_exp / orc_det_tanh and the cell
 * update as fma(f, c, i * g). */
static void orc_cell(const float s[4], float c_prev, float* c_out, float* h_out) {
    const float ig = 1.0f / (1.0f + orc_det_exp(-s[0]));
    const float fg = 1.0f / (1.0f + orc_det_exp(-s[1]));
    const float cg = orc_det_tanh(s[2]);
    const float og = 1.0f / (1.0f + orc_det_exp(-s[3]));
    *c_out = fmaf(fg, c_prev, ig * cg);
    *h_out = og * orc_det_tanh(*c_out);
}

/* One prediction-network update of the long form (decoder.cu:613-672).
 * q_hh0, q_hh1, q_ih1: INT8 [4H x H]; cq[3] = their scale / 127; bias[2][4H] =
 * b_ih + b_hh per layer; qh (committed INT8 h of layers 0, 1, [2][H]) and c
 * ([2][H]) are the committed state; table_row = the last token's
 * [4H] fp16 input terms or NULL before the first token.  Writes the
 * candidate INT8 h (qh_out [2][H]), cell states (c_out [2][H]) and layer-1
 * output (h1_out [H]).  Gate sums: layer 0 fma(dot, cq0, bias) + table,
 * layer 1 fma(dot_ih1, cq2, fma(dot_hh1, cq1, bias)); each integer dot is
 * exact and converted once. */
void orc_lstm_long_update(const int8_t* q_hh0, const int8_t* q_hh1, const int8_t* q_ih1, const float* cq,
                          const float* bias, const uint16_t* table_row, const int8_t* qh, const float* c, int hidden,
                          int8_t* qh_out, float* c_out, float* h1_out) {
    for (int u = 0; u < hidden; ++u) {
        float s[4], h;
        for (int g = 0; g < 4; ++g) {
            const int row = g * hidden + u;
            const float tv = table_row ? orc_f16_to_f32(table_row[row]) : 0.0f;
            s[g] = fmaf((float)orc_dot_i8(q_hh0, row, qh, hidden), cq[0], bias[row]) + tv;
        }
        orc_cell(s, c[u], &c_out[u], &h);
        qh_out[u] = (int8_t)orc_quant_i8(h * 127.0f);
    }
    for (int u = 0; u < hidden; ++u) {
        float s[4];
        for (int g = 0; g < 4; ++g) {
            const int row = g * hidden + u;
            const float rec = fmaf((float)orc_dot_i8(q_hh1, row, qh + hidden, hidden), cq[1], bias[4 * hidden + row]);
            s[g] = fmaf((float)orc_dot_i8(q_ih1, row, qh_out, hidden), cq[2], rec);
        }
        orc_cell(s, c[hidden + u], &c_out[hidden + u], &h1_out[u]);
        qh_out[hidden + u] = (int8_t)orc_quant_i8(h1_out[u] * 127.0f);
    }
}

/* decoder.cu:452-784 (tdt_persistent_fp8): the greedy decode of
 * orc_tdt_decode with the long-request prediction network: per-tensor INT8
 * W_hh0, W_hh1, W_ih1 (orc_quantize_tensor_i8), INT8 hidden states at 1/127,
 * layer-0 input terms from input_table [(token_outputs - 1) x 4H] fp16, fp32
 * cells, the projection of the fp32 layer-1 output.  The zero state and no
 * input before the first token; the candidate state is committed when a token
 * is emitted.  Returns the token count; pred_out, *frame_out as
 * orc_tdt_decode. */
int orc_tdt_decode_long(const uint16_t* enc, int frames, int enc_stride, const uint16_t* table, const uint16_t* w_hh0,
                        const float* b_ih0, const float* b_hh0, const uint16_t* w_ih1, const uint16_t* w_hh1,
                        const float* b_ih1, const float* b_hh1, const uint16_t* w_proj, const float* b_proj,
                        const void* w_joint, int joint_int8, const float* joint_scales, const float* b_joint, int hidden,
                        int token_outputs, int durations, int max_symbols, int32_t* tokens, int capacity,
                        float* pred_out, int* frame_out) {
    const int H = hidden, outputs = token_outputs + durations, blank = token_outputs - 1;
    const size_t n = (size_t)4 * H * H;
    int8_t* q = (int8_t*)malloc(3 * n);
    float cq[3];
    cq[0] = orc_quantize_tensor_i8(w_hh0, n, q) / 127.0f;
    cq[1] = orc_quantize_tensor_i8(w_hh1, n, q + n) / 127.0f;
    cq[2] = orc_quantize_tensor_i8(w_ih1, n, q + 2 * n) / 127.0f;
    float* bias = (float*)malloc((size_t)8 * H * sizeof(float));
    for (int i = 0; i < 4 * H; ++i) {
        bias[i] = b_ih0[i] + b_hh0[i];
        bias[4 * H + i] = b_ih1[i] + b_hh1[i];
    }
    int8_t* qh = (int8_t*)calloc((size_t)2 * H, 1);
    int8_t* qh_cand = (int8_t*)calloc((size_t)2 * H, 1);
    float* c = (float*)calloc((size_t)2 * H, sizeof(float));
    float* c_cand = (float*)calloc((size_t)2 * H, sizeof(float));
    float* h1 = (float*)calloc((size_t)H, sizeof(float));
    float* pred = (float*)calloc((size_t)H, sizeof(float));
    float* scores = (float*)malloc((size_t)outputs * sizeof(float));
    int frame = 0, symbols = 0, last = blank, emitted = 0, valid = 0, count = 0;
    while (frame < frames) {
        if (!valid) {
            orc_lstm_long_update(q, q + n, q + 2 * n, cq, bias, emitted ? table + (size_t)last * 4 * H : NULL, qh, c, H,
                                 qh_cand, c_cand, h1);
            for (int o = 0; o < H; ++o) {
                double s = (double)b_proj[o];
                for (int k = 0; k < H; ++k) s += (double)orc_f16_to_f32(w_proj[(size_t)o * H + k]) * (double)h1[k];
                pred[o] = (float)s;
            }
            valid = 1;
        }
        const uint16_t* e = enc + (size_t)frame * enc_stride;
        if (joint_int8)
            orc_joint_scores_i8((const int8_t*)w_joint, joint_scales, b_joint, e, pred, outputs, H, scores);
        else
            orc_joint_scores_f16((const uint16_t*)w_joint, b_joint, e, pred, outputs, H, scores);
        int tok, dur;
        orc_joint_decide(scores, token_outputs, durations, &tok, &dur);
        if (tok != blank) {
            if (count < capacity) tokens[count] = tok;
            ++count;
            last = tok;
            emitted = 1;
            valid = 0;
            memcpy(qh, qh_cand, (size_t)2 * H);
            memcpy(c, c_cand, (size_t)2 * H * sizeof(float));
        }
        ++symbols;
        frame += dur;
        if (dur != 0 || symbols == max_symbols) {
            if (dur == 0) ++frame;
            symbols = 0;
        }
    }
    memcpy(pred_out, pred, (size_t)H * sizeof(float));
    *frame_out = frame;
    free(q);
    free(bias);
    free(qh);
    free(qh_cand);
    free(c);
    free(c_cand);
    free(h1);
    free(pred);
    free(scores);
    return count;
}

/* ======================================================================== */
/* Local relative-position attention and its packers                        */
/* (encoder.cu:1476-2097, launch_attention_arena encoder.rs:1839-1968).      */
/* Model constants: width 1024, 8 heads of 128, position rows padded to 272 */
/* (encoder.cu:12-17), window 128 left / 128 right (encoder.rs:24-26).       */
/* ======================================================================== */

#define ORC_MODEL 1024
#define ORC_HEAD 128
#define ORC_HEADS 8
#define ORC_MAXATT 257
#define ORC_POSROWS 272
#define ORC_FP8ROWS 288

/* bf16 round to nearest even of a finite float (__float2bfloat16_rn). */
static float round_bf16(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
    float r;
    memcpy(&r, &b, 4);
    return r;
}

/* Storage byte of dimension d in an INT8 score vector: the byte written by
 * pk_sm89_pack_score_vectors (encoder.cu:2054-2074), lane = d / 4 stores its
 * four bytes at (lane/8)*32 + (lane%4)*8 + (lane&4). */
int orc_score_vector_byte(int d) {
    const int lane = d / 4;
    return (lane / 8) * 32 + (lane % 4) * 8 + (lane & 4) + d % 4;
}

/* Storage nibble of dimension d in an INT4 key vector: lane = d / 4 stores a
 * u16 of four nibbles at byte (lane/16)*32 + ((lane/2)%4)*8 + ((lane/2)&4) +
 * (lane&1)*2 (pk_sm89_pack_key_int4, encoder.cu:2076-2097). */
int orc_key_int4_nibble(int d) {
    const int lane = d / 4;
    const int byte = (lane / 16) * 32 + ((lane / 2) % 4) * 8 + ((lane / 2) & 4) + (lane & 1) * 2;
    return 2 * byte + d % 4;
}

/* encoder.cu:2054-2074: per 128-value vector, scale = max|v|/127 (1 if the
 * vector is zero), byte = (uint8)rn(v/scale), stored in the MMA byte order. */
void orc_pack_score_vectors(const uint16_t* in, int vectors, uint8_t* out, float* scales) {
    for (int vec = 0; vec < vectors; ++vec) {
        const uint16_t* x = in + (size_t)vec * 128;
        float m = 0.0f;
        for (int d = 0; d < 128; ++d) m = fmaxf(m, fabsf(orc_f16_to_f32(x[d])));
        const float scale = m > 0.0f ? m / 127.0f : 1.0f;
        scales[vec] = scale;
        for (int d = 0; d < 128; ++d)
            out[(size_t)vec * 128 + orc_score_vector_byte(d)] = (uint8_t)(int)rintf(orc_f16_to_f32(x[d]) / scale);
    }
}

/* encoder.cu:2076-2097: per vector, scale = max|v|/7, nibble = rn(v/scale)&15,
 * 64 bytes per vector in the MMA nibble order. */
void orc_pack_key_int4(const uint16_t* in, int vectors, uint8_t* out, float* scales) {
    for (int vec = 0; vec < vectors; ++vec) {
        const uint16_t* x = in + (size_t)vec * 128;
        uint8_t* o = out + (size_t)vec * 64;
        float m = 0.0f;
        for (int d = 0; d < 128; ++d) m = fmaxf(m, fabsf(orc_f16_to_f32(x[d])));
        const float scale = m > 0.0f ? m / 7.0f : 1.0f;
        scales[vec] = scale;
        memset(o, 0, 64);
        for (int d = 0; d < 128; ++d) {
            const int q = (int)rintf(orc_f16_to_f32(x[d]) / scale) & 15;
            const int s = orc_key_int4_nibble(d);
            o[s / 2] |= (uint8_t)(q << (4 * (s & 1)));
        }
    }
}

/* encoder.cu:561-634 pk_sm89_quantize_value_int4{,_register}.  Input V is
 * feature-major [1024 x rows] fp16.  Output: FP8 V (e4m3(v*inverse_scale))
 * [1024 x rows], then S4 V (clamp(rn(v/s_f), -7, 7), two keys per byte, even
 * key in the low nibble), then 1024 float scales s_f = max|V_f|/7 (1 when
 * zero).  With edge_only the FP8 copy is written only for row pairs with
 * row < 272 or row + 1 >= valid_rows - 272 (the register variant). */
void orc_quantize_value_int4(const uint16_t* vt, int rows, float inverse_scale, int edge_only, int valid_rows,
                             uint8_t* out) {
    const size_t elements = (size_t)rows * ORC_MODEL;
    float* scales = (float*)(out + elements + elements / 2);
    for (int f = 0; f < ORC_MODEL; ++f) {
        const uint16_t* x = vt + (size_t)f * rows;
        float m = 0.0f;
        for (int r = 0; r < rows; ++r) m = fmaxf(m, fabsf(orc_f16_to_f32(x[r])));
        const float scale = m > 0.0f ? m / 7.0f : 1.0f;
        scales[f] = scale;
        for (int r = 0; r + 1 < rows; r += 2) {
            const float a = orc_f16_to_f32(x[r]), b = orc_f16_to_f32(x[r + 1]);
            if (!edge_only || r < 272 || r + 1 >= valid_rows - 272) {
                out[(size_t)f * rows + r] = orc_f32_to_e4m3(a * inverse_scale);
                out[(size_t)f * rows + r + 1] = orc_f32_to_e4m3(b * inverse_scale);
            }
            int qa = (int)rintf(a / scale), qb = (int)rintf(b / scale);
            qa = qa < -7 ? -7 : (qa > 7 ? 7 : qa);
            qb = qb < -7 ? -7 : (qb > 7 ? 7 : qb);
            out[elements + ((size_t)f * rows + r) / 2] = (uint8_t)((qa & 15) | ((qb & 15) << 4));
        }
    }
}

static int sext4(int v) { return (v & 8) ? (v & 15) - 16 : (v & 15); }

/* Output store of the attention kernels (encoder.cu:1463-1474): the context is
 * rounded to fp16; the packed form stores e4m3(fp16 * 28). */
static void store_context(int packed, void* output, size_t index, float value) {
    const uint16_t h = orc_f32_to_f16(value);
    if (packed)
        ((uint8_t*)output)[index] = orc_f32_to_e4m3(orc_f16_to_f32(h) * 28.0f);
    else
        ((uint16_t*)output)[index] = h;
}

/* The per-query FP32 path every boundary tile takes (encoder.cu:1548-1684).
 * Reduction orders follow the 32-lane warp: lane pairs of 16 accumulate a
 * score over dimensions 2*l + 32*quarter with interleaved content/position
 * FMAs, then a shuffle-down tree over 16 lanes; denominators sum slots
 * l, l+32, ... per lane, then a shuffle-down tree over 32 lanes. */
static void attention_scalar_row(int packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                                 const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output,
                                 int head, int qr, int rows, int padded_rows, int valid_rows, int left, int right,
                                 int value_stride, float* scores) {
    if (qr >= rows || qr >= valid_rows) {
        if (qr < padded_rows)
            for (int d = 0; d < ORC_HEAD; ++d) store_context(packed, output, (size_t)qr * ORC_MODEL + head * ORC_HEAD + d, 0.0f);
        return;
    }
    const int first = qr - left > 0 ? qr - left : 0;
    const int last = qr + right < valid_rows - 1 ? qr + right : valid_rows - 1;
    const int count = last - first + 1;
    const size_t qh = (size_t)qr * ORC_MODEL + head * ORC_HEAD;
    float su[ORC_HEAD], sv[ORC_HEAD];
    for (int d = 0; d < ORC_HEAD; ++d) {
        const float q = orc_f16_to_f32(query[qh + d]);
        su[d] = q + orc_f16_to_f32(bias_u[head * ORC_HEAD + d]);
        sv[d] = q + orc_f16_to_f32(bias_v[head * ORC_HEAD + d]);
    }
    for (int slot = 0; slot < count; ++slot) {
        const int key_row = first + slot;
        const int prow = left - qr + key_row;
        const uint16_t* k = key + (size_t)key_row * ORC_MODEL + head * ORC_HEAD;
        const uint16_t* p = position + ((size_t)head * ORC_POSROWS + prow) * ORC_HEAD;
        float part[16];
        for (int l = 0; l < 16; ++l) {
            float s = 0.0f;
            for (int quarter = 0; quarter < 4; ++quarter) {
                const int d = 2 * l + 32 * quarter;
                s = fmaf(su[d], orc_f16_to_f32(k[d]), s);
                s = fmaf(sv[d], orc_f16_to_f32(p[d]), s);
                s = fmaf(su[d + 1], orc_f16_to_f32(k[d + 1]), s);
                s = fmaf(sv[d + 1], orc_f16_to_f32(p[d + 1]), s);
            }
            part[l] = s;
        }
        for (int off = 8; off > 0; off /= 2)
            for (int l = 0; l < off; ++l) part[l] = part[l] + part[l + off];
        scores[slot] = part[0] * 0.08838834764831845f;
    }
    float maximum = -FLT_MAX;
    for (int slot = 0; slot < count; ++slot) maximum = fmaxf(maximum, scores[slot]);
    float lane_sum[32];
    for (int l = 0; l < 32; ++l) lane_sum[l] = 0.0f;
    for (int slot = 0; slot < count; ++slot) {
        scores[slot] = expf(scores[slot] - maximum);
        lane_sum[slot % 32] += scores[slot];
    }
    for (int off = 16; off > 0; off /= 2)
        for (int l = 0; l < off; ++l) lane_sum[l] = lane_sum[l] + lane_sum[l + off];
    const float denominator = lane_sum[0];
    const float value_scale = 8.0f / 448.0f;
    for (int d = 0; d < ORC_HEAD; ++d) {
        const int feature = head * ORC_HEAD + d;
        float context = 0.0f;
        for (int key_row = first; key_row <= last; ++key_row) {
            const float weight = scores[key_row - first] / denominator;
            const float value = orc_e4m3_to_f32(value_fp8[(size_t)feature * value_stride + key_row]) * value_scale;
            context = fmaf(weight, value, context);
        }
        store_context(packed, output, qh + d, context);
    }
}

/* Interior tile of pk_sm89_local_relpos_attention_packed (encoder.cu:1687-1966):
 * 16 queries qb..qb+15 share keys qb-128 .. qb+143.  q+u is quantized per
 * query to INT4 (max/7) against the INT4 keys, q+v to INT8 (max/127) against
 * the INT8 position vectors; each integer score is scaled by both scales and
 * rounded to bf16; softmax in FP32; probabilities quantized to U4 (rn(e*15),
 * scale 1/(15*denominator)); context = sum U4 * S4(V) times the probability
 * and per-feature value scales, rounded to fp16 and stored as e4m3(x*28). */
static void attention_packed_tile(const uint16_t* query, const uint8_t* value_fp8, const uint16_t* bias_u,
                                  const uint16_t* bias_v, uint8_t* output, int head, int qb, int value_stride,
                                  const uint8_t* packed_key, const float* key_scales, const uint8_t* packed_position,
                                  const float* position_scales) {
    const int first_key = qb - 128;
    int qu[16][ORC_HEAD], qv[16][ORC_HEAD];
    float su[16], sv[16];
    for (int r = 0; r < 16; ++r) {
        float vals[2][ORC_HEAD], mx[2] = {0.0f, 0.0f};
        for (int d = 0; d < ORC_HEAD; ++d) {
            const float q = orc_f16_to_f32(query[(size_t)(qb + r) * ORC_MODEL + head * ORC_HEAD + d]);
            vals[0][d] = round_f16(q + orc_f16_to_f32(bias_u[head * ORC_HEAD + d]));
            vals[1][d] = round_f16(q + orc_f16_to_f32(bias_v[head * ORC_HEAD + d]));
            mx[0] = fmaxf(mx[0], fabsf(vals[0][d]));
            mx[1] = fmaxf(mx[1], fabsf(vals[1][d]));
        }
        su[r] = mx[0] > 0.0f ? mx[0] / 7.0f : 1.0f;
        sv[r] = mx[1] > 0.0f ? mx[1] / 127.0f : 1.0f;
        for (int d = 0; d < ORC_HEAD; ++d) {
            qu[r][d] = sext4((int)rintf(vals[0][d] / su[r]));
            qv[r][d] = (int8_t)(uint8_t)(int)rintf(vals[1][d] / sv[r]);
        }
    }
    static float content[16][ORC_POSROWS], pos[16][ORC_POSROWS];
#pragma omp threadprivate(content, pos)
    for (int col = 0; col < ORC_POSROWS; ++col) {
        const int kvec = (first_key + col) * ORC_HEADS + head;
        const int pvec = head * ORC_POSROWS + col;
        int kd[ORC_HEAD], pd[ORC_HEAD];
        for (int d = 0; d < ORC_HEAD; ++d) {
            const int s = orc_key_int4_nibble(d);
            kd[d] = sext4(packed_key[(size_t)kvec * 64 + s / 2] >> (4 * (s & 1)));
            pd[d] = (int8_t)packed_position[(size_t)pvec * 128 + orc_score_vector_byte(d)];
        }
        for (int r = 0; r < 16; ++r) {
            int32_t a = 0, b = 0;
            for (int d = 0; d < ORC_HEAD; ++d) {
                a += qu[r][d] * kd[d];
                b += qv[r][d] * pd[d];
            }
            content[r][col] = round_bf16((float)a * (su[r] * key_scales[kvec]));
            pos[r][col] = round_bf16((float)b * (sv[r] * position_scales[pvec]));
        }
    }
    int prob[16][ORC_POSROWS];
    float prob_scale[16];
    for (int r = 0; r < 16; ++r) {
        float e[ORC_MAXATT], maximum = -FLT_MAX;
        for (int slot = 0; slot < ORC_MAXATT; ++slot) {
            e[slot] = (content[r][r + slot] + pos[r][slot]) * 0.08838834764831845f;
            maximum = fmaxf(maximum, e[slot]);
        }
        float lane_sum[32];
        for (int l = 0; l < 32; ++l) lane_sum[l] = 0.0f;
        for (int slot = 0; slot < ORC_MAXATT; ++slot) {
            e[slot] = expf(e[slot] - maximum);
            lane_sum[slot % 32] += e[slot];
        }
        for (int off = 16; off > 0; off /= 2)
            for (int l = 0; l < off; ++l) lane_sum[l] = lane_sum[l] + lane_sum[l + off];
        prob_scale[r] = 1.0f / (15.0f * lane_sum[0]);
        for (int k = 0; k < ORC_POSROWS; ++k) prob[r][k] = 0;
        for (int slot = 0; slot < ORC_MAXATT; ++slot) prob[r][r + slot] = (int)rintf(e[slot] * 15.0f);
    }
    const uint8_t* s4 = value_fp8 + (size_t)ORC_MODEL * value_stride;
    const float* vscales = (const float*)(value_fp8 + (size_t)ORC_MODEL * value_stride * 3 / 2);
    for (int d = 0; d < ORC_HEAD; ++d) {
        const int feature = head * ORC_HEAD + d;
        int v[ORC_POSROWS];
        for (int k = 0; k < ORC_POSROWS; ++k) {
            const size_t nib = (size_t)feature * value_stride + first_key + k;
            v[k] = sext4(s4[nib / 2] >> (4 * (nib & 1)));
        }
        for (int r = 0; r < 16; ++r) {
            int32_t acc = 0;
            for (int k = 0; k < ORC_POSROWS; ++k) acc += prob[r][k] * v[k];
            const float out = (float)acc * (prob_scale[r] * vscales[feature]);
            store_context(1, output, (size_t)(qb + r) * ORC_MODEL + feature, out);
        }
    }
}

/* Interior tile of pk_sm89_local_relpos_attention_tc_scores (encoder.cu:
 * 1768-2018): q+u and q+v rounded to fp16; FP32 dot products with fp16 K and
 * position rows; softmax; probabilities e4m3(p*448); context = sum e4m3(p) *
 * e4m3(V) over keys qb-128 .. qb+143, times (1/448)*(8/448), stored as fp16.
 * The tensor-core accumulation order is unspecified; this sums in k order. */
static void attention_tc_tile(const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                              const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, uint16_t* output,
                              int head, int qb, int value_stride) {
    const int first_key = qb - 128;
    static float qu[16][ORC_HEAD], qv[16][ORC_HEAD], content[16][ORC_POSROWS], pos[16][ORC_POSROWS];
#pragma omp threadprivate(qu, qv, content, pos)
    for (int r = 0; r < 16; ++r)
        for (int d = 0; d < ORC_HEAD; ++d) {
            const float q = orc_f16_to_f32(query[(size_t)(qb + r) * ORC_MODEL + head * ORC_HEAD + d]);
            qu[r][d] = round_f16(q + orc_f16_to_f32(bias_u[head * ORC_HEAD + d]));
            qv[r][d] = round_f16(q + orc_f16_to_f32(bias_v[head * ORC_HEAD + d]));
        }
    for (int col = 0; col < ORC_POSROWS; ++col) {
        const uint16_t* k = key + (size_t)(first_key + col) * ORC_MODEL + head * ORC_HEAD;
        const uint16_t* p = position + ((size_t)head * ORC_POSROWS + col) * ORC_HEAD;
        for (int r = 0; r < 16; ++r) {
            float a = 0.0f, b = 0.0f;
            for (int d = 0; d < ORC_HEAD; ++d) {
                a += qu[r][d] * orc_f16_to_f32(k[d]);
                b += qv[r][d] * orc_f16_to_f32(p[d]);
            }
            content[r][col] = a;
            pos[r][col] = b;
        }
    }
    uint8_t prob[16][ORC_FP8ROWS];
    for (int r = 0; r < 16; ++r) {
        float e[ORC_MAXATT], maximum = -FLT_MAX;
        for (int slot = 0; slot < ORC_MAXATT; ++slot) {
            e[slot] = (content[r][r + slot] + pos[r][slot]) * 0.08838834764831845f;
            maximum = fmaxf(maximum, e[slot]);
        }
        float lane_sum[32];
        for (int l = 0; l < 32; ++l) lane_sum[l] = 0.0f;
        for (int slot = 0; slot < ORC_MAXATT; ++slot) {
            e[slot] = expf(e[slot] - maximum);
            lane_sum[slot % 32] += e[slot];
        }
        for (int off = 16; off > 0; off /= 2)
            for (int l = 0; l < off; ++l) lane_sum[l] = lane_sum[l] + lane_sum[l + off];
        const float denominator = lane_sum[0];
        for (int u = 0; u < ORC_FP8ROWS; ++u) {
            const int in_window = u >= r && u < r + ORC_MAXATT;
            prob[r][u] = orc_f32_to_e4m3((in_window ? e[u - r] / denominator : 0.0f) * 448.0f);
        }
    }
    const float context_scale = (1.0f / 448.0f) * (8.0f / 448.0f);
    for (int d = 0; d < ORC_HEAD; ++d) {
        const int feature = head * ORC_HEAD + d;
        float v[ORC_POSROWS];
        for (int k = 0; k < ORC_POSROWS; ++k)
            v[k] = orc_e4m3_to_f32(value_fp8[(size_t)feature * value_stride + first_key + k]);
        for (int r = 0; r < 16; ++r) {
            float acc = 0.0f;
            for (int k = 0; k < ORC_POSROWS; ++k) acc += orc_e4m3_to_f32(prob[r][k]) * v[k];
            output[(size_t)(qb + r) * ORC_MODEL + feature] = orc_f32_to_f16(acc * context_scale);
        }
    }
}

/* Both long-form attention kernels over query tiles [tile_begin, tile_end) of
 * 16 rows and all 8 heads.  packed != 0: pk_sm89_local_relpos_attention_packed
 * (output e4m3 bytes); packed == 0: pk_sm89_local_relpos_attention_tc_scores
 * (output fp16).  Tiles with qb >= left, qb + 15 + right < valid_rows and
 * qb + 16 <= rows take the tile path; all others the per-query path. */
void orc_local_attention(int packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                         const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output, int rows,
                         int padded_rows, int valid_rows, int left, int right, int value_stride,
                         const uint8_t* packed_key, const float* key_scales, const uint8_t* packed_position,
                         const float* position_scales, int tile_begin, int tile_end) {
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int tile = tile_begin; tile < tile_end; ++tile)
        for (int head = 0; head < ORC_HEADS; ++head) {
            const int qb = 16 * tile;
            if (qb >= padded_rows) continue;
            const int interior = qb >= left && qb + 15 + right < valid_rows && qb + 16 <= rows;
            if (!interior) {
                float scores[1024];
                for (int r = 0; r < 16; ++r)
                    attention_scalar_row(packed, query, key, value_fp8, position, bias_u, bias_v, output, head, qb + r,
                                         rows, padded_rows, valid_rows, left, right, value_stride, scores);
            } else if (packed) {
                attention_packed_tile(query, value_fp8, bias_u, bias_v, (uint8_t*)output, head, qb, value_stride,
                                      packed_key, key_scales, packed_position, position_scales);
            } else {
                attention_tc_tile(query, key, value_fp8, position, bias_u, bias_v, (uint16_t*)output, head, qb,
                                  value_stride);
            }
        }
}

/* ---- short-form attention and attention-side layouts ---------------------- */

/* encoder.cu:644-671: out[f * rows + r] = e4m3(in[r * 1024 + f] * inverse_scale). */
void orc_quantize_fp8_transpose(const uint16_t* in, int rows, float inverse_scale, uint8_t* out) {
    for (int r = 0; r < rows; ++r)
        for (int f = 0; f < ORC_MODEL; ++f)
            out[(size_t)f * rows + r] = orc_f32_to_e4m3(orc_f16_to_f32(in[(size_t)r * ORC_MODEL + f]) * inverse_scale);
}

/* encoder.cu:1321-1336: [272 x 1024] -> [8 heads x 272 x 128]. */
void orc_pack_position_heads(const uint16_t* in, uint16_t* out) {
    for (int p = 0; p < ORC_POSROWS; ++p)
        for (int h = 0; h < ORC_HEADS; ++h)
            memcpy(out + ((size_t)h * ORC_POSROWS + p) * ORC_HEAD, in + (size_t)p * ORC_MODEL + h * ORC_HEAD,
                   ORC_HEAD * sizeof(uint16_t));
}

/* encoder.cu:1338-1461 pk_sm89_local_relpos_attention: for query r < min(rows,
 * valid_rows) and head h, keys first = max(0, r - left) .. min(valid - 1, r +
 * right); score = ((q + u).k + (q + v).p[left - r + key]) / sqrt(128) with
 * q + u, q + v formed in float and the dot products summed in double (the
 * reference's lane order is not reproducible); probabilities expf(s - max) /
 * their sum; context = fmaf over keys in order, rounded to fp16.  Other rows
 * are zero.  position = packed [8 x 272 x 128]. */
void orc_local_attention_short(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* pos,
                               const uint16_t* bu, const uint16_t* bv, uint16_t* out, int rows, int padded_rows,
                               int valid_rows, int left, int right) {
#pragma omp parallel for schedule(dynamic, 4) num_threads(orc_threads())
    for (int r = 0; r < padded_rows; ++r) {
        float sc[ORC_MAXATT];
        for (int h = 0; h < ORC_HEADS; ++h) {
            uint16_t* o = out + (size_t)r * ORC_MODEL + h * ORC_HEAD;
            if (r >= rows || r >= valid_rows) {
                memset(o, 0, ORC_HEAD * sizeof(uint16_t));
                continue;
            }
            const int first = r - left > 0 ? r - left : 0;
            const int last = r + right < valid_rows - 1 ? r + right : valid_rows - 1;
            const int count = last - first + 1;
            float qu[ORC_HEAD], qv[ORC_HEAD];
            for (int d = 0; d < ORC_HEAD; ++d) {
                const float qf = orc_f16_to_f32(q[(size_t)r * ORC_MODEL + h * ORC_HEAD + d]);
                qu[d] = qf + orc_f16_to_f32(bu[h * ORC_HEAD + d]);
                qv[d] = qf + orc_f16_to_f32(bv[h * ORC_HEAD + d]);
            }
            float mx = -FLT_MAX;
            for (int slot = 0; slot < count; ++slot) {
                const int key = first + slot, prow = left - r + key;
                double s = 0.0;
                for (int d = 0; d < ORC_HEAD; ++d) {
                    s += (double)qu[d] * orc_f16_to_f32(k[(size_t)key * ORC_MODEL + h * ORC_HEAD + d]);
                    s += (double)qv[d] * orc_f16_to_f32(pos[((size_t)h * ORC_POSROWS + prow) * ORC_HEAD + d]);
                }
                sc[slot] = (float)s * 0.08838834764831845f;
                mx = fmaxf(mx, sc[slot]);
            }
            double den = 0.0;
            for (int slot = 0; slot < count; ++slot) {
                sc[slot] = expf(sc[slot] - mx);
                den += sc[slot];
            }
            const float denf = (float)den;
            for (int d = 0; d < ORC_HEAD; ++d) {
                float c = 0.0f;
                for (int slot = 0; slot < count; ++slot)
                    c = fmaf(sc[slot] / denf, orc_f16_to_f32(v[(size_t)(first + slot) * ORC_MODEL + h * ORC_HEAD + d]), c);
                o[d] = orc_f32_to_f16(c);
            }
        }
    }
}

