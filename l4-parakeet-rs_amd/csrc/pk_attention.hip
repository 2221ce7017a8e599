// Long-form local relative-position attention of the Conformer encoder and
// the producers of its packed operands (encoder.cu:561-634, :1476-2097).
//
// Model constants (encoder.cu:12-17): width 1024 = 8 heads x 128, window
// 128 left / 128 right (257 keys), position table padded to 272 rows.
//
// A workgroup (256 threads, four waves) owns one 16-query tile of one head.
// Tiles whose whole key window lies inside [0, valid_rows) run the tile path:
// every 16 queries share the 272-key union qb-128 .. qb+143, so the scores
// are two 16x272 MFMA products (content q+u against the keys, position q+v
// against the 272 position rows) and the context is one 16x272x128 product.
//   packed: q+u -> INT4, keys INT4, q+v -> INT8, positions INT8, all on
//           v_mfma_i32_16x16x64_i8 (signed nibbles are widened to the high
//           half of a byte, i.e. times 16, and the exact sums shifted back);
//           U4 probabilities x S4 values on the same instruction.
//   tc:     fp16 scores on v_mfma_f32_16x16x32_f16; e4m3 probabilities x
//           e4m3 values on v_mfma_scale_f32_16x16x128_f8f6f4.
// Boundary tiles run the per-query FP32 path: one 32-lane half wave per
// query, with the score, maximum and denominator reductions in the order of
// the reference's 32-lane warps.
//
// The MFMA reduction dimension may be permuted freely as long as both
// operands use the same permutation (integer sums are exact).  The key and
// position vectors keep the byte order of the reference packers so that the
// packed buffers are interchangeable; the queries are quantized inside the
// kernel directly into the matching operand order.
#include <float.h>

#include "pk_common.hpp"
#include "pk_kernels.hpp"

namespace pk {
namespace {

constexpr int kModel = 1024, kHead = 128, kHeads = 8;
constexpr int kMaxAtt = 257, kPosRows = 272;
constexpr float kScoreScale = 0.08838834764831845f;  // 1/sqrt(128)
constexpr float kValueScale = 8.0f / 448.0f;         // FP8 V holds v * 56

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The reference builds encoder.cu with --use_fast_math (build.rs:68-73, :101-103), so
// the softmax exponentials of its tensor-core paths are the hardware's
// approximate exponential, not the correctly rounded expf; HIP's __expf is
// the same kind of function here (v_exp_f32 of x * log2(e)).
__device__ __forceinline__ float softmax_exp(float x) { return __expf(x); }

__device__ __forceinline__ uint16_t bf16_rn(float v) {  // finite inputs only
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// Two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rn(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// rint(v / s) for the IEEE quotient with |v / s| <= 127.5, from v * rcp(s):
// v_rcp_f32 is within 1 ulp of 1/s, so the product is within 3.1e-5 of the
// rounded quotient and both round to the same integer unless the product
// lies within 5e-5 of a half-integer.  quant8 returns rint(v * rcp(s)) and
// flags the lanes that must divide instead.
__device__ __forceinline__ float quant_fast(float v, float inv_s, bool& tie) {
    const float r = v * inv_s;
    const float t = __builtin_rintf(r);
    tie = tie || __builtin_fabsf(r - t) > 0.49995f;
    return t;
}
// rint(v[i] / s) for n values of one lane (|v / s| <= 127.5): the product
// form, then, if any lane of the wave met a near-tie, the IEEE quotient for
// those values (a wave-uniform branch, so the division is rarely executed).
template <int N>
__device__ __forceinline__ void quant_n(const float (&v)[N], float s, float (&q)[N]) {
    const float inv = __builtin_amdgcn_rcpf(s);
    bool tie = false;
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = quant_fast(v[i], inv, tie);
    if (__builtin_amdgcn_ballot_w64(tie) != 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) q[i] = __builtin_rintf(v[i] / s);
    }
}

// Four integer-valued floats in [-128, 127] -> four int8 bytes.
__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d) {
    return ((uint32_t)(int)a & 255u) | (((uint32_t)(int)b & 255u) << 8) | (((uint32_t)(int)c & 255u) << 16) |
           ((uint32_t)(int)d << 24);
}
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
// Integers n with |n| < 2^22 and the float 1.5 * 2^23 + n share bits: the
// float's bits are 0x4B400000 + n.  An integer MFMA whose accumulator starts
// at kIntBias therefore ends with the bits of the float kFloatBias + sum, and
// one exact subtraction gives (float)sum (full-rate VALU instead of
// v_cvt_f32_i32); adding kFloatBias to an integer-valued float leaves n in
// the low byte of its bits (two's complement), so the byte is a plain store.
constexpr int kIntBias = 0x4B400000;
constexpr float kFloatBias = 12582912.0f;
__device__ __forceinline__ float unbias(int biased) { return __builtin_bit_cast(float, biased) - kFloatBias; }
__device__ __forceinline__ uint32_t biased_bits(float integral) { return __builtin_bit_cast(uint32_t, integral + kFloatBias); }
// Four integer-valued floats in [-128, 127] -> four int8 bytes (low bytes of
// their biased bits, gathered by v_perm_b32).
__device__ __forceinline__ uint32_t pack_i8x4_biased(float a, float b, float c, float d) {
    const uint32_t ab = __builtin_amdgcn_perm(biased_bits(b), biased_bits(a), 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(biased_bits(d), biased_bits(c), 0x04000c0cu);
    return ab | cd;
}


// Byte `b` of w as OCP e4m3 -> float (v_cvt_f32_fp8, exact); b folds to a
// constant in unrolled loops.
__device__ __forceinline__ float fp8_byte(uint32_t w, int b) {
    switch (b) {
        case 0: return __builtin_amdgcn_cvt_f32_fp8((int)w, 0);
        case 1: return __builtin_amdgcn_cvt_f32_fp8((int)w, 1);
        case 2: return __builtin_amdgcn_cvt_f32_fp8((int)w, 2);
        default: return __builtin_amdgcn_cvt_f32_fp8((int)w, 3);
    }
}

// e4m3 of two finite values (saturating), without the NaN handling of e4m3x2.
__device__ __forceinline__ uint32_t e4m3x2_finite(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_fminf(__builtin_fmaxf(a, -448.0f), 448.0f),
                                                     __builtin_fminf(__builtin_fmaxf(b, -448.0f), 448.0f), 0, false) & 0xffffu;
}

// Lane moves within rows of 16 lanes (DPP, no LDS round trip).  row_shl(v, n)
// gives lane i the value of lane i + n of its row (lanes past the row's end
// get 0): in a reduction tree v += row_shl(v, n), n = 8, 4, 2, 1, the row's
// lane 0 adds exactly the operands of a shuffle-down tree.  row_ror rotates
// the row, so a max over rotations 8, 4, 2, 1 reaches every lane.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, true));
}
template <int N>
__device__ __forceinline__ float row_shl(float v) { return dpp<0x100 + N>(v); }
__device__ __forceinline__ float row_max16(float v) {
    v = __builtin_fmaxf(v, dpp<0x128>(v));
    v = __builtin_fmaxf(v, dpp<0x124>(v));
    v = __builtin_fmaxf(v, dpp<0x122>(v));
    return __builtin_fmaxf(v, dpp<0x121>(v));
}
__device__ __forceinline__ float row_sum_tree16(float v) {  // exact shuffle-down tree, valid in the row's lane 0
    v += row_shl<8>(v);
    v += row_shl<4>(v);
    v += row_shl<2>(v);
    return v + row_shl<1>(v);
}

// Eight signed nibbles -> two words of four bytes, each nibble in the high
// half of its byte (value * 16): lo takes the even nibbles, hi the odd ones.
__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xf0f0f0f0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xf0f0f0f0u; }
__device__ __forceinline__ v4i widen_s4x16(uint2 w) {
    return v4i{(int)nib_lo16(w.x), (int)nib_hi16(w.x), (int)nib_lo16(w.y), (int)nib_hi16(w.y)};
}

// Position of key k (0..319, relative to the tile's first key) in a row of
// the U4 probability operand: within each 16 keys the order is
// 0,2,4,6, 1,3,5,7, 8,10,12,14, 9,11,13,15, which is the order widen_s4x16
// produces from 16 consecutive S4 values.
__device__ __forceinline__ int prob_pos(int k) { return (k & ~15) + (k & 8) + ((k & 1) << 2) + ((k & 7) >> 1); }

// ---- packers ------------------------------------------------------------

// encoder.cu:2054-2074 / :2076-2097.  16 lanes per 128-value vector, lane j
// holding dimensions 8j..8j+7.  INT8: dims 8j..8j+3 go to the four bytes of
// reference lane 2j, 8j+4..8j+7 to those of lane 2j+1.  INT4: both reference
// lanes' u16 words are adjacent, so the eight nibbles form one u32 at
// (j/8)*32 + (j%4)*8 + (j&4).
template <bool kInt4>
__global__ __launch_bounds__(256) void pack_vectors_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                           float* __restrict__ scales, int vectors) {
    const int vec = (int)(blockIdx.x * 16 + (threadIdx.x >> 4));
    const int j = threadIdx.x & 15;
    if (vec >= vectors) return;
    const uint4 raw = *(const uint4*)(in + (size_t)vec * 128 + 8 * j);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8], m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = h2f((uint16_t)(w[i / 2] >> (16 * (i & 1))));
        m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) m = max_level(m, off);  // DPP levels within the 16-lane vector
    const float scale = m > 0.0f ? m / (kInt4 ? 7.0f : 127.0f) : 1.0f;
    if (j == 0) scales[vec] = scale;
    float qv[8];
    quant_n<8>(v, scale, qv);
    if constexpr (kInt4) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= ((uint32_t)(int)qv[i] & 15u) << (4 * i);
        *(uint32_t*)(out + (size_t)vec * 64 + (j / 8) * 32 + (j % 4) * 8 + (j & 4)) = word;
    } else {
        uint32_t word[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) word[i / 4] |= ((uint32_t)(int)qv[i] & 255u) << (8 * (i & 3));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int lane = 2 * j + h;
            *(uint32_t*)(out + (size_t)vec * 128 + (lane / 8) * 32 + (lane % 4) * 8 + (lane & 4)) = word[h];
        }
    }
}

// encoder.cu:561-634.  One 256-thread workgroup per feature row of the
// feature-major V [1024 x rows], 8 consecutive keys per thread and pass: the
// first pass takes the row's maximum, the second re-reads the row and
// quantizes it.  Few registers, so all 1024 workgroups are resident at once.
// Measured ≈ 49 µs at T = 45000 (2.4 TB/s of algorithmic bytes), the same as a
// register-resident single pass with 1024-thread workgroups, deeper unrolling
// or rotated start offsets.
constexpr int kValueThreads = 256;
__global__ __launch_bounds__(kValueThreads) void quantize_value_int4_kernel(const uint16_t* __restrict__ vt, uint8_t* __restrict__ out,
                                                                           int rows, float inverse_scale, int edge_only,
                                                                           int valid_rows) {
    const int f = blockIdx.x, tid = threadIdx.x;
    constexpr int kChunk = 8 * kValueThreads;
    const size_t elements = (size_t)rows * kModel;
    const uint16_t* x = vt + (size_t)f * rows;
    __shared__ float wave_max_s[kValueThreads / 64];
    __shared__ float scale_s;
    float m = 0.0f;
#pragma unroll 8
    for (int r = 8 * tid; r < rows; r += kChunk) {
        const uint4 u = *(const uint4*)(x + r);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(h2f((uint16_t)(w[i / 2] >> (16 * (i & 1))))));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) wave_max_s[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        float t = 0.0f;
        for (int i = 0; i < kValueThreads / 64; ++i) t = __builtin_fmaxf(t, wave_max_s[i]);
        const float sc = t > 0.0f ? t / 7.0f : 1.0f;
        scale_s = sc;
        ((float*)(out + elements + elements / 2))[f] = sc;
    }
    __syncthreads();
    const float scale = scale_s;
#pragma unroll 4
    for (int r = 8 * tid; r < rows; r += kChunk) {
        const uint4 u = *(const uint4*)(x + r);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        uint32_t fp8[2] = {0, 0}, s4 = 0;
        bool all = true;
        float vals[8], qv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) vals[i] = h2f((uint16_t)(w[i / 2] >> (16 * (i & 1))));
        quant_n<8>(vals, scale, qv);
        const bool any8 = !edge_only || r < 272 || r + 7 >= valid_rows - 272;  // some pair stores FP8
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float a = vals[2 * p], b = vals[2 * p + 1];
            if (any8) fp8[p / 2] |= e4m3x2(a * inverse_scale, b * inverse_scale) << (16 * (p & 1));
            // clamp(rn(v / s), -7, 7); a NaN input quantizes to 0
            const int qa = a != a ? 0 : (int)__builtin_fminf(__builtin_fmaxf(qv[2 * p], -7.0f), 7.0f);
            const int qb = b != b ? 0 : (int)__builtin_fminf(__builtin_fmaxf(qv[2 * p + 1], -7.0f), 7.0f);
            s4 |= (uint32_t)((qa & 15) | ((qb & 15) << 4)) << (8 * p);
            const int row = r + 2 * p;
            all = all && (!edge_only || row < 272 || row + 1 >= valid_rows - 272);
        }
        *(uint32_t*)(out + elements + ((size_t)f * rows + r) / 2) = s4;
        if (!any8) continue;
        uint8_t* o = out + (size_t)f * rows + r;
        if (all) {
            *(uint2*)o = uint2{fp8[0], fp8[1]};
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int row = r + 2 * p;
                if (row < 272 || row + 1 >= valid_rows - 272) *(uint16_t*)(o + 2 * p) = (uint16_t)(fp8[p / 2] >> (16 * (p & 1)));
            }
        }
    }
}

// ---- attention -----------------------------------------------------------

struct QueryShared {
    float scores[4][264];  // one row per wave: scores, then exp, then weights
};
// Interior tiles of one head streamed through one workgroup: the keys and
// S4 values of the current window live in rings indexed by key % 288 (the
// 272-key window plus the 16 keys of the next tile), so each tile fetches only
// its 16 new keys.
constexpr int kRing = 288;
struct StreamShared {
    uint8_t ring_k[kRing][72];  // INT4 key vectors (64 bytes, row padded)
    float ring_ks[kRing];
    uint8_t ring_v[kHead][144];  // S4 V of the head's 128 features, ring key / 2
    uint8_t qa_u[16][144];       // INT4 (q+u) as int8, MFMA operand order, rows padded
    uint8_t qa_v[16][144];       // INT8 (q+v), reference score-vector byte order
    uint16_t cs[16][kPosRows];
    uint16_t ps[16][kPosRows];
    uint8_t prob[16][336];  // U4 probabilities as bytes, prob_pos order
    uint8_t out[16][128];
    float qs_u[16], qs_v[16], pscale[16];
};
struct TcShared {
    uint16_t qu[16][136];
    uint16_t qv[16][136];
    float cs[16][kPosRows];
    float ps[16][kPosRows];
    uint8_t prob[16][400];  // e4m3 probabilities for keys 0..383 (zero past the window)
    uint16_t out[16][128];
};

// Context store (encoder.cu:1463-1474) of two adjacent features: fp16 round,
// packed form e4m3(x * 28).
template <bool kPacked>
__device__ __forceinline__ void store2(void* output, size_t index, float c0, float c1) {
    if constexpr (kPacked)
        *(uint16_t*)((uint8_t*)output + index) = (uint16_t)e4m3x2(round_f16(c0) * 28.0f, round_f16(c1) * 28.0f);
    else
        *(uint32_t*)((uint16_t*)output + index) = (uint32_t)f2h(c0) | ((uint32_t)f2h(c1) << 16);
}

// encoder.cu:1548-1684: the per-query FP32 path of boundary tiles, one wave
// per query.  The arithmetic is the reference's, in its 32-lane warp order:
// a slot's score is 16 partial sums (lane h of 16 accumulates dimensions
// 2h + 32q, q = 0..3, interleaving content and position FMAs) reduced by a
// shuffle tree; the denominator is 32 partial sums (partial l adds slots l,
// l + 32, ... in order) reduced by a shuffle tree; each output feature's
// context is one FMA chain over the keys in order.  Which lane runs which of
// these chains is free, so a wave evaluates four slots per step, keeps eight
// steps of loads in flight, and owns two features per lane.
template <bool kPacked>
__device__ void attention_query(float* scores, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
                                const uint8_t* __restrict__ value_fp8, const uint16_t* __restrict__ position,
                                const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v, void* output, int qr,
                                int head, int rows, int padded_rows, int valid_rows, int left, int right, int value_stride) {
    const int lane = threadIdx.x & 63;
    const size_t oidx = (size_t)qr * kModel + head * kHead + 2 * lane;
    if (qr >= rows || qr >= valid_rows) {
        if (qr < padded_rows) store2<kPacked>(output, oidx, 0.0f, 0.0f);
        return;
    }
    const int first = max(0, qr - left), last = min(valid_rows - 1, qr + right);
    const int count = last - first + 1;
    const int grp = lane >> 4, hl = lane & 15;
    float2 su[4], sv[4];
#pragma unroll
    for (int quarter = 0; quarter < 4; ++quarter) {
        const int d = head * kHead + 2 * hl + 32 * quarter;
        const uint32_t q = *(const uint32_t*)(query + (size_t)qr * kModel + d);
        const uint32_t u = *(const uint32_t*)(bias_u + d);
        const uint32_t v = *(const uint32_t*)(bias_v + d);
        const float q0 = h2f((uint16_t)q), q1 = h2f((uint16_t)(q >> 16));
        su[quarter] = make_float2(q0 + h2f((uint16_t)u), q1 + h2f((uint16_t)(u >> 16)));
        sv[quarter] = make_float2(q0 + h2f((uint16_t)v), q1 + h2f((uint16_t)(v >> 16)));
    }
    constexpr int kU = 8;
    for (int sp0 = 0; sp0 < count; sp0 += 4 * kU) {
        uint32_t kw[kU][4], pw[kU][4];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int key_row = first + min(sp0 + 4 * u + grp, count - 1);
            const int prow = left - qr + key_row;
#pragma unroll
            for (int quarter = 0; quarter < 4; ++quarter) {
                const int d = 2 * hl + 32 * quarter;
                kw[u][quarter] = *(const uint32_t*)(key + (size_t)key_row * kModel + head * kHead + d);
                pw[u][quarter] = *(const uint32_t*)(position + ((size_t)head * kPosRows + prow) * kHead + d);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int slot = sp0 + 4 * u + grp;
            float s = 0.0f;
#pragma unroll
            for (int quarter = 0; quarter < 4; ++quarter) {
                const uint32_t k = kw[u][quarter], p = pw[u][quarter];
                s = __builtin_fmaf(su[quarter].x, h2f((uint16_t)k), s);
                s = __builtin_fmaf(sv[quarter].x, h2f((uint16_t)p), s);
                s = __builtin_fmaf(su[quarter].y, h2f((uint16_t)(k >> 16)), s);
                s = __builtin_fmaf(sv[quarter].y, h2f((uint16_t)(p >> 16)), s);
            }
            s = sum_desc<16>(s);  // xor 8, 4, 2, 1
            if (hl == 0 && slot < count) scores[slot] = s * kScoreScale;
        }
    }
    wave_sync();
    float mx = -FLT_MAX;
    for (int slot = lane; slot < count; slot += 64) mx = __builtin_fmaxf(mx, scores[slot]);
    mx = wave_max(mx);
    for (int slot = lane; slot < count; slot += 64) scores[slot] = softmax_exp(scores[slot] - mx);
    wave_sync();
    float den = 0.0f;
    if (lane < 32)
        for (int slot = lane; slot < count; slot += 32) den += scores[slot];
    den = sum_desc<32>(den);  // xor 16, ..., 1 over lanes 0..31
    den = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(den)));
    wave_sync();
    for (int slot = lane; slot < count; slot += 64) scores[slot] = scores[slot] / den;
    wave_sync();
    float c0 = 0.0f, c1 = 0.0f;
    const int feature = head * kHead + 2 * lane;
    constexpr int kC = 16;  // chunks of four keys in flight per batch
    for (int chunk0 = first & ~3; chunk0 <= last; chunk0 += 4 * kC) {
        uint32_t words[kC][2];
#pragma unroll
        for (int b = 0; b < kC; ++b) {
            const int chunk = min(chunk0 + 4 * b, last & ~3);
            words[b][0] = *(const uint32_t*)(value_fp8 + (size_t)feature * value_stride + chunk);
            words[b][1] = *(const uint32_t*)(value_fp8 + (size_t)(feature + 1) * value_stride + chunk);
        }
#pragma unroll
        for (int b = 0; b < kC; ++b) {
#pragma unroll
            for (int item = 0; item < 4; ++item) {
                const int kr = chunk0 + 4 * b + item;
                if (kr < first || kr > last) continue;
                const float weight = scores[kr - first];
                c0 = __builtin_fmaf(weight, fp8_byte(words[b][0], item) * kValueScale, c0);
                c1 = __builtin_fmaf(weight, fp8_byte(words[b][1], item) * kValueScale, c1);
            }
        }
    }
    store2<kPacked>(output, oidx, c0, c1);
}

// Softmax of query lq over its 257 slots from the combined logits held by a
// half wave (lane ln has slots ln + 32 part).  Returns e = exp(l - max) in
// place and the denominator (shuffle tree in 32-lane warp order).
__device__ __forceinline__ float softmax_half(float (&l)[9], int ln) {
    float mx = -FLT_MAX;
#pragma unroll
    for (int part = 0; part < 9; ++part)
        if (ln + 32 * part < kMaxAtt) mx = __builtin_fmaxf(mx, l[part]);
#pragma unroll
    for (int off = 1; off <= 16; off <<= 1) mx = max_level(mx, off);
    float den = 0.0f;
#pragma unroll
    for (int part = 0; part < 9; ++part)
        if (ln + 32 * part < kMaxAtt) {
            l[part] = softmax_exp(l[part] - mx);
            den += l[part];
        }
    return sum_desc<32>(den);  // xor 16, ..., 1 within the half wave
}

// encoder.cu:1687-1966 for the interior tiles [t0, t1) of one head: INT4
// content and INT8 position scores, U4 probabilities x S4 V, e4m3(x*28) out.
// The position operands (the same for every tile of a head) stay in
// registers; keys and values stream through the LDS rings; the next tile's
// queries and 16 new keys are loaded while the current tile computes.
__device__ void attention_packed_stream(StreamShared& sh, const uint16_t* __restrict__ query, const uint8_t* __restrict__ value_fp8,
                                        const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
                                        uint8_t* __restrict__ output, int t0, int t1, int head, int value_stride,
                                        const uint8_t* __restrict__ packed_key, const float* __restrict__ key_scales,
                                        const uint8_t* __restrict__ packed_position, const float* __restrict__ position_scales) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, l16 = lane & 15;
    const int qr16 = tid >> 4, qj = tid & 15;  // query row / 8-dimension slice this thread quantizes
    const uint8_t* s4 = value_fp8 + (size_t)kModel * value_stride;
    const float* vscales = (const float*)(value_fp8 + (size_t)kModel * value_stride * 3 / 2);

    // Position operands of this wave's key tiles kt = wave + 4i.
    uint4 pq[5][2];
    float psc[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int kt = min(wave + 4 * i, kPosRows / 16 - 1);
        const int pvec = head * kPosRows + 16 * kt + l16;
        const uint8_t* pb = packed_position + (size_t)pvec * 128;
        pq[i][0] = *(const uint4*)(pb + 16 * g);
        pq[i][1] = *(const uint4*)(pb + 64 + 16 * g);
        psc[i] = position_scales[pvec];
    }
    const uint4 bu = *(const uint4*)(bias_u + head * kHead + 8 * qj);
    const uint4 bv = *(const uint4*)(bias_v + head * kHead + 8 * qj);
    float vs[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) vs[c] = vscales[head * kHead + 16 * (2 * wave + c) + l16];

    // Prologue: the first tile's whole key window into the rings.
    {
        const int fk = 16 * t0 - 128;
        for (int i = tid; i < kPosRows * 4; i += 256) {
            const int key = fk + (i >> 2);
            *(uint4*)&sh.ring_k[key % kRing][16 * (i & 3)] =
                *(const uint4*)(packed_key + ((size_t)key * kHeads + head) * 64 + 16 * (i & 3));
        }
        for (int i = tid; i < kPosRows; i += 256) sh.ring_ks[(fk + i) % kRing] = key_scales[(size_t)(fk + i) * kHeads + head];
        for (int i = tid; i < kHead * (kPosRows / 16); i += 256) {
            const int f = i / (kPosRows / 16), seg = i % (kPosRows / 16);
            const int key = fk + 16 * seg;
            *(uint2*)&sh.ring_v[f][(key % kRing) / 2] = *(const uint2*)(s4 + ((size_t)(head * kHead + f) * value_stride + key) / 2);
        }
    }
    uint4 qn = *(const uint4*)(query + (size_t)(16 * t0 + qr16) * kModel + head * kHead + 8 * qj);

    for (int t = t0; t < t1; ++t) {
        const int qb = 16 * t, first_key = qb - 128;
        const bool more = t + 1 < t1;

        // Phase 1: clear the probability rows; quantize q+u and q+v.
        for (int i = tid; i < 16 * 336 / 4; i += 256) ((uint32_t*)sh.prob)[i] = 0;
        {
            // q+u and q+v as fp16 adds: for fp16 operands, rounding the fp32 sum
            // to fp16 is the same as one fp16 addition (24 >= 2*11 + 2 bits).
            const uint32_t qw[4] = {qn.x, qn.y, qn.z, qn.w}, uw[4] = {bu.x, bu.y, bu.z, bu.w}, vw[4] = {bv.x, bv.y, bv.z, bv.w};
            h2_t au[4], av[4], mxu = h2_t{0, 0}, mxv = h2_t{0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                au[i] = __builtin_bit_cast(h2_t, qw[i]) + __builtin_bit_cast(h2_t, uw[i]);
                av[i] = __builtin_bit_cast(h2_t, qw[i]) + __builtin_bit_cast(h2_t, vw[i]);
                mxu = __builtin_elementwise_max(mxu, __builtin_elementwise_abs(au[i]));
                mxv = __builtin_elementwise_max(mxv, __builtin_elementwise_abs(av[i]));
            }
            float mu = __builtin_fmaxf((float)mxu[0], (float)mxu[1]), mv = __builtin_fmaxf((float)mxv[0], (float)mxv[1]);
            mu = row_max16(mu);
            mv = row_max16(mv);
            const float su = mu > 0.0f ? mu / 7.0f : 1.0f, sv = mv > 0.0f ? mv / 127.0f : 1.0f;
            const float isu = __builtin_amdgcn_rcpf(su), isv = __builtin_amdgcn_rcpf(sv);
            if (qj == 0) {
                sh.qs_u[qr16] = su * 0.0625f;  // carries the 1/16 of the widened INT4 keys
                sh.qs_v[qr16] = sv;
            }
            float fu[8], fv[8];
            bool tie = false;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                fu[i] = quant_fast((float)au[i / 2][i & 1], isu, tie);
                fv[i] = quant_fast((float)av[i / 2][i & 1], isv, tie);
            }
            if (__builtin_amdgcn_ballot_w64(tie) != 0) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    fu[i] = __builtin_rintf((float)au[i / 2][i & 1] / su);
                    fv[i] = __builtin_rintf((float)av[i / 2][i & 1] / sv);
                }
            }
            const uint32_t ue = pack_i8x4_biased(fu[0], fu[2], fu[4], fu[6]), uo = pack_i8x4_biased(fu[1], fu[3], fu[5], fu[7]);
            const uint32_t v8[2] = {pack_i8x4_biased(fv[0], fv[1], fv[2], fv[3]), pack_i8x4_biased(fv[4], fv[5], fv[6], fv[7])};
            // INT4 plane: dimension 8j+i sits at storage nibble 2*off_j + i of
            // the key vectors; widen_s4x16 of the key's bytes [32m + 8g, +8)
            // yields even nibbles then odd nibbles per word, hence this order.
            const int pa = 64 * (qj >> 3) + 16 * (qj & 3) + 8 * ((qj >> 2) & 1);
            *(uint2*)&sh.qa_u[qr16][pa] = uint2{ue, uo};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int L = 2 * qj + h;
                *(uint32_t*)&sh.qa_v[qr16][(L / 8) * 32 + (L % 4) * 8 + (L & 4)] = v8[h];
            }
        }
        // Next tile's queries and its 16 new keys (qb + 144 .. qb + 159).
        uint4 nk = uint4{0, 0, 0, 0};
        uint2 nv = uint2{0, 0};
        float nks = 0.0f;
        const int nkey = qb + 144;
        if (more) {
            qn = *(const uint4*)(query + (size_t)(qb + 16 + qr16) * kModel + head * kHead + 8 * qj);
            if (tid < 64) nk = *(const uint4*)(packed_key + ((size_t)(nkey + (tid >> 2)) * kHeads + head) * 64 + 16 * (tid & 3));
            else if (tid < 80) nks = key_scales[(size_t)(nkey + tid - 64) * kHeads + head];
            else if (tid >= 128) nv = *(const uint2*)(s4 + ((size_t)(head * kHead + tid - 128) * value_stride + nkey) / 2);
        }
        __syncthreads();

        // Phase 2: scores for the 17 key tiles of 16 columns, four waves.
        {
            const v4i au0 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_u[l16][16 * g]);
            const v4i au1 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_u[l16][64 + 16 * g]);
            const v4i av0 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_v[l16][16 * g]);
            const v4i av1 = __builtin_bit_cast(v4i, *(const uint4*)&sh.qa_v[l16][64 + 16 * g]);
            float qsu[4], qsv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                qsu[r] = sh.qs_u[4 * g + r];
                qsv[r] = sh.qs_v[4 * g + r];
            }
            const int ring0 = first_key % kRing;
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                const int kt = min(wave + 4 * i, kPosRows / 16 - 1);  // wave 0 alone has a fifth tile
                const int col = 16 * kt + l16;
                int slot = ring0 + col;
                slot = slot >= kRing ? slot - kRing : slot;
                const uint2 k0 = *(const uint2*)&sh.ring_k[slot][8 * g], k1 = *(const uint2*)&sh.ring_k[slot][32 + 8 * g];
                const float ks = sh.ring_ks[slot], pscl = psc[i];
                // |sums| <= 7 * 128 * 128 (INT4 x widened INT4) and 127 * 127 * 128 (INT8), below 2^22
                const v4i bias = v4i{kIntBias, kIntBias, kIntBias, kIntBias};
                v4i acu = __builtin_amdgcn_mfma_i32_16x16x64_i8(au0, widen_s4x16(k0), bias, 0, 0, 0);
                acu = __builtin_amdgcn_mfma_i32_16x16x64_i8(au1, widen_s4x16(k1), acu, 0, 0, 0);
                v4i acv = __builtin_amdgcn_mfma_i32_16x16x64_i8(av0, __builtin_bit_cast(v4i, pq[i][0]), bias, 0, 0, 0);
                acv = __builtin_amdgcn_mfma_i32_16x16x64_i8(av1, __builtin_bit_cast(v4i, pq[i][1]), acv, 0, 0, 0);
                if (wave + 4 * i < kPosRows / 16) {
#pragma unroll
                    for (int r = 0; r < 4; r += 2) {
                        const uint32_t c2 = bf16x2_rn(unbias(acu[r]) * (qsu[r] * ks), unbias(acu[r + 1]) * (qsu[r + 1] * ks));
                        const uint32_t p2 = bf16x2_rn(unbias(acv[r]) * (qsv[r] * pscl), unbias(acv[r + 1]) * (qsv[r + 1] * pscl));
                        sh.cs[4 * g + r][col] = (uint16_t)c2;
                        sh.cs[4 * g + r + 1][col] = (uint16_t)(c2 >> 16);
                        sh.ps[4 * g + r][col] = (uint16_t)p2;
                        sh.ps[4 * g + r + 1][col] = (uint16_t)(p2 >> 16);
                    }
                }
            }
        }
        __syncthreads();

        // Phase 3: softmax and U4 probabilities, 16 lanes per query: lane j
        // owns slots j + 16k.  The reference's 32 denominator partials (slots
        // l, l + 32, ...) are this lane's two chains over even and odd k; its
        // first tree step (partial l plus partial l + 16) is the lane's own
        // add, the remaining four run over the row.
        {
            const int lq = tid >> 4, j = tid & 15;
            float l[17], mx = -FLT_MAX;
#pragma unroll
            for (int k = 0; k < 17; ++k) {
                const int slot = j + 16 * k;
                l[k] = slot < kMaxAtt ? (bf16_f32(sh.cs[lq][lq + slot]) + bf16_f32(sh.ps[lq][slot])) * kScoreScale : -FLT_MAX;
                mx = __builtin_fmaxf(mx, l[k]);
            }
            mx = row_max16(mx);
            float even = 0.0f, odd = 0.0f;
#pragma unroll
            for (int k = 0; k < 17; ++k) {
                if (j + 16 * k < kMaxAtt) {
                    l[k] = softmax_exp(l[k] - mx);
                    if (k & 1) odd += l[k];
                    else even += l[k];
                }
            }
            const float den = row_sum_tree16(even + odd);
            if (j == 0) sh.pscale[lq] = 1.0f / (15.0f * den);
            uint8_t* prow = &sh.prob[lq][prob_pos(lq + j)];  // slot j + 16k sits 16k further
#pragma unroll
            for (int k = 0; k < 17; ++k)
                if (j + 16 * k < kMaxAtt) prow[16 * k] = (uint8_t)biased_bits(l[k] * 15.0f);  // rint: the add rounds to nearest even
        }
        __syncthreads();

        // Phase 4: context = U4 probabilities x S4 V over keys 0..271 (five
        // K=64 steps; keys >= 272 contribute zero operands).
        {
            // |sums| <= 15 * 128 * 320, below 2^22
            v4i acc[2] = {v4i{kIntBias, kIntBias, kIntBias, kIntBias}, v4i{kIntBias, kIntBias, kIntBias, kIntBias}};
            const int ring0 = first_key % kRing;
#pragma unroll
            for (int st = 0; st < 5; ++st) {
                const int ko = 64 * st + 16 * g;
                const v4i a = __builtin_bit_cast(v4i, *(const uint4*)&sh.prob[l16][ko]);
                int slot = ring0 + ko;
                slot = slot >= kRing ? slot - kRing : slot;
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const uint2 w = ko < kPosRows ? *(const uint2*)&sh.ring_v[16 * (2 * wave + c) + l16][slot / 2] : uint2{0, 0};
                    acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, widen_s4x16(w), acc[c], 0, 0, 0);
                }
            }
            float ps4[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ps4[r] = sh.pscale[4 * g + r] * 0.0625f;  // the sums carry V x 16
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int fl = 16 * (2 * wave + c) + l16;
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    // (sum / 16) * (p * v) == sum * ((p / 16) * v): scaling by 2^-4 is exact
                    const float x0 = unbias(acc[c][r]) * (ps4[r] * vs[c]);
                    const float x1 = unbias(acc[c][r + 1]) * (ps4[r + 1] * vs[c]);
                    const uint32_t b2 = e4m3x2_finite(round_f16(x0) * 28.0f, round_f16(x1) * 28.0f);
                    sh.out[4 * g + r][fl] = (uint8_t)b2;
                    sh.out[4 * g + r + 1][fl] = (uint8_t)(b2 >> 8);
                }
            }
        }
        __syncthreads();
        *(uint2*)(output + (size_t)(qb + qr16) * kModel + head * kHead + 8 * qj) = *(const uint2*)&sh.out[qr16][8 * qj];
        // The 16 new keys go to ring slots of keys qb-144 .. qb-129, which this
        // tile no longer reads; the next tile's first barrier publishes them.
        if (more) {
            if (tid < 64) *(uint4*)&sh.ring_k[(nkey + (tid >> 2)) % kRing][16 * (tid & 3)] = nk;
            else if (tid < 80) sh.ring_ks[(nkey + tid - 64) % kRing] = nks;
            else if (tid >= 128) *(uint2*)&sh.ring_v[tid - 128][(nkey % kRing) / 2] = nv;
        }
    }
}

// encoder.cu:1768-2018 (kPackedOutput = false): fp16 scores, e4m3 probabilities
// (p * 448) x e4m3 V, scaled by (1/448)*(8/448), fp16 out.
__device__ void attention_tc_tile(TcShared& sh, const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
                                  const uint8_t* __restrict__ value_fp8, const uint16_t* __restrict__ position,
                                  const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
                                  uint16_t* __restrict__ output, int qb, int head, int value_stride) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, l16 = lane & 15;
    const int first_key = qb - 128;
    {
        const int r = tid >> 4, j = tid & 15;
        const uint4 q = *(const uint4*)(query + (size_t)(qb + r) * kModel + head * kHead + 8 * j);
        const uint4 u = *(const uint4*)(bias_u + head * kHead + 8 * j);
        const uint4 v = *(const uint4*)(bias_v + head * kHead + 8 * j);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, uw[4] = {u.x, u.y, u.z, u.w}, vw[4] = {v.x, v.y, v.z, v.w};
        uint32_t ou[4], ov[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q0 = h2f((uint16_t)qw[i]), q1 = h2f((uint16_t)(qw[i] >> 16));
            ou[i] = (uint32_t)f2h(q0 + h2f((uint16_t)uw[i])) | ((uint32_t)f2h(q1 + h2f((uint16_t)(uw[i] >> 16))) << 16);
            ov[i] = (uint32_t)f2h(q0 + h2f((uint16_t)vw[i])) | ((uint32_t)f2h(q1 + h2f((uint16_t)(vw[i] >> 16))) << 16);
        }
        *(uint4*)&sh.qu[r][8 * j] = uint4{ou[0], ou[1], ou[2], ou[3]};
        *(uint4*)&sh.qv[r][8 * j] = uint4{ov[0], ov[1], ov[2], ov[3]};
    }
    __syncthreads();
    {
        v8h au[4], av[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            au[m] = __builtin_bit_cast(v8h, *(const uint4*)&sh.qu[l16][32 * m + 8 * g]);
            av[m] = __builtin_bit_cast(v8h, *(const uint4*)&sh.qv[l16][32 * m + 8 * g]);
        }
        for (int kt = wave; kt < kPosRows / 16; kt += 4) {
            const int col = 16 * kt + l16;
            const uint16_t* kr = key + (size_t)(first_key + col) * kModel + head * kHead + 8 * g;
            const uint16_t* pr = position + ((size_t)head * kPosRows + col) * kHead + 8 * g;
            uint4 kb[4], pb[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                kb[m] = *(const uint4*)(kr + 32 * m);
                pb[m] = *(const uint4*)(pr + 32 * m);
            }
            v4f acu = v4f{0, 0, 0, 0}, acv = v4f{0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acu = __builtin_amdgcn_mfma_f32_16x16x32_f16(au[m], __builtin_bit_cast(v8h, kb[m]), acu, 0, 0, 0);
                acv = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[m], __builtin_bit_cast(v8h, pb[m]), acv, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sh.cs[4 * g + r][col] = acu[r];
                sh.ps[4 * g + r][col] = acv[r];
            }
        }
    }
    __syncthreads();
    {
        const int hw = tid >> 5, ln = tid & 31;
#pragma unroll
        for (int item = 0; item < 2; ++item) {
            const int lq = hw + 8 * item;
            float l[9];
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                l[part] = slot < kMaxAtt ? (sh.cs[lq][lq + slot] + sh.ps[lq][slot]) * kScoreScale : -FLT_MAX;
            }
            const float den = softmax_half(l, ln);
            // Union slot u = lq + slot; bytes outside the window are e4m3(0).
            for (int u = ln; u < 384; u += 32) sh.prob[lq][u] = 0;
            wave_sync();
#pragma unroll
            for (int part = 0; part < 9; ++part) {
                const int slot = ln + 32 * part;
                if (slot < kMaxAtt) sh.prob[lq][lq + slot] = (uint8_t)e4m3x2(l[part] / den * 448.0f, 0.0f);
            }
        }
    }
    __syncthreads();
    {
        v4f acc[2] = {v4f{0, 0, 0, 0}, v4f{0, 0, 0, 0}};
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int ko = 128 * s + 32 * g;
            const uint4 a0 = *(const uint4*)&sh.prob[l16][ko], a1 = *(const uint4*)&sh.prob[l16][ko + 16];
            const v8i a = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int fg = head * kHead + 16 * (2 * wave + c) + l16;
                const uint8_t* vr = value_fp8 + (size_t)fg * value_stride + first_key + ko;
                uint4 b0 = uint4{0, 0, 0, 0}, b1 = uint4{0, 0, 0, 0};
                if (ko < kPosRows) b0 = *(const uint4*)vr;
                if (ko + 16 < kPosRows) b1 = *(const uint4*)(vr + 16);
                const v8i b = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
                acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[c], 0, 0, 0, 0, 0, 0);
            }
        }
        constexpr float kContextScale = (1.0f / 448.0f) * (8.0f / 448.0f);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int fl = 16 * (2 * wave + c) + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) sh.out[4 * g + r][fl] = f2h(acc[c][r] * kContextScale);
        }
    }
    __syncthreads();
    {
        const int r = tid >> 4, j = tid & 15;
        *(uint4*)(output + (size_t)(qb + r) * kModel + head * kHead + 8 * j) = *(const uint4*)&sh.out[r][8 * j];
    }
}

// The boundary queries: tiles [0, ib) and [ie, tiles), four queries (one
// per wave) of one head per workgroup, small LDS.
template <bool kPacked>
__global__ __launch_bounds__(256) void boundary_attention_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key, const uint8_t* __restrict__ value_fp8,
    const uint16_t* __restrict__ position, const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
    void* __restrict__ output, int rows, int padded_rows, int valid_rows, int left, int right, int value_stride, int ib, int ie) {
    __shared__ QueryShared sh;
    const int L = (int)blockIdx.x;
    const int head = L & 7, grp = L >> 3, t = grp >> 2;
    const int tile = t < ib ? t : ie + (t - ib);
    attention_query<kPacked>(sh.scores[threadIdx.x >> 6], query, key, value_fp8, position, bias_u, bias_v, output,
                             16 * tile + 4 * (grp & 3) + (int)(threadIdx.x >> 6), head, rows, padded_rows, valid_rows, left, right,
                             value_stride);
}

// The interior tiles [ib, ie): packed -> `chunks` runs of consecutive tiles
// per head, one workgroup each; tc -> one workgroup per tile and head.
// Workgroup L runs on XCD L % 8; the work is split into eight contiguous
// ranges of (tile or run, head) pairs so that each XCD's L2 holds the keys
// and values of neighbouring tiles.
template <bool kPacked>
__global__ __launch_bounds__(256) void interior_attention_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key, const uint8_t* __restrict__ value_fp8,
    const uint16_t* __restrict__ position, const uint16_t* __restrict__ bias_u, const uint16_t* __restrict__ bias_v,
    void* __restrict__ output, int value_stride, const uint8_t* __restrict__ packed_key, const float* __restrict__ key_scales,
    const uint8_t* __restrict__ packed_position, const float* __restrict__ position_scales, int ib, int ie, int chunks) {
    const int J = (int)blockIdx.x, n = ie - ib;
    if constexpr (kPacked) {
        __shared__ StreamShared sh;
        const int K = (J & 7) * chunks + (J >> 3);
        const int run = K >> 3, head = K & 7;
        const int t0 = ib + (int)((long)n * run / chunks), t1 = ib + (int)((long)n * (run + 1) / chunks);
        if (t0 < t1)
            attention_packed_stream(sh, query, value_fp8, bias_u, bias_v, (uint8_t*)output, t0, t1, head, value_stride, packed_key,
                                    key_scales, packed_position, position_scales);
    } else {
        __shared__ TcShared sh;
        const int K = (J & 7) * n + (J >> 3);
        attention_tc_tile(sh, query, key, value_fp8, position, bias_u, bias_v, (uint16_t*)output, 16 * (ib + (K >> 3)), K & 7,
                          value_stride);
    }
}

// A second stream per device for the boundary kernel, forked from and joined
// back into the caller's stream with events (the caller's stream order is
// kept: everything before the call precedes both kernels, everything after
// follows both).  Created on first use, default priority; the mutex also
// keeps the record / wait pairs of concurrent callers apart.
struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool ok = false, tried = false;
};
std::mutex g_side_mu;
SideStream g_side[64];

}  // namespace


int launch_pack_vectors(bool int4, const uint16_t* in, uint8_t* out, float* scales, int vectors, hipStream_t s) {
    if (vectors <= 0) return 0;
    const dim3 grid((unsigned)((vectors + 15) / 16));
    if (int4) pack_vectors_kernel<true><<<grid, 256, 0, s>>>(in, out, scales, vectors);
    else pack_vectors_kernel<false><<<grid, 256, 0, s>>>(in, out, scales, vectors);
    return 0;
}

int launch_quantize_value_int4(const uint16_t* vt, uint8_t* out, int rows, float inverse_scale, bool edge_only, int valid_rows,
                               hipStream_t s) {
    quantize_value_int4_kernel<<<kModel, kValueThreads, 0, s>>>(vt, out, rows, inverse_scale, edge_only ? 1 : 0, valid_rows);
    return 0;
}

int launch_local_attention(bool packed, const uint16_t* query, const uint16_t* key, const uint8_t* value_fp8,
                           const uint16_t* position, const uint16_t* bias_u, const uint16_t* bias_v, void* output, int rows,
                           int padded_rows, int valid_rows, int left, int right, int value_stride, const uint8_t* packed_key,
                           const float* key_scales, const uint8_t* packed_position, const float* position_scales, hipStream_t s) {
    // Interior tiles t satisfy 16t >= left, 16t + 15 + right < valid_rows and
    // 16t + 16 <= rows: a contiguous range [ib, ie).
    const int tiles = (padded_rows + 15) / 16;
    const int ib = min((left + 15) / 16, tiles);
    const int hi = min(valid_rows - 16 - right, rows - 16);  // largest admissible qb
    const int ie = hi >= 16 * ib ? min(hi / 16 + 1, tiles) : ib;
    const int n = ie - ib;
    const int boundary_wgs = 8 * 4 * (ib + (tiles - ie));
    // Runs of consecutive tiles per head: two resident workgroups per CU
    // (the rings take 70 KB of LDS) for all eight heads.
    const int chunks = n > 0 ? max(1, min(n, 2 * cu_count() / 8)) : 1;
    const int interior_wgs = n > 0 ? 8 * (packed ? chunks : n) : 0;

    auto interior = [&](hipStream_t st) {
        if (packed)
            interior_attention_kernel<true><<<interior_wgs, 256, 0, st>>>(query, key, value_fp8, position, bias_u, bias_v, output,
                                                                          value_stride, packed_key, key_scales, packed_position,
                                                                          position_scales, ib, ie, chunks);
        else
            interior_attention_kernel<false><<<interior_wgs, 256, 0, st>>>(query, key, value_fp8, position, bias_u, bias_v, output,
                                                                           value_stride, nullptr, nullptr, nullptr, nullptr, ib, ie, 1);
    };
    auto boundary = [&](hipStream_t st) {
        if (packed)
            boundary_attention_kernel<true><<<boundary_wgs, 256, 0, st>>>(query, key, value_fp8, position, bias_u, bias_v, output, rows,
                                                                          padded_rows, valid_rows, left, right, value_stride, ib, ie);
        else
            boundary_attention_kernel<false><<<boundary_wgs, 256, 0, st>>>(query, key, value_fp8, position, bias_u, bias_v, output,
                                                                           rows, padded_rows, valid_rows, left, right, value_stride, ib,
                                                                           ie);
    };
    if (interior_wgs == 0 || boundary_wgs == 0) {
        if (interior_wgs) interior(s);
        if (boundary_wgs) boundary(s);
        return 0;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
    std::lock_guard<std::mutex> lock(g_side_mu);
    SideStream* side = dev >= 0 ? &g_side[dev] : nullptr;
    if (side && !side->tried) {
        side->tried = true;
        side->ok = hipStreamCreateWithFlags(&side->stream, hipStreamNonBlocking) == hipSuccess &&
                   hipEventCreateWithFlags(&side->fork, hipEventDisableTiming) == hipSuccess &&
                   hipEventCreateWithFlags(&side->join, hipEventDisableTiming) == hipSuccess;
    }
    // The interior kernel is issued first so that its workgroups take their
    // LDS before the boundary workgroups fill the space left beside them.
    if (side && side->ok && hipEventRecord(side->fork, s) == hipSuccess &&
        hipStreamWaitEvent(side->stream, side->fork, 0) == hipSuccess) {
        interior(s);
        boundary(side->stream);
        if (hipEventRecord(side->join, side->stream) == hipSuccess && hipStreamWaitEvent(s, side->join, 0) == hipSuccess) return 0;
        // could not order the join on the stream: complete the side stream's work here
        if (hipStreamSynchronize(side->stream) != hipSuccess) {
            set_error("attention: the boundary stream did not complete");
            return -3;
        }
        return 0;
    }
    interior(s);
    boundary(s);
    return 0;
}

}  // namespace pk
