// Shared device helpers for the gfx950 quantized-linear kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

namespace pk {

// ---- fp16 --------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ uint16_t f2h(float v) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}
__device__ __forceinline__ float round_f16(float v) { return (float)(_Float16)v; }

// ---- OCP FP8 E4M3 --------------------------------------------------------
// gfx950's v_cvt_pk_fp8_f32 encodes OCP E4M3 with round-to-nearest-even.
// The reference's encoders saturate finite overflow to +-448
// (encoder.cu:557 `__nv_fp8_e4m3`, quant_benchmark.rs:797), so values are
// clamped first; NaN is mapped to 0x7f explicitly because the clamp would
// otherwise turn it into a finite value.
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
    float ca = __builtin_fminf(__builtin_fmaxf(a, -448.0f), 448.0f);
    float cb = __builtin_fminf(__builtin_fmaxf(b, -448.0f), 448.0f);
    uint32_t packed = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xffffu;
    if (a != a) packed = (packed & 0xff00u) | 0x7fu;
    if (b != b) packed = (packed & 0x00ffu) | 0x7f00u;
    return packed;
}
__device__ __forceinline__ uint8_t e4m3(float a) { return (uint8_t)(e4m3x2(a, 0.0f) & 0xff); }

__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
    uint32_t e = (byte >> 3) & 15, m = byte & 7;
    float mag = e == 0 ? (float)m * 0.001953125f
                       : __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
    return (byte & 0x80) ? -mag : mag;
}

// x / s correctly rounded (the IEEE quotient) from inv = 1 / s correctly
// rounded, in three operations: q0 = x * inv is within one ulp of x / s, the
// residual r = q0 * s - x is exact in one fma, and q0 - r * inv rounds to the
// correctly rounded quotient (Markstein's theorem, P. Markstein, "Computation
// of elementary functions on the IBM RISC System/6000 processor", IBM J. Res.
// Dev. 34(1), 1990).  Zeros keep their sign (r is +0 and q0 - (+0) * inv is
// q0).  Requires a finite, nonzero s and x finite or NaN (NaN gives NaN);
// x / s and r must stay clear of the fp32 overflow and underflow ranges.
__device__ __forceinline__ float div_rn(float x, float s, float inv) {
    const float q0 = x * inv;
    const float r = __builtin_fmaf(q0, s, -x);
    return __builtin_fmaf(-r, inv, q0);
}

// ---- integer helpers -------------------------------------------------------
__device__ __forceinline__ int rne_clamp(float v, int lo, int hi) {
    float r = __builtin_rintf(v);
    r = __builtin_fminf(__builtin_fmaxf(r, (float)lo), (float)hi);
    return (v != v) ? 0 : (int)r;
}

// Eight signed nibbles (two per byte) -> eight int8 bytes.  `lo` gets the low
// nibbles of the four bytes, `hi` the high nibbles.  Each byte x in [0,15]
// becomes x - 16*(x >= 8) without carries between bytes.
__device__ __forceinline__ void s4x8_to_s8(uint32_t w, uint32_t& lo, uint32_t& hi) {
    uint32_t l = w & 0x0f0f0f0fu, h = (w >> 4) & 0x0f0f0f0fu;
    lo = ((l ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u;
    hi = ((h ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u;
}

// One butterfly level (off = 1, 2, 4, ..., 32, taken in ascending order),
// without the LDS crossbar: xor 1 and xor 2 are quad permutes; once every lane
// of a quad (of an 8-lane half row) holds the same partial, the row
// half-mirror (mirror) delivers exactly the xor-4 (xor-8) partner's value; for
// xor 16 / 32, v_permlane16_swap / v_permlane32_swap of a register with itself
// hands every lane both values of its pair {v[l & ~off], v[l | off]}, which a
// sum or maximum combines directly (the same operands as own + partner).
template <int CTRL> __device__ __forceinline__ int dpp_mov(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
__device__ __forceinline__ int partner(int v, int off) {  // off <= 8
    switch (off) {
    case 1: return dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    case 2: return dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    case 4: return dpp_mov<0x141>(v);  // row_half_mirror
    default: return dpp_mov<0x140>(v); // row_mirror
    }
}
// {v[l & ~off], v[l | off]} for off = 16 or 32
__device__ __forceinline__ void pair_of(int v, int off, int& a, int& b) {
    if (off == 16) {
        const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = (int)q[0];
        b = (int)q[1];
    } else {
        const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = (int)q[0];
        b = (int)q[1];
    }
}
__device__ __forceinline__ int add_level(int v, int off) {
    if (off <= 8) return v + partner(v, off);
    int a, b;
    pair_of(v, off, a, b);
    return a + b;
}
__device__ __forceinline__ float add_level(float v, int off) {
    if (off <= 8) return v + __int_as_float(partner(__float_as_int(v), off));
    int a, b;
    pair_of(__float_as_int(v), off, a, b);
    return __int_as_float(a) + __int_as_float(b);
}
__device__ __forceinline__ float max_level(float v, int off) {
    if (off <= 8) return __builtin_fmaxf(v, __int_as_float(partner(__float_as_int(v), off)));
    int a, b;
    pair_of(__float_as_int(v), off, a, b);
    return __builtin_fmaxf(__int_as_float(a), __int_as_float(b));
}
__device__ __forceinline__ unsigned long long max_level(unsigned long long v, int off) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    unsigned long long x, y;
    if (off <= 8) {
        x = v;
        y = ((unsigned long long)(uint32_t)partner(hi, off) << 32) | (uint32_t)partner(lo, off);
    } else {
        int la, lb, ha, hb;
        pair_of(lo, off, la, lb);
        pair_of(hi, off, ha, hb);
        x = ((unsigned long long)(uint32_t)ha << 32) | (uint32_t)la;
        y = ((unsigned long long)(uint32_t)hb << 32) | (uint32_t)lb;
    }
    return x > y ? x : y;
}

// Sum over an aligned group of kWidth lanes (16, 32 or 64) in the association
// of the descending xor butterfly (off = kWidth / 2, ..., 2, 1, own +
// partner), the total in every lane of the group.  The xor-32 / xor-16
// levels are permlane swaps; below them DPP row rotations by 8, 4, 2, 1
// stand in for xor 8, 4, 2, 1: after the levels above, the lane a rotation
// reads holds the same value as the xor partner (they differ only in bits
// already reduced), so every lane adds exactly the butterfly's operands.
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_mov<CTRL>(__float_as_int(v))); }
template <int kWidth> __device__ __forceinline__ float sum_desc(float v) {
    int a, b;
    if constexpr (kWidth >= 64) {
        pair_of(__float_as_int(v), 32, a, b);
        v = __int_as_float(a) + __int_as_float(b);
    }
    if constexpr (kWidth >= 32) {
        pair_of(__float_as_int(v), 16, a, b);
        v = __int_as_float(a) + __int_as_float(b);
    }
    v = v + dpp_f<0x128>(v);  // row_ror:8
    v = v + dpp_f<0x124>(v);  // row_ror:4
    v = v + dpp_f<0x122>(v);  // row_ror:2
    v = v + dpp_f<0x121>(v);  // row_ror:1
    return v;
}

// ---- reductions over a 256-thread block ------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 1; off <= 32; off <<= 1) v = max_level(v, off);
    return v;
}

// SiLU with the hardware reciprocal (<= 1 ulp) instead of an IEEE division.
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Q4_K group g (0..7) of a superblock header: d * scale and dmin * min
// (linear.cu:431-457; 6-bit scale/min pairs, groups 4..7 split over bytes).
__device__ __forceinline__ void q4k_coeffs(const uint4& h, int g, float& a, float& b) {
    auto byte = [&](int i) { return ((i < 4 ? h.y : (i < 8 ? h.z : h.w)) >> ((i & 3) * 8)) & 0xffu; };
    uint32_t sc, mn;
    if (g < 4) {
        sc = byte(g) & 63u;
        mn = byte(g + 4) & 63u;
    } else {
        sc = (byte(g + 4) & 15u) | ((byte(g - 4) >> 6) << 4);
        mn = (byte(g + 4) >> 4) | ((byte(g) >> 6) << 4);
    }
    a = h2f((uint16_t)(h.x & 0xffffu)) * (float)sc;
    b = h2f((uint16_t)(h.x >> 16)) * (float)mn;
}

// Eight nibbles (byte j of lo / hi, j = 0..3) -> f16(a * q - b), in k order.
__device__ __forceinline__ uint4 q4k_decode8(uint32_t lo, uint32_t hi, float a, float b) {
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t w = j < 2 ? lo : hi;
        const float q0 = (float)((w >> (16 * (j & 1))) & 0xffu), q1 = (float)((w >> (16 * (j & 1) + 8)) & 0xffu);
        r[j] = (uint32_t)f2h(a * q0 - b) | ((uint32_t)f2h(a * q1 - b) << 16);
    }
    return uint4{r[0], r[1], r[2], r[3]};
}

}  // namespace pk
