// Activation quantizers, load-time weight packers and LayerNorm producers.
// All are HBM-bound byte work: one wave per row for the per-row activation
// kinds, one 256-thread block per row for the load-time weight packers, 8
// elements (16 bytes of fp16) per thread for the elementwise kinds.
#include "pk_kernels.hpp"

namespace pk {

// linear.cu:537-547, encoder.cu:549-559: e4m3(f16 * inverse_scale).
__global__ void quantize_fp8_static_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                           float inverse_scale, size_t elements) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i + 8 <= elements) {
        const uint4 raw = *(const uint4*)(in + i);
        const uint16_t* h = (const uint16_t*)&raw;
        uint32_t w0 = e4m3x2(h2f(h[0]) * inverse_scale, h2f(h[1]) * inverse_scale) |
                      (e4m3x2(h2f(h[2]) * inverse_scale, h2f(h[3]) * inverse_scale) << 16);
        uint32_t w1 = e4m3x2(h2f(h[4]) * inverse_scale, h2f(h[5]) * inverse_scale) |
                      (e4m3x2(h2f(h[6]) * inverse_scale, h2f(h[7]) * inverse_scale) << 16);
        *(uint2*)(out + i) = uint2{w0, w1};
    } else {
        for (size_t j = i; j < elements; ++j) out[j] = e4m3(h2f(in[j]) * inverse_scale);
    }
}

// linear.cu:549-560: rne(clamp(f16 * inverse_scale, +-127)).
__global__ void quantize_int8_static_kernel(const uint16_t* __restrict__ in, int8_t* __restrict__ out,
                                            float inverse_scale, size_t elements) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const size_t end = i + 8 <= elements ? i + 8 : elements;
    for (size_t j = i; j < end; ++j) {
        const float s = __builtin_fminf(127.0f, __builtin_fmaxf(-127.0f, h2f(in[j]) * inverse_scale));
        out[j] = (int8_t)__builtin_rintf(s);
    }
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

// Byte packing and the per-element fast paths of the row quantizers.  They
// assume a finite scale (rows with an inf or NaN take the exact path).
//  * INT8: |x / scale| <= 127 (1 + 2^-23) when scale = RN(max|x| / 127), so
//    rne needs no clamp; adding 1.5 * 2^23 leaves rne(q) in the low mantissa
//    bits, whose low byte is the two's-complement int8.
//  * FP8: |x / scale| can exceed 448 by an ulp; the clamp keeps the
//    conversion saturating.
__device__ __forceinline__ uint32_t rne_bits(float q) { return __builtin_bit_cast(uint32_t, q + 12582912.0f); }
__device__ __forceinline__ uint32_t low_bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// FP6 e3m2 (sign, 3 exponent bits of bias 3, 2 mantissa bits) of an INT4 code
// in -8..7 (the low byte of q as int8), exact: 1..8 are 2^e (1 + m / 4).
__device__ __forceinline__ uint32_t e3m2_of_code(uint32_t q) {
    const int v = (int)(int8_t)(q & 0xffu);
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    // magnitudes 0..8 as 6-bit fields of one 64-bit constant
    constexpr uint64_t kMag = 0x00ull | 0x0cull << 6 | 0x10ull << 12 | 0x12ull << 18 | 0x14ull << 24 | 0x15ull << 30 |
                              0x16ull << 36 | 0x17ull << 42 | 0x18ull << 48;
    return (uint32_t)(kMag >> (6 * a)) & 0x1fu | (v < 0 ? 0x20u : 0u);
}

// e3m2 bytes of four int8 codes in -8..7 (one per byte of c): per-byte
// magnitude, the e3m2 magnitudes of 0..7 from one byte permute of an 8-byte
// table, 8 (only -8 has it) patched in, then the sign bit.
__device__ __forceinline__ uint32_t e3m2_bytes4(uint32_t c) {
    const uint32_t neg = (c >> 7) & 0x01010101u;                                      // 1 in each negative byte
    const uint32_t a = (c ^ (neg * 0xffu)) + neg;                                     // |code| per byte, 0..8
    const uint32_t big = (a >> 3) & 0x01010101u;                                      // |code| == 8
    const uint32_t lut = __builtin_amdgcn_perm(0x17161514u, 0x12100c00u, a & 0x07070707u);  // 0..3 | 4..7
    return lut | big * 0x18u | neg * 0x20u;
}

// FP6 chunk layout of 16 codes (one 16-byte chunk: code j at bits 6j.. of its
// first 12 bytes, then 4 zero bytes).  Lane t = lane % 4 of a quad holds
// codes 4t..4t+3 of the chunk (the int8 bytes of c) and writes its dword t:
// the 24 bits of its own codes shifted into place and the first bits of lane
// t + 1's.
__device__ __forceinline__ uint32_t e3m2_chunk_dword(uint32_t c, int lane) {
    const uint32_t e = e3m2_bytes4(c);
    const uint32_t piece = (e & 0x3fu) | ((e >> 2) & 0xfc0u) | ((e >> 4) & 0x3f000u) | ((e >> 6) & 0xfc0000u);
    const uint32_t next = (uint32_t)dpp_mov<0xF9>((int)piece);  // quad_perm [1, 2, 3, 3]: lane t + 1's piece
    const int t = lane & 3;
    return t == 3 ? 0u : (piece >> (8 * t)) | (next << (24 - 8 * t));
}
__device__ __forceinline__ uint32_t e4m3x4_sat(float a, float b, float c, float d) {
    const float lo = -448.0f, hi = 448.0f;
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, lo, hi), __builtin_amdgcn_fmed3f(b, lo, hi), 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, lo, hi), __builtin_amdgcn_fmed3f(d, lo, hi), (int)w, true);
}
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// max over two fp16 magnitudes per word, as integers: for non-NaN halves the
// order of (bits & 0x7fff) is the order of |x|; any value above 0x7c00 is NaN.
__device__ __forceinline__ uint32_t abs_max16(uint32_t acc, uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, acc), __builtin_bit_cast(u16x2, w & 0x7fff7fffu)));
}

// Dynamic per-row quantization of fp16 rows [rows x k] (k % 8 == 0).
//   kind 0: FP8,  scale = max|x| / 448 (encoder.cu:1129-1180, :264-292)
//   kind 1: INT8, scale = max|x| / 127 (per-token dynamic INT8)
//   kind 2: INT4, scale = max(max(x/7, -x/8)), nibble pairs (encoder.cu:264-290)
// Scale is 1 for a row without a positive maximum; rows >= valid_rows are
// written as zeros with scale 1 (padding rows, encoder.cu:226-237).
// One wave per row (four rows per 256-thread block, rows strided over the
// grid): a lane holds up to kCh 16-byte chunks of its row in registers as
// fp16 (with kPrefetch it issues the loads of its next row before it works
// on the current one); the maximum is a wave reduction (order-free); rows
// longer than 64 * kCh * 8 are read a second time for the quantization pass.
// Kinds 0 and 1 fold |x| as packed integers and quantize with the fast paths
// above unless the row holds an inf or NaN; kind 2 and those rows divide.
template <int kind, int kCh, bool kPrefetch>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                            float* __restrict__ scales, int rows, int k, int valid_rows) {
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * 4;
    const int chunks = k >> 3;
    const int out_row = kind == 2 ? k / 2 : k;
    uint4 cur[kCh], nxt[kPrefetch ? kCh : 1];
    auto load = [&](int row, uint4* r) {
        const uint16_t* x = in + (size_t)row * k;
#pragma unroll
        for (int i = 0; i < kCh; ++i) {
            const int c = lane + 64 * i;
            r[i] = (row < valid_rows && c < chunks) ? *(const uint4*)(x + c * 8) : uint4{0, 0, 0, 0};
        }
    };
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (kPrefetch && row < rows) load(row, cur);
    for (; row < rows; row += nw) {
        if constexpr (kPrefetch) {
            if (row + nw < rows) load(row + nw, nxt);
        } else {
            load(row, cur);
        }
        const uint16_t* x = in + (size_t)row * k;
        uint8_t* o = out + (size_t)row * out_row;
        if (row >= valid_rows) {
            for (int c = lane; c < chunks; c += 64) {
                if constexpr (kind == 2) *(uint32_t*)(o + c * 4) = 0u;
                else *(uint2*)(o + c * 8) = uint2{0, 0};
            }
            if (lane == 0) scales[row] = 1.0f;
        } else {
            float m = 0.0f;
            bool exact = true;
            if constexpr (kind == 2) {
                auto fold = [&](const uint4& r) {
                    const uint16_t* h = (const uint16_t*)&r;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float v = h2f(h[j]);
                        m = __builtin_fmaxf(m, __builtin_fmaxf(v / 7.0f, -v / 8.0f));
                    }
                };
#pragma unroll
                for (int i = 0; i < kCh; ++i) fold(cur[i]);
                for (int c = lane + 64 * kCh; c < chunks; c += 64) fold(*(const uint4*)(x + c * 8));
                m = wave_max(m);
            } else {
                uint32_t acc = 0;
                auto fold = [&](const uint4& r) { acc = abs_max16(abs_max16(abs_max16(abs_max16(acc, r.x), r.y), r.z), r.w); };
#pragma unroll
                for (int i = 0; i < kCh; ++i) fold(cur[i]);
                for (int c = lane + 64 * kCh; c < chunks; c += 64) fold(*(const uint4*)(x + c * 8));
                const uint32_t lane_max = (acc & 0xffffu) > (acc >> 16) ? (acc & 0xffffu) : (acc >> 16);
                const uint32_t bits = __builtin_amdgcn_readfirstlane((uint32_t)wave_max((float)lane_max));
                exact = bits >= 0x7c00u;  // inf or NaN in the row
                // NaN is ignored by the maximum (fmaxf), as in the oracle
                if (exact) {
                    m = 0.0f;
#pragma unroll
                    for (int i = 0; i < kCh; ++i) {
                        const uint16_t* h = (const uint16_t*)&cur[i];
#pragma unroll
                        for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(h[j])));
                    }
                    for (int c = lane + 64 * kCh; c < chunks; c += 64) {
                        const uint4 r = *(const uint4*)(x + c * 8);
                        const uint16_t* h = (const uint16_t*)&r;
                        for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(h[j])));
                    }
                    m = wave_max(m);
                } else {
                    m = h2f((uint16_t)bits);
                }
            }
            const float scale = m > 0.0f ? (kind == 0 ? m / 448.0f : (kind == 1 ? m / 127.0f : m)) : 1.0f;
            const float inv = 1.0f / scale;
            if (lane == 0) scales[row] = scale;
            auto emit = [&](int c, const uint4& r) {
                const uint16_t* h = (const uint16_t*)&r;
                if constexpr (kind == 2) {
                    uint32_t w = 0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) w |= ((uint32_t)rne_clamp(h2f(h[j]) / scale, -8, 7) & 15u) << (4 * j);
                    *(uint32_t*)(o + c * 4) = w;
                } else if (exact) {
                    uint32_t w[2] = {0, 0};
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const float a = h2f(h[j]) / scale, b = h2f(h[j + 1]) / scale;
                        const uint32_t pair = kind == 0 ? e4m3x2(a, b)
                                                        : (((uint32_t)rne_clamp(a, -127, 127) & 255u) | (((uint32_t)rne_clamp(b, -127, 127) & 255u) << 8));
                        w[j >> 2] |= pair << (8 * (j & 3));
                    }
                    *(uint2*)(o + c * 8) = uint2{w[0], w[1]};
                } else {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = div_rn(h2f(h[j]), scale, inv);
                    uint2 w;
                    if constexpr (kind == 0) {
                        w.x = e4m3x4_sat(v[0], v[1], v[2], v[3]);
                        w.y = e4m3x4_sat(v[4], v[5], v[6], v[7]);
                    } else {
                        w.x = low_bytes4(rne_bits(v[0]), rne_bits(v[1]), rne_bits(v[2]), rne_bits(v[3]));
                        w.y = low_bytes4(rne_bits(v[4]), rne_bits(v[5]), rne_bits(v[6]), rne_bits(v[7]));
                    }
                    *(uint2*)(o + c * 8) = w;
                }
            };
#pragma unroll
            for (int i = 0; i < kCh; ++i) {
                const int c = lane + 64 * i;
                if (c < chunks) emit(c, cur[i]);
            }
            for (int c = lane + 64 * kCh; c < chunks; c += 64) emit(c, *(const uint4*)(x + c * 8));
        }
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < kCh; ++i) cur[i] = nxt[i];
        }
    }
}

// ---- INT8 rows in 2:4 form plus an overflow list (activation-sparse FF2) ----
//
// Quartet (4 consecutive int8 of a row) -> the reference's 2:4 selection
// (encoder.cu:685-704, there on e4m3 bytes): keep the two largest |v|, ties to
// the lower index, in index order; returns the two kept bytes in bits 0-15,
// idx0 | idx1 << 2 in bits 16-19, and in `drop` bit i set for each nonzero
// byte i that was not kept (at most two).  The kept pair plus the dropped
// nonzeros are the quartet, exactly.
__device__ __forceinline__ uint32_t compress_i8_quartet(uint32_t packed, uint32_t& drop, uint32_t& rest) {
    // |v| per byte (0 .. 128) without carries between bytes: (x ^ 0xff) + 1 for negatives
    const uint32_t sgn = (packed >> 7) & 0x01010101u;
    const uint32_t mag = (packed ^ (sgn * 255u)) + sgn;
    // keys 4 |v_i| + (3 - i) are distinct and order the bytes by magnitude, ties
    // to the lower index; the two largest keys are the kept pair
    const uint32_t k0 = ((mag & 0xffu) << 2) | 3u, k1 = (((mag >> 8) & 0xffu) << 2) | 2u;
    const uint32_t k2 = (((mag >> 16) & 0xffu) << 2) | 1u, k3 = (mag >> 24) << 2;
    const uint32_t h01 = max(k0, k1), l01 = min(k0, k1), h23 = max(k2, k3), l23 = min(k2, k3);
    const uint32_t top = max(h01, h23), next = max(min(h01, h23), max(l01, l23));
    const uint32_t ia = 3u - (top & 3u), ib = 3u - (next & 3u);
    const uint32_t i0 = min(ia, ib), i1 = max(ia, ib);
    // bytes i0, i1 of the quartet to bytes 0, 1 (selector 0x0c gives zero)
    const uint32_t d = __builtin_amdgcn_perm(0u, packed, i0 | (i1 << 8) | 0x0c0c0000u);
    // nonzero bytes: |v| + 0x7f sets the byte's top bit iff |v| > 0 (no carry out at 128)
    const uint32_t t = (mag + 0x7f7f7f7fu) & 0x80808080u;
    const uint32_t nz = ((t >> 7) & 1u) | ((t >> 14) & 2u) | ((t >> 21) & 4u) | ((t >> 28) & 8u);
    const uint32_t others = 15u & ~((1u << i0) | (1u << i1));
    drop = nz & others;
    // the residual pair: the two positions not kept, ascending, with their bytes
    const uint32_t j0 = (uint32_t)__builtin_ctz(others), j1 = 31u - (uint32_t)__builtin_clz(others);
    rest = (__builtin_amdgcn_perm(0u, packed, j0 | (j1 << 8) | 0x0c0c0000u) & 0xffffu) | ((j0 | (j1 << 2)) << 16);
    return (d & 0xffffu) | ((i0 | (i1 << 2)) << 16);
}

// Dynamic per-row INT8 quantization (the arithmetic of quantize_rows_kernel
// kind 1: scale = max|x| / 127, 1 for rows without a positive maximum, rows
// >= valid_rows zero with scale 1), written as 2:4 data [rows x k/2] and
// metadata [rows x k/8] (quartet p's idx0 | idx1 << 2 at bits 4 (p % 2) of
// byte p / 2) plus, per row, the nonzeros the 2:4 selection dropped:
// ovf_count[row] entries at ovf[row * k/2 ...], each (kk << 8) | byte for
// element kk, in ascending kk.  At most two per quartet, so k/2 entries per
// row always suffice.  With data2 / meta2 (both or neither) the residual 2:4
// form as well: per quartet the two positions not kept, ascending, with their
// bytes, in the layout of data / meta.  One wave per row, the row held in registers (k <= 64 *
// kCh * 8); a lane handles chunk c = lane + 64 i (8 elements = 2 quartets) and
// the overflow slots are a wave prefix sum over the lanes' counts.
template <int kCh>
__global__ __launch_bounds__(256) void quantize_rows_sp24_kernel(const uint16_t* __restrict__ in, uint8_t* __restrict__ data,
                                                                 uint8_t* __restrict__ meta, float* __restrict__ scales,
                                                                 uint32_t* __restrict__ ovf_count, uint32_t* __restrict__ ovf,
                                                                 uint8_t* __restrict__ data2, uint8_t* __restrict__ meta2,
                                                                 int rows, int k, int valid_rows) {
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * 4;
    const int chunks = k >> 3;
    for (int row = blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += nw) {
        const bool live = row < valid_rows;
        const uint16_t* x = in + (size_t)row * k;
        uint4 cur[kCh];
#pragma unroll
        for (int i = 0; i < kCh; ++i) {
            const int c = lane + 64 * i;
            cur[i] = (live && c < chunks) ? *(const uint4*)(x + c * 8) : uint4{0, 0, 0, 0};
        }
        uint32_t acc = 0;
#pragma unroll
        for (int i = 0; i < kCh; ++i) acc = abs_max16(abs_max16(abs_max16(abs_max16(acc, cur[i].x), cur[i].y), cur[i].z), cur[i].w);
        const uint32_t lane_max = (acc & 0xffffu) > (acc >> 16) ? (acc & 0xffffu) : (acc >> 16);
        const uint32_t bits = __builtin_amdgcn_readfirstlane((uint32_t)wave_max((float)lane_max));
        const bool exact = bits >= 0x7c00u;  // inf or NaN in the row: plain division
        float m;
        if (exact) {
            m = 0.0f;
#pragma unroll
            for (int i = 0; i < kCh; ++i) {
                const uint16_t* h = (const uint16_t*)&cur[i];
#pragma unroll
                for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(h[j])));
            }
            m = wave_max(m);
        } else {
            m = h2f((uint16_t)bits);
        }
        const float scale = m > 0.0f ? m / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        if (lane == 0) scales[row] = scale;
        uint8_t* drow = data + (size_t)row * (k >> 1);
        uint8_t* mrow = meta + (size_t)row * (k >> 3);
        uint32_t* orow = ovf + (size_t)row * (k >> 1);
        uint32_t base = 0;
#pragma unroll
        for (int i = 0; i < kCh; ++i) {
            const int c = lane + 64 * i;
            const uint16_t* h = (const uint16_t*)&cur[i];
            uint32_t w[2];
            if (exact) {
                w[0] = w[1] = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) w[j >> 2] |= ((uint32_t)rne_clamp(h2f(h[j]) / scale, -127, 127) & 255u) << (8 * (j & 3));
            } else {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = div_rn(h2f(h[j]), scale, inv);
                w[0] = low_bytes4(rne_bits(v[0]), rne_bits(v[1]), rne_bits(v[2]), rne_bits(v[3]));
                w[1] = low_bytes4(rne_bits(v[4]), rne_bits(v[5]), rne_bits(v[6]), rne_bits(v[7]));
            }
            uint32_t drop0, drop1, r0, r1;
            const uint32_t q0 = compress_i8_quartet(w[0], drop0, r0);
            const uint32_t q1 = compress_i8_quartet(w[1], drop1, r1);
            const uint32_t drops = drop0 | (drop1 << 4);  // element j of the chunk
            const uint32_t n = (uint32_t)__builtin_popcount(drops);
            // exclusive prefix of n over the lanes below (n <= 4: three bit planes)
            const uint64_t b0 = __builtin_amdgcn_ballot_w64((n & 1u) != 0);
            const uint64_t b1 = __builtin_amdgcn_ballot_w64((n & 2u) != 0);
            const uint64_t b2 = __builtin_amdgcn_ballot_w64((n & 4u) != 0);
            auto below_count = [](uint64_t b) {  // set bits of b in the lanes below this one
                return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
            };
            const uint32_t pre = below_count(b0) + 2u * below_count(b1) + 4u * below_count(b2);
            if (c < chunks) {
                *(uint32_t*)(drow + 4 * c) = (q0 & 0xffffu) | (q1 << 16);
                mrow[c] = (uint8_t)(((q0 >> 16) & 15u) | (((q1 >> 16) & 15u) << 4));
                if (data2) {
                    *(uint32_t*)(data2 + (size_t)row * (k >> 1) + 4 * c) = (r0 & 0xffffu) | (r1 << 16);
                    meta2[(size_t)row * (k >> 3) + c] = (uint8_t)(((r0 >> 16) & 15u) | (((r1 >> 16) & 15u) << 4));
                }
                uint32_t slot = base + pre;
                for (uint32_t d = drops; d != 0; d &= d - 1) {
                    const int j = __builtin_ctz(d);
                    orow[slot++] = ((uint32_t)(8 * c + j) << 8) | ((w[j >> 2] >> (8 * (j & 3))) & 255u);
                }
            }
            base += (uint32_t)__builtin_popcountll(b0) + 2u * (uint32_t)__builtin_popcountll(b1) + 4u * (uint32_t)__builtin_popcountll(b2);
        }
        if (lane == 0) ovf_count[row] = base;
    }
}

// Per-row weight packers (load-time derivation, encoder.rs:361-422 and
// quant_benchmark.rs:779-829), rows of fp16 [n x k]:
//   kind 0: FP8  scale = max|w| / 448 (1 for zero rows)
//   kind 1: INT8 scale = max|w| / 127 (1 for zero rows)
//   kind 2: INT4 scale = max(max(w/7, -w/8)) folded from 0; zero rows keep
//           scale 0 and pack to zero bytes (encoder.rs:378-407).
template <int kind>
__global__ __launch_bounds__(256) void pack_rows_kernel(const uint16_t* __restrict__ w, uint8_t* __restrict__ out,
                                                        float* __restrict__ scales, int k) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const uint16_t* x = w + (size_t)row * k;
    float m = 0.0f;
    for (int i = threadIdx.x; i < k; i += 256) {
        const float v = h2f(x[i]);
        m = kind == 2 ? __builtin_fmaxf(m, __builtin_fmaxf(v / 7.0f, -v / 8.0f)) : __builtin_fmaxf(m, __builtin_fabsf(v));
    }
    m = block_max_256(m, red);
    const float scale = kind == 2 ? m : (m > 0.0f ? m / (kind == 0 ? 448.0f : 127.0f) : 1.0f);
    if (threadIdx.x == 0) scales[row] = scale;
    if constexpr (kind == 2) {
        for (int j = threadIdx.x; j < k / 2; j += 256) {
            const int a = rne_clamp(h2f(x[2 * j]) / scale, -8, 7);
            const int b = rne_clamp(h2f(x[2 * j + 1]) / scale, -8, 7);
            out[(size_t)row * (k / 2) + j] = (uint8_t)((a & 15) | ((b & 15) << 4));
        }
    } else {
        for (int i = threadIdx.x; i < k; i += 256) {
            const float v = h2f(x[i]) / scale;
            out[(size_t)row * k + i] = kind == 0 ? e4m3(v) : (uint8_t)(int8_t)rne_clamp(v, -127, 127);
        }
    }
}

// Group-wise asymmetric INT4 packer, one thread per (row, 128-K group):
// lo = min(0, min w), hi = max(0, max w), s = fp16((hi - lo) / 15) (1 if not
// positive), z = clamp(rne(-lo / s), 0, 15), q = clamp(rne(w / s) + z, 0, 15).
// Device layout: word j of a row holds k = 8j .. 8j+7; byte b of the word
// holds k = 8j+b in its low nibble and k = 8j+4+b in its high nibble, so
// (w & 0x0f0f0f0f) and (w >> 4 & 0x0f0f0f0f) are the eight levels in k order.
__global__ void pack_g128_kernel(const uint16_t* __restrict__ w, uint32_t* __restrict__ q, uint16_t* __restrict__ scales,
                                 uint16_t* __restrict__ zeros, int n, int k) {
    const int groups = k / 128;
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n * groups) return;
    const int row = id / groups, g = id - row * groups;
    const uint16_t* x = w + (size_t)row * k + g * 128;
    float lo = 0.0f, hi = 0.0f;
    for (int i = 0; i < 128; ++i) {
        const float v = h2f(x[i]);
        lo = __builtin_fminf(lo, v);
        hi = __builtin_fmaxf(hi, v);
    }
    float s = round_f16((hi - lo) / 15.0f);
    if (!(s > 0.0f)) s = 1.0f;
    const int z = rne_clamp(-lo / s, 0, 15);
    scales[id] = f2h(s);
    zeros[id] = f2h((float)z);
    for (int j = 0; j < 16; ++j) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) {
            int level = rne_clamp(h2f(x[8 * j + i]) / s, -64, 64) + z;
            level = level < 0 ? 0 : (level > 15 ? 15 : level);
            word |= (uint32_t)level << (8 * (i & 3) + 4 * (i >> 2));
        }
        q[(size_t)row * (k / 8) + g * 16 + j] = word;
    }
}

// LayerNorm over 1024 features + dynamic per-row FP8 / INT4 quantization
// (encoder.cu:211-306), one wave per row (four rows per 256-thread block,
// rows strided over the grid).  Lane l holds features 4l..4l+3 of each
// 256-feature quarter i (8-byte loads, 4-byte FP8 / 2-byte INT4 stores) and
// its gamma and beta in registers.  The sums keep the reference's reduction
// shape, whose 256 partials are
// partial(t) = ((x[t] + x[t+256]) + x[t+512]) + x[t+768]: lane l forms
// partials 4l..4l+3 and writes them to its wave's slice of LDS; lane l then
// reads partials t = l, l+64, l+128, l+192, lanes 0..31 form
// (p[l] + p[l+128]) + (p[l+64] + p[l+192]) and add lane l+32's value of the
// same expression (= (p[l+32] + p[l+160]) + (p[l+96] + p[l+224])), and a
// shuffle-down tree over 32 lanes finishes (encoder.cu:36-54).  inverse_std =
// 1 / sqrtf(.) correctly rounded.
__device__ __forceinline__ float ln_tree_sum(const float (&p)[4]) {
    // (p[l] + p[l+128]) + (p[l+64] + p[l+192]) in lane l, then the tree over
    // pairs (l, l + off) for off = 32, 16, ..., 1.  Lane 0 holds the total:
    // at every level the lanes it depends on (l < 2 off) read exactly their
    // partner l + off -- permlane32 / permlane16 swaps for off = 32 / 16, DPP
    // row shifts (lane l reads lane l + off of its 16-lane row) below.
    float r = (p[0] + p[2]) + (p[1] + p[3]);
    int a, b;
    pair_of(__float_as_int(r), 32, a, b);
    r = __int_as_float(a) + __int_as_float(b);
    pair_of(__float_as_int(r), 16, a, b);
    r = __int_as_float(a) + __int_as_float(b);
    r = r + __int_as_float(dpp_mov<0x108>(__float_as_int(r)));  // row_shl:8
    r = r + __int_as_float(dpp_mov<0x104>(__float_as_int(r)));  // row_shl:4
    r = r + __int_as_float(dpp_mov<0x102>(__float_as_int(r)));  // row_shl:2
    r = r + __int_as_float(dpp_mov<0x101>(__float_as_int(r)));  // row_shl:1
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(r)));
}

// LDS ordering inside one wave: the wave's LDS operations execute in order;
// the fences keep the compiler from moving them across this point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum of the 256 partials part[t] (lane l holds t = 4l..4l+3) in the tree
// above, through the wave's 256-float LDS slice.
__device__ __forceinline__ float ln_partials_sum(const float (&part)[4], float* slice) {
    const int lane = threadIdx.x & 63;
    *(float4*)(slice + 4 * lane) = float4{part[0], part[1], part[2], part[3]};
    wave_lds_sync();
    const float p[4] = {slice[lane], slice[lane + 64], slice[lane + 128], slice[lane + 192]};
    wave_lds_sync();
    return ln_tree_sum(p);
}

//
// Quantization: y is finite unless mean, inverse_std, gamma or beta is not
// (normalized values are bounded by sqrt(1024)) or its fp16 rounding
// overflows; rows where either may have happened take the exact per-element
// divisions, the others the fast paths: the maximum comes from the row's
// extremes (x / 7 rounded is monotone in x), the quotients from div_rn and
// the INT4 codes need no clamp (|y / scale| <= 8 (1 + 2^-23)).
// kCodes (with kInt4): the INT4 codes as int8 bytes [rows x 1024] instead of
// nibble pairs -- the operand the INT8 MFMA consumes, which has no 4-bit form.
// kFp6 (with kCodes): the same codes as FP6 e3m2 chunks (e3m2_chunk_dword),
// the operand of the f8f6f4 MFMA at the FP6 rate; same row size and stores.
template <bool kInt4, bool kCodes = false, bool kFp6 = false>
__global__ __launch_bounds__(256) void layer_norm_quantize_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ gamma,
                                                                  const uint16_t* __restrict__ beta, uint8_t* __restrict__ out,
                                                                  float* __restrict__ scales, uint16_t* __restrict__ normalized,
                                                                  int rows, int padded_rows, float epsilon) {
    __shared__ __attribute__((aligned(16))) float red[4][2][256];
    // gamma and beta as fp32 in LDS, read per row (registers stay free for
    // occupancy): gb[i][lane] holds features 256 i + 4 lane .. + 3
    __shared__ __attribute__((aligned(16))) float4 gb_s[2][4][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nw = gridDim.x * 4;
    // element e = 4 i + u of a lane is feature f = 256 i + 4 lane + u
    bool gb_finite = true;
    {
        const int i = wave;  // wave i stages quarter i
        const uint2 gw = *(const uint2*)(gamma + 256 * i + 4 * lane);
        const uint2 bw = *(const uint2*)(beta + 256 * i + 4 * lane);
        const uint16_t* gh = (const uint16_t*)&gw;
        const uint16_t* bh = (const uint16_t*)&bw;
        gb_s[0][i][lane] = float4{h2f(gh[0]), h2f(gh[1]), h2f(gh[2]), h2f(gh[3])};
        gb_s[1][i][lane] = float4{h2f(bh[0]), h2f(bh[1]), h2f(bh[2]), h2f(bh[3])};
#pragma unroll
        for (int u = 0; u < 4; ++u) gb_finite = gb_finite && __builtin_isfinite(h2f(gh[u])) && __builtin_isfinite(h2f(bh[u]));
    }
    gb_finite = __syncthreads_and(gb_finite);
    static_assert(kInt4 || !kCodes, "codes are an INT4 output");
    const size_t out_row = (kInt4 && !kCodes) ? 512 : 1024;
    for (int row = blockIdx.x * 4 + wave; row < padded_rows; row += nw) {
        uint8_t* o = out + (size_t)row * out_row;
        uint16_t* nrm = normalized ? normalized + (size_t)row * 1024 : nullptr;
        if (row >= rows) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (kInt4 && !kCodes) *(uint16_t*)(o + 128 * i + 2 * lane) = 0;
                else *(uint32_t*)(o + 256 * i + 4 * lane) = 0u;
                if (nrm) *(uint2*)(nrm + 256 * i + 4 * lane) = uint2{0, 0};
            }
            if (lane == 0) scales[row] = 1.0f;
            continue;
        }
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint2 w = *(const uint2*)(in + (size_t)row * 1024 + 256 * i + 4 * lane);
            const uint16_t* h = (const uint16_t*)&w;
#pragma unroll
            for (int u = 0; u < 4; ++u) v[4 * i + u] = h2f(h[u]);
        }
        float part[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) part[u] = ((v[u] + v[4 + u]) + v[8 + u]) + v[12 + u];
        const float mean = ln_partials_sum(part, red[wave][0]) / 1024.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float sq = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = v[4 * i + u] - mean;
                sq += d * d;
            }
            part[u] = sq;
        }
        const float inverse_std = 1.0f / sqrtf(ln_partials_sum(part, red[wave][1]) / 1024.0f + epsilon);
        float hi = 0.0f, lo = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint16_t h[4];
            const float4 g4 = gb_s[0][i][lane], b4 = gb_s[1][i][lane];
            const float g[4] = {g4.x, g4.y, g4.z, g4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = 4 * i + u;
                h[u] = f2h((v[e] - mean) * inverse_std * g[u] + b[u]);
                v[e] = h2f(h[u]);
                hi = __builtin_fmaxf(hi, v[e]);
                lo = __builtin_fminf(lo, v[e]);
            }
            if (nrm) *(uint2*)(nrm + 256 * i + 4 * lane) = uint2{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
        }
        hi = wave_max(hi);
        lo = -wave_max(-lo);
        // wave-uniform: every lane holds the same reductions
        const bool fast = __builtin_amdgcn_readfirstlane(gb_finite && __builtin_isfinite(mean) && __builtin_isfinite(inverse_std) &&
                                                         __builtin_isfinite(hi) && __builtin_isfinite(lo));
        float m;
        if (fast) {
            m = kInt4 ? __builtin_fmaxf(div_rn(hi, 7.0f, 1.0f / 7.0f), -lo / 8.0f) : __builtin_fmaxf(hi, -lo);
        } else {
            m = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e)
                m = kInt4 ? __builtin_fmaxf(m, __builtin_fmaxf(v[e] / 7.0f, -v[e] / 8.0f)) : __builtin_fmaxf(m, __builtin_fabsf(v[e]));
            m = wave_max(m);
        }
        const float scale = m > 0.0f ? (kInt4 ? m : m / 448.0f) : 1.0f;
        const float inv = 1.0f / scale;
        if (lane == 0) scales[row] = scale;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float* y = v + 4 * i;
            if constexpr (kInt4) {
                uint32_t q[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) q[u] = fast ? rne_bits(div_rn(y[u], scale, inv)) : (uint32_t)rne_clamp(y[u] / scale, -8, 7);
                if constexpr (kFp6)
                    *(uint32_t*)(o + 256 * i + 4 * lane) = e3m2_chunk_dword(low_bytes4(q[0], q[1], q[2], q[3]), lane);
                else if constexpr (kCodes)
                    *(uint32_t*)(o + 256 * i + 4 * lane) = low_bytes4(q[0], q[1], q[2], q[3]);
                else
                    *(uint16_t*)(o + 128 * i + 2 * lane) =
                        (uint16_t)((q[0] & 15u) | ((q[1] & 15u) << 4) | ((q[2] & 15u) << 8) | ((q[3] & 15u) << 12));
            } else {
                const uint32_t w = fast ? e4m3x4_sat(div_rn(y[0], scale, inv), div_rn(y[1], scale, inv), div_rn(y[2], scale, inv),
                                                     div_rn(y[3], scale, inv))
                                        : (e4m3x2(y[0] / scale, y[1] / scale) | (e4m3x2(y[2] / scale, y[3] / scale) << 16));
                *(uint32_t*)(o + 256 * i + 4 * lane) = w;
            }
        }
    }
}

// LayerNorm pair (encoder.cu:128-209): layer i's norm_out and layer i+1's
// norm_ff1 from one read of the row.  first = fp16(LN(x; weight, bias)) is
// written to `out` (the next FF1 residual needs it); second =
// fp16(LN(first; next_weight, next_bias)) goes to `next_out` as fp16, or, when
// inverse_scale != 0, as e4m3(second * inverse_scale) bytes (the fixed-scale
// FF1 FP8 input).  Both LayerNorms use the reduction shape of
// layer_norm_quantize_kernel above (the reference's second one sums the four
// rounded first values of a thread in the same order as the first sums x).
// Rows in [rows, padded_rows) are written as zeros.  Same wave-per-row
// layout; the four fp16 parameter vectors are staged as fp32 in LDS.
template <bool kFp8>
__global__ __launch_bounds__(256) void layer_norm_pair_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ g1,
                                                              const uint16_t* __restrict__ b1, uint16_t* __restrict__ out,
                                                              const uint16_t* __restrict__ g2, const uint16_t* __restrict__ b2,
                                                              void* __restrict__ next_out, int rows, int padded_rows, float epsilon,
                                                              float inverse_scale) {
    __shared__ __attribute__((aligned(16))) float red[4][2][256];
    // prm[p][i][lane]: parameter p (weight, bias, next weight, next bias) at
    // features 256 i + 4 lane .. + 3
    __shared__ __attribute__((aligned(16))) float4 prm[4][4][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nw = gridDim.x * 4;
    {
        const uint16_t* src[4] = {g1, b1, g2, b2};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint2 w = *(const uint2*)(src[p] + 256 * wave + 4 * lane);
            const uint16_t* h = (const uint16_t*)&w;
            prm[p][wave][lane] = float4{h2f(h[0]), h2f(h[1]), h2f(h[2]), h2f(h[3])};
        }
    }
    __syncthreads();
    for (int row = blockIdx.x * 4 + wave; row < padded_rows; row += nw) {
        uint16_t* o1 = out + (size_t)row * 1024;
        if (row >= rows) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *(uint2*)(o1 + 256 * i + 4 * lane) = uint2{0, 0};
                if (kFp8) *(uint32_t*)((uint8_t*)next_out + (size_t)row * 1024 + 256 * i + 4 * lane) = 0u;
                else *(uint2*)((uint16_t*)next_out + (size_t)row * 1024 + 256 * i + 4 * lane) = uint2{0, 0};
            }
            continue;
        }
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint2 w = *(const uint2*)(in + (size_t)row * 1024 + 256 * i + 4 * lane);
            const uint16_t* h = (const uint16_t*)&w;
#pragma unroll
            for (int u = 0; u < 4; ++u) v[4 * i + u] = h2f(h[u]);
        }
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            float part[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) part[u] = ((v[u] + v[4 + u]) + v[8 + u]) + v[12 + u];
            const float mean = ln_partials_sum(part, red[wave][0]) / 1024.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float sq = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float d = v[4 * i + u] - mean;
                    sq += d * d;
                }
                part[u] = sq;
            }
            const float inverse_std = 1.0f / sqrtf(ln_partials_sum(part, red[wave][1]) / 1024.0f + epsilon);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 g4 = prm[2 * pass][i][lane], b4 = prm[2 * pass + 1][i][lane];
                const float g[4] = {g4.x, g4.y, g4.z, g4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
                uint16_t h[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int e = 4 * i + u;
                    h[u] = f2h((v[e] - mean) * inverse_std * g[u] + b[u]);
                    v[e] = h2f(h[u]);
                }
                const uint2 packed{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16)};
                if (pass == 0) {
                    *(uint2*)(o1 + 256 * i + 4 * lane) = packed;
                } else if (kFp8) {
                    const uint32_t q = e4m3x2(v[4 * i] * inverse_scale, v[4 * i + 1] * inverse_scale) |
                                       (e4m3x2(v[4 * i + 2] * inverse_scale, v[4 * i + 3] * inverse_scale) << 16);
                    *(uint32_t*)((uint8_t*)next_out + (size_t)row * 1024 + 256 * i + 4 * lane) = q;
                } else {
                    *(uint2*)((uint16_t*)next_out + (size_t)row * 1024 + 256 * i + 4 * lane) = packed;
                }
            }
        }
    }
}

// Nibble pairs (byte j = q[2j] & 15 | q[2j+1] << 4, encoder.rs:405) -> signed
// int8 codes in k order, 16 bytes in and 32 out per thread: the operand form
// of per-row INT4 weights / activations for the INT8 MFMA.  A nibble n becomes
// n | 0xf0 when its bit 3 is set: t = nibbles & 0x08 per byte, t * 30 = 0xf0.
__device__ __forceinline__ uint32_t s4x4_to_s8(uint32_t nib) {
    const uint32_t t = nib & 0x08080808u;
    return nib | ((t << 5) - (t << 1));
}
__global__ __launch_bounds__(256) void unpack_s4_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, size_t chunks) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks) return;
    const uint4 w = in[i];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // bytes b0..b3 of word j hold k = 8j' + 2b (low) and 2b + 1 (high)
        const uint32_t lo = s4x4_to_s8(ws[j] & 0x0f0f0f0fu), hi = s4x4_to_s8((ws[j] >> 4) & 0x0f0f0f0fu);
        o[2 * j] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);      // lo0 hi0 lo1 hi1
        o[2 * j + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo2 hi2 lo3 hi3
    }
    out[2 * i] = uint4{o[0], o[1], o[2], o[3]};
    out[2 * i + 1] = uint4{o[4], o[5], o[6], o[7]};
}

// Nibble pairs -> the FP6 e3m2 chunk layout of the same codes (16 codes a
// 16-byte chunk: code j at bits 6j.. of the first 12 bytes, 4 zero bytes), 16
// bytes in and 32 out per thread: the operand form for the f8f6f4 MFMA.
__global__ __launch_bounds__(256) void unpack_s4_fp6_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, size_t chunks) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks) return;
    const uint4 w = in[i];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        uint64_t bits[2] = {0, 0};  // 96 bits of 16 codes
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (ws[2 * c + (j >> 3)] >> (8 * ((j >> 1) & 3))) & 0xffu;
            const uint32_t nib = (j & 1) ? byte >> 4 : byte & 15u;
            const uint32_t code = nib >= 8 ? nib - 16u : nib;  // low byte: the int8 code
            const uint64_t f = e3m2_of_code(code);
            const int b = 6 * j;
            if (b < 64) {
                bits[0] |= f << b;
                if (b > 58) bits[1] |= f >> (64 - b);  // a field across the 64-bit boundary
            } else {
                bits[1] |= f << (b - 64);
            }
        }
        out[2 * i + c] = uint4{(uint32_t)bits[0], (uint32_t)(bits[0] >> 32), (uint32_t)bits[1], 0u};
    }
}

// INT4-g128 weights (pk_pack_int4_g128 layout) -> e4m3 (q - z) bytes [n x k]
// in k order (|q - z| <= 15 is exact in e4m3), the weight operand of the
// G128F8 GEMM: one thread per 4 words (32 K values of one group).
// HBM-bound: reads k/2 + 2 k/128 bytes and writes k bytes per row.
__global__ __launch_bounds__(256) void expand_g128_e4m3_kernel(const uint4* __restrict__ q, const uint16_t* __restrict__ zeros,
                                                               const uint16_t* __restrict__ scales, uint16_t* __restrict__ scales_t,
                                                               uint4* __restrict__ out, int n, int k, size_t quads) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= quads) return;
    const size_t per_row = (size_t)k / 32;  // quads per row
    const size_t row = i / per_row;
    const int quad = (int)(i - row * per_row), group = quad >> 2;
    const float z = h2f(zeros[row * (size_t)(k >> 7) + group]);
    // the group's first quad also moves its scale to the group-major table
    if ((quad & 3) == 0) scales_t[(size_t)group * n + row] = scales[row * (size_t)(k >> 7) + group];
    const uint4 w = q[i];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // word j: byte b holds k 8j + b (low nibble) and 8j + 4 + b (high)
        float v[8];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            v[b] = (float)((ws[j] >> (8 * b)) & 15u) - z;
            v[4 + b] = (float)((ws[j] >> (8 * b + 4)) & 15u) - z;
        }
        o[2 * j] = e4m3x2(v[0], v[1]) | (e4m3x2(v[2], v[3]) << 16);
        o[2 * j + 1] = e4m3x2(v[4], v[5]) | (e4m3x2(v[6], v[7]) << 16);
    }
    out[2 * i] = uint4{o[0], o[1], o[2], o[3]};
    out[2 * i + 1] = uint4{o[4], o[5], o[6], o[7]};
}

// ---- launchers -------------------------------------------------------------

// Q4_K superblocks -> fp16 [n x k] (linear.cu:459-472): one thread per 8
// consecutive values of one 32-value group.
__global__ __launch_bounds__(256) void q4k_dequant_kernel(const uint8_t* __restrict__ blocks, uint16_t* __restrict__ out, int n,
                                                          int k) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t per_row = (size_t)k / 8;
    if (idx >= (size_t)n * per_row) return;
    const size_t row = idx / per_row;
    const int t = (int)(idx - row * per_row) * 8;
    const uint8_t* blk = blocks + (row * (size_t)(k / 256) + (size_t)(t >> 8)) * 144;
    const int v = t & 255, group = v >> 5;
    const uint4 h = *(const uint4*)blk;
    const uint2 q = *(const uint2*)(blk + 16 + (group >> 1) * 32 + (v & 31));
    float a, b;
    q4k_coeffs(h, group, a, b);
    const int sh = (group & 1) * 4;
    *(uint4*)(out + row * (size_t)k + t) = q4k_decode8((q.x >> sh) & 0x0f0f0f0fu, (q.y >> sh) & 0x0f0f0f0fu, a, b);
}

int launch_quantize_static(const void* in, void* out, float inverse_scale, size_t elements, bool int8, hipStream_t s) {
    if (elements == 0) return 0;
    const size_t threads = (elements + 7) / 8;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (int8) quantize_int8_static_kernel<<<grid, 256, 0, s>>>((const uint16_t*)in, (int8_t*)out, inverse_scale, elements);
    else quantize_fp8_static_kernel<<<grid, 256, 0, s>>>((const uint16_t*)in, (uint8_t*)out, inverse_scale, elements);
    return 0;
}

static unsigned row_grid(int rows) {
    // four rows per block, at most eight blocks per CU (rows are strided)
    const int blocks = (rows + 3) / 4, cap = 8 * cu_count();
    return (unsigned)(blocks < cap ? blocks : cap);
}

int launch_quantize_rows(int kind, const void* in, void* out, float* scales, int rows, int valid_rows, int k, hipStream_t s) {
    if (rows == 0) return 0;
    const unsigned grid = row_grid(rows);
    const uint16_t* x = (const uint16_t*)in;
    uint8_t* o = (uint8_t*)out;
    // rows of up to 1024 (kCh 2) or 4096 (kCh 8) elements stay in registers
    if (k <= 1024) {
        if (kind == 0) quantize_rows_kernel<0, 2, true><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
        else if (kind == 1) quantize_rows_kernel<1, 2, true><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
        else quantize_rows_kernel<2, 2, true><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
    } else {
        if (kind == 0) quantize_rows_kernel<0, 8, false><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
        else if (kind == 1) quantize_rows_kernel<1, 8, false><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
        else quantize_rows_kernel<2, 8, false><<<grid, 256, 0, s>>>(x, o, scales, rows, k, valid_rows);
    }
    return 0;
}

int launch_quantize_rows_sp24(const void* in, uint8_t* data, uint8_t* meta, float* scales, uint32_t* ovf_count, uint32_t* ovf,
                              uint8_t* data2, uint8_t* meta2, int rows, int valid_rows, int k, hipStream_t s) {
    if (rows == 0) return 0;
    const unsigned grid = row_grid(rows);
    const uint16_t* x = (const uint16_t*)in;
    if (k <= 1024) quantize_rows_sp24_kernel<2><<<grid, 256, 0, s>>>(x, data, meta, scales, ovf_count, ovf, data2, meta2, rows, k, valid_rows);
    else quantize_rows_sp24_kernel<8><<<grid, 256, 0, s>>>(x, data, meta, scales, ovf_count, ovf, data2, meta2, rows, k, valid_rows);
    return 0;
}

int launch_pack_rows(int kind, const void* w, void* out, float* scales, int n, int k, hipStream_t s) {
    if (n == 0) return 0;
    if (kind == 0) pack_rows_kernel<0><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    else if (kind == 1) pack_rows_kernel<1><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    else pack_rows_kernel<2><<<n, 256, 0, s>>>((const uint16_t*)w, (uint8_t*)out, scales, k);
    return 0;
}

int launch_pack_g128(const void* w, uint32_t* q, uint16_t* scales, uint16_t* zeros, int n, int k, hipStream_t s) {
    const int total = n * (k / 128);
    if (total == 0) return 0;
    pack_g128_kernel<<<(total + 255) / 256, 256, 0, s>>>((const uint16_t*)w, q, scales, zeros, n, k);
    return 0;
}

int launch_layer_norm_quantize(int mode, const void* in, const void* gamma, const void* beta, void* out, float* scales,
                               void* normalized, int rows, int padded_rows, float epsilon, hipStream_t s) {
    if (padded_rows == 0) return 0;
    const unsigned grid = row_grid(padded_rows);
    if (mode == 3)
        layer_norm_quantize_kernel<true, true, true><<<grid, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                                          (uint8_t*)out, scales, (uint16_t*)normalized, rows, padded_rows, epsilon);
    else if (mode == 2)
        layer_norm_quantize_kernel<true, true><<<grid, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                                    (uint8_t*)out, scales, (uint16_t*)normalized, rows, padded_rows, epsilon);
    else if (mode == 1)
        layer_norm_quantize_kernel<true><<<grid, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                               (uint8_t*)out, scales, (uint16_t*)normalized, rows, padded_rows, epsilon);
    else
        layer_norm_quantize_kernel<false><<<grid, 256, 0, s>>>((const uint16_t*)in, (const uint16_t*)gamma, (const uint16_t*)beta,
                                                                (uint8_t*)out, scales, (uint16_t*)normalized, rows, padded_rows, epsilon);
    return 0;
}

int launch_layer_norm_pair(const void* in, const void* g1, const void* b1, void* out, const void* g2, const void* b2, void* next_out,
                           int rows, int padded_rows, float epsilon, float inverse_scale, hipStream_t s) {
    if (padded_rows == 0) return 0;
    const unsigned grid = row_grid(padded_rows);
    const uint16_t *x = (const uint16_t*)in, *w1 = (const uint16_t*)g1, *c1 = (const uint16_t*)b1, *w2 = (const uint16_t*)g2,
                   *c2 = (const uint16_t*)b2;
    if (inverse_scale != 0.0f)
        layer_norm_pair_kernel<true><<<grid, 256, 0, s>>>(x, w1, c1, (uint16_t*)out, w2, c2, next_out, rows, padded_rows, epsilon,
                                                           inverse_scale);
    else
        layer_norm_pair_kernel<false><<<grid, 256, 0, s>>>(x, w1, c1, (uint16_t*)out, w2, c2, next_out, rows, padded_rows, epsilon,
                                                            inverse_scale);
    return 0;
}

int launch_unpack_s4(const uint8_t* in, int8_t* out, size_t bytes, hipStream_t s) {
    const size_t chunks = bytes / 16;
    if (chunks == 0) return 0;
    unpack_s4_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, s>>>((const uint4*)in, (uint4*)out, chunks);
    return 0;
}

int launch_unpack_s4_fp6(const uint8_t* in, uint8_t* out, size_t bytes, hipStream_t s) {
    const size_t chunks = bytes / 16;
    if (chunks == 0) return 0;
    unpack_s4_fp6_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, s>>>((const uint4*)in, (uint4*)out, chunks);
    return 0;
}

int launch_expand_g128_e4m3(const uint32_t* q, const uint16_t* zeros, const uint16_t* scales, uint16_t* scales_t, uint8_t* out,
                            int n, int k, hipStream_t s) {
    const size_t quads = (size_t)n * (k / 32);
    if (quads == 0) return 0;
    expand_g128_e4m3_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>((const uint4*)q, zeros, scales, scales_t, (uint4*)out, n,
                                                                              k, quads);
    return 0;
}

int launch_q4k_dequant(const uint8_t* blocks, uint16_t* out, int n, int k, hipStream_t s) {
    const size_t threads = (size_t)n * (k / 8);
    if (threads == 0) return 0;
    hipLaunchKernelGGL(q4k_dequant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, blocks, out, n, k);
    return 0;
}

}  // namespace pk
