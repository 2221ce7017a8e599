// Byte-tile GEMM engine for the quantized linears (gfx950 / CDNA4).
//
// One workgroup = 8 wave64s computing a 256x256 output tile; wave w owns
// rows 128*(w/4) .. +128 and columns 64*(w%4) .. +64 as 8x4 MFMA 16x16
// tiles.  Every K-step moves 128 bytes of each A row (256 rows) and up to 128
// bytes of each B row (256 rows) global -> registers -> LDS (double
// buffered, one barrier per step); the 16-byte chunks of each 128-byte LDS row
// are XOR-swizzled by (row & 7) so the 16 lanes that read one chunk column hit
// distinct banks.  The operand format only changes how a lane's two 16-byte
// chunks (K slots [16g, 16g+16) and [64+16g, 64+16g+16) of the step, g =
// lane/16) are decoded and which MFMA consumes them:
//   FP8     e4m3 x e4m3   v_mfma_f32_16x16x128_f8f6f4      K/step 128
//   I8      s8 x s8       2 x v_mfma_i32_16x16x64_i8       K/step 128 (exact)
//   S4      s4 x s4       nibbles -> s8, 4 x i8 MFMA       K/step 256 (exact)
//   G128A8  s8 x (q-z)    group-wise INT4 weights, i8 MFMA per 128-K group,
//                         fp32 fma of each group sum with its fp16 scale
//   F16     f16 x f16     2 x v_mfma_f32_16x16x32_f16      K/step 64
//   G128A16 f16 x f16((q-z)*s)  INT4 weights dequantized in registers
// The epilogue stages each wave's accumulators through LDS (16 rows at a
// time) so every lane finishes 16 consecutive columns of one row with 16- or
// 32-byte global stores.
#pragma once

#include "pk_common.hpp"

namespace pk {

enum Fmt { FMT_FP8 = 0, FMT_I8 = 1, FMT_S4 = 2, FMT_G128A8 = 3, FMT_F16 = 4, FMT_G128A16 = 5 };

enum Epi {
    EPI_F16 = 0,     // fp16 out: act(scale(acc) [+bias]) * out_scale [+ res_scale * residual]
    EPI_F8 = 1,      // e4m3 out: e4m3(fp16(silu(scale(acc))) * 16)
    EPI_F8_24 = 2,   // as EPI_F8, then 2:4 compressed data + 4-bit metadata
    EPI_F32 = 3,     // fp32 out: scale(acc) [+bias]
    EPI_I32 = 4,     // raw int32 accumulators (integer formats only)
    EPI_GLU = 5,     // fp16 out: fp16(v) * sigmoid(fp16(g)), column pairs (c, c + N/2)
};

struct GemmArgs {
    const uint8_t* a;           // [M x K] activations, row-major
    const uint8_t* b;           // [N x K] weights (weight_oi), row-major, format-specific bytes
    int m, n, k;                // logical sizes, k in elements
    const float* w_scales;      // [N] per output channel, or null (1.0)
    const float* row_scales;    // [M] per-row activation scales, or null (in_scale)
    float in_scale;
    int fused_scale;            // 1: v = fma(acc, in_scale * w_scale, bias) (linear.cu:362-365)
                                // 0: v = acc * row_scale * w_scale [+ bias] (encoder.cu:975-995)
    const float* bias;          // [N] or null
    const uint16_t* residual;   // fp16 [M x ldo] or null (may alias out)
    float out_scale;
    float res_scale;
    int act;                    // 0 none, 1 SiLU, 2 ReLU
    const uint16_t* g_scales;   // G128 formats: fp16 [N x K/128]
    const uint16_t* g_zeros;    // G128 formats: fp16 [N x K/128], integer valued
    void* out;
    uint8_t* out_meta;          // EPI_F8_24: [M x ldo/8] metadata bytes
    int ldo;                    // output row stride in elements (of the output type)
    int valid_rows;             // EPI_GLU: rows >= valid_rows are written as 0
};

constexpr int kBlockM = 256;
constexpr int kBlockN = 256;
constexpr int kThreads = 512;
constexpr int kRowBytes = 128;
constexpr int kTileBytes = kBlockM * kRowBytes;  // one operand tile per stage
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kMaxG128Groups = 32;  // K <= 4096 for the group-wise INT4 formats

template <int F> struct FmtTraits;
template <> struct FmtTraits<FMT_FP8> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_I8> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = true; };
template <> struct FmtTraits<FMT_S4> { static constexpr int kStep = 256, bRow = 128, aElemNum = 1, aElemDen = 2, bNum = 1, bDen = 2; static constexpr bool kInt = true; };
template <> struct FmtTraits<FMT_G128A8> { static constexpr int kStep = 128, bRow = 64, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 2; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_F16> { static constexpr int kStep = 64, bRow = 128, aElemNum = 2, aElemDen = 1, bNum = 2, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_G128A16> { static constexpr int kStep = 64, bRow = 32, aElemNum = 2, aElemDen = 1, bNum = 1, bDen = 2; static constexpr bool kInt = false; };

__device__ __forceinline__ int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ (row & 7)) << 4); }

// Four unsigned nibbles (byte j of `w`, low nibble = k j, high = k 4+j) ->
// eight int8 (q - z), natural k order, as two dwords.
__device__ __forceinline__ void u4x8_minus_z(uint32_t w, uint32_t zz, uint32_t& first, uint32_t& second) {
    uint32_t l = w & 0x0f0f0f0fu, h = (w >> 4) & 0x0f0f0f0fu;
    first = ((l | 0x80808080u) - zz) ^ 0x80808080u;
    second = ((h | 0x80808080u) - zz) ^ 0x80808080u;
}

// Eight unsigned nibbles of one word -> eight halves f16((q - z) * s), k order.
__device__ __forceinline__ v8h u4x8_to_h(uint32_t w, v2h zz, v2h ss) {
    uint32_t l = w & 0x0f0f0f0fu, h = (w >> 4) & 0x0f0f0f0fu;
    uint32_t p0 = __builtin_amdgcn_perm(0u, l, 0x0c010c00u) | 0x64006400u;
    uint32_t p1 = __builtin_amdgcn_perm(0u, l, 0x0c030c02u) | 0x64006400u;
    uint32_t p2 = __builtin_amdgcn_perm(0u, h, 0x0c010c00u) | 0x64006400u;
    uint32_t p3 = __builtin_amdgcn_perm(0u, h, 0x0c030c02u) | 0x64006400u;
    v2h r0 = (__builtin_bit_cast(v2h, p0) - zz) * ss;
    v2h r1 = (__builtin_bit_cast(v2h, p1) - zz) * ss;
    v2h r2 = (__builtin_bit_cast(v2h, p2) - zz) * ss;
    v2h r3 = (__builtin_bit_cast(v2h, p3) - zz) * ss;
    v8h out = {r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    return out;
}

template <int F>
__device__ __forceinline__ void mfma_step(v4f& accf, v4i& acci, const uint4& a0, const uint4& a1,
                                          const uint4& b0, const uint4& b1, float gscale) {
    if constexpr (F == FMT_FP8) {
        v8i A = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        v8i B = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        accf = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, accf, 0, 0, 0, 0, 0, 0);
    } else if constexpr (F == FMT_I8) {
        v4i A0 = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w};
        v4i A1 = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        v4i B0 = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w};
        v4i B1 = {(int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, acci, 0, 0, 0);
    } else if constexpr (F == FMT_S4) {
        uint32_t al[8], bl[8];
        s4x8_to_s8(a0.x, al[0], al[4]); s4x8_to_s8(a0.y, al[1], al[5]);
        s4x8_to_s8(a0.z, al[2], al[6]); s4x8_to_s8(a0.w, al[3], al[7]);
        s4x8_to_s8(b0.x, bl[0], bl[4]); s4x8_to_s8(b0.y, bl[1], bl[5]);
        s4x8_to_s8(b0.z, bl[2], bl[6]); s4x8_to_s8(b0.w, bl[3], bl[7]);
        v4i A0 = {(int)al[0], (int)al[1], (int)al[2], (int)al[3]}, A1 = {(int)al[4], (int)al[5], (int)al[6], (int)al[7]};
        v4i B0 = {(int)bl[0], (int)bl[1], (int)bl[2], (int)bl[3]}, B1 = {(int)bl[4], (int)bl[5], (int)bl[6], (int)bl[7]};
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, acci, 0, 0, 0);
        s4x8_to_s8(a1.x, al[0], al[4]); s4x8_to_s8(a1.y, al[1], al[5]);
        s4x8_to_s8(a1.z, al[2], al[6]); s4x8_to_s8(a1.w, al[3], al[7]);
        s4x8_to_s8(b1.x, bl[0], bl[4]); s4x8_to_s8(b1.y, bl[1], bl[5]);
        s4x8_to_s8(b1.z, bl[2], bl[6]); s4x8_to_s8(b1.w, bl[3], bl[7]);
        v4i A2 = {(int)al[0], (int)al[1], (int)al[2], (int)al[3]}, A3 = {(int)al[4], (int)al[5], (int)al[6], (int)al[7]};
        v4i B2 = {(int)bl[0], (int)bl[1], (int)bl[2], (int)bl[3]}, B3 = {(int)bl[4], (int)bl[5], (int)bl[6], (int)bl[7]};
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, B2, acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, B3, acci, 0, 0, 0);
    } else if constexpr (F == FMT_G128A8) {
        // b0/b1 already hold (q - z) as int8 (decoded once per step).
        v4i A0 = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w};
        v4i A1 = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        v4i B0 = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w};
        v4i B1 = {(int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        v4i zero = {0, 0, 0, 0};
        v4i g = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, zero, 0, 0, 0);
        g = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, g, 0, 0, 0);
        accf[0] = __builtin_fmaf((float)g[0], gscale, accf[0]);
        accf[1] = __builtin_fmaf((float)g[1], gscale, accf[1]);
        accf[2] = __builtin_fmaf((float)g[2], gscale, accf[2]);
        accf[3] = __builtin_fmaf((float)g[3], gscale, accf[3]);
    } else {  // F16 and G128A16 (B already dequantized to halves)
        v8h A0 = __builtin_bit_cast(v8h, a0), A1 = __builtin_bit_cast(v8h, a1);
        v8h B0 = __builtin_bit_cast(v8h, b0), B1 = __builtin_bit_cast(v8h, b1);
        accf = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B0, accf, 0, 0, 0);
        accf = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B1, accf, 0, 0, 0);
    }
}

// 16 bytes global -> LDS per lane (global_load_lds_dwordx4): lane l writes
// LDS bytes [lds_addr + 16 l, + 16).  lds_addr must be wave-uniform.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory", "m0");
}

// Orders this wave's LDS writes before its later LDS reads (and the reads
// before the next writes) when lanes exchange data through LDS.
// A wave's LDS instructions execute in order, so only the compiler must be
// kept from reordering them (no global-memory fence, which would also wait
// for the wave's outstanding global stores).
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// Epilogue: each wave stages 8 rows x 64 columns of fp32 accumulators per
// pass through its own LDS slab so that lane l finishes columns
// [8(l%8), 8(l%8)+8) of row l/8 with one contiguous store.  Column scales and
// bias and the 16 row scales of the lane are loaded once per tile.
template <int F, int E>
__device__ __forceinline__ void epilogue(const GemmArgs& p, v4f (&accf)[8][4], v4i (&acci)[8][4], float* stage, int m0,
                                         int n0, int wm, int wn, int lane) {
    using T = FmtTraits<F>;
    const int g = lane >> 4, l16 = lane & 15;
    const int er = lane >> 3, ec = (lane & 7) * 8;
    const int gcol = n0 + wn * 64 + ec;
    const int ccol = min(gcol, p.n - 8);
    float wsv[8], bsv[8], rsv[16];
#pragma unroll
    for (int j = 0; j < 8; j += 4) {
        const float4 w4 = p.w_scales ? *(const float4*)(p.w_scales + ccol + j) : float4{1.f, 1.f, 1.f, 1.f};
        const float4 b4 = p.bias ? *(const float4*)(p.bias + ccol + j) : float4{0.f, 0.f, 0.f, 0.f};
        wsv[j] = w4.x; wsv[j + 1] = w4.y; wsv[j + 2] = w4.z; wsv[j + 3] = w4.w;
        bsv[j] = b4.x; bsv[j + 1] = b4.y; bsv[j + 2] = b4.z; bsv[j + 3] = b4.w;
    }
#pragma unroll
    for (int ps = 0; ps < 16; ++ps) {
        const int row = min(m0 + wm * 128 + ps * 8 + er, p.m - 1);
        rsv[ps] = p.row_scales ? p.row_scales[row] : p.in_scale;
    }
#pragma unroll
    for (int ps = 0; ps < 16; ++ps) {
        const int ai = ps >> 1, h = ps & 1;
        if ((g >> 1) == h) {
#pragma unroll
            for (int bj = 0; bj < 4; ++bj)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v;
                    if constexpr (T::kInt) {
                        const int iv = acci[ai][bj][r];
                        v = E == EPI_I32 ? __int_as_float(iv) : (float)iv;
                    } else {
                        v = accf[ai][bj][r];
                    }
                    stage[(4 * (g & 1) + r) * 68 + bj * 16 + l16] = v;
                }
        }
        wave_lds_sync();
        float v[8];
        {
            const float4 q0 = *(const float4*)(stage + er * 68 + ec);
            const float4 q1 = *(const float4*)(stage + er * 68 + ec + 4);
            v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
            v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
        }
        wave_lds_sync();
        const int grow = m0 + wm * 128 + ps * 8 + er;
        if (grow >= p.m || gcol >= p.n) continue;

        if constexpr (E == EPI_I32) {
            int32_t* o = (int32_t*)p.out + (size_t)grow * p.ldo + gcol;
            *(int4*)o = __builtin_bit_cast(int4, float4{v[0], v[1], v[2], v[3]});
            *(int4*)(o + 4) = __builtin_bit_cast(int4, float4{v[4], v[5], v[6], v[7]});
            continue;
        }
        const float rs = rsv[ps];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float fused = __builtin_fmaf(v[j], rs * wsv[j], bsv[j]);
            const float plain = v[j] * rs * wsv[j] + bsv[j];
            v[j] = p.fused_scale ? fused : plain;
        }
        if constexpr (E == EPI_F32) {
            float* o = (float*)p.out + (size_t)grow * p.ldo + gcol;
            *(float4*)o = float4{v[0], v[1], v[2], v[3]};
            *(float4*)(o + 4) = float4{v[4], v[5], v[6], v[7]};
        } else if constexpr (E == EPI_F16) {
            uint4 res = {0, 0, 0, 0};
            if (p.residual) res = *(const uint4*)(p.residual + (size_t)grow * p.ldo + gcol);
            const uint32_t rw[4] = {res.x, res.y, res.z, res.w};
            const float rsc = p.residual ? p.res_scale : 0.0f;
            uint32_t h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float x0 = __builtin_fmaf(rsc, h2f((uint16_t)(rw[j] & 0xffff)), v[2 * j] * p.out_scale);
                float x1 = __builtin_fmaf(rsc, h2f((uint16_t)(rw[j] >> 16)), v[2 * j + 1] * p.out_scale);
                x0 = p.act == 1 ? silu(x0) : (p.act == 2 ? __builtin_fmaxf(x0, 0.0f) : x0);
                x1 = p.act == 1 ? silu(x1) : (p.act == 2 ? __builtin_fmaxf(x1, 0.0f) : x1);
                h[j] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
            }
            *(uint4*)((uint16_t*)p.out + (size_t)grow * p.ldo + gcol) = uint4{h[0], h[1], h[2], h[3]};
        } else if constexpr (E == EPI_F8 || E == EPI_F8_24) {
            uint32_t w[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float x0 = round_f16(silu(v[4 * j])) * 16.0f, x1 = round_f16(silu(v[4 * j + 1])) * 16.0f;
                const float x2 = round_f16(silu(v[4 * j + 2])) * 16.0f, x3 = round_f16(silu(v[4 * j + 3])) * 16.0f;
                w[j] = e4m3x2(x0, x1) | (e4m3x2(x2, x3) << 16);
            }
            if constexpr (E == EPI_F8) {
                *(uint2*)((uint8_t*)p.out + (size_t)grow * p.ldo + gcol) = uint2{w[0], w[1]};
            } else {
                // encoder.cu:685-704: keep the two largest |e4m3| of each
                // quartet (ties to the lower index), metadata idx0 | idx1 << 2.
                uint32_t data = 0, meta = 0;
#pragma unroll
                for (int qd = 0; qd < 2; ++qd) {
                    const uint32_t packed = w[qd];
                    uint32_t d = 0, md = 0;
                    int count = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t mi = (packed >> (8 * i)) & 127;
                        int rank = 0;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t mj = (packed >> (8 * j)) & 127;
                            rank += (mj > mi) || (mj == mi && j < i);
                        }
                        if (rank < 2) {
                            d |= ((packed >> (8 * i)) & 255u) << (8 * count);
                            md |= (uint32_t)i << (2 * count);
                            ++count;
                        }
                    }
                    data |= d << (16 * qd);
                    meta |= md << (4 * qd);
                }
                *(uint32_t*)((uint8_t*)p.out + (size_t)grow * (p.ldo / 2) + gcol / 2) = data;
                p.out_meta[(size_t)grow * (p.ldo / 8) + gcol / 8] = (uint8_t)meta;
            }
        }
    }
}

// Persistent tile schedule.  The grid is one workgroup per CU (G of them);
// iteration i of workgroup b computes logical tile i*G + slot(b).  Workgroups
// are dispatched round-robin over the 8 XCDs, so slot() gives each XCD a
// contiguous run of G/8 logical tiles per iteration; tiles are numbered N
// fastest, so an XCD's concurrent tiles share one or two A row-strips and the
// same B columns in its L2.
__device__ __forceinline__ int tile_slot(int G) {
    const int b = blockIdx.x;
    return (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
}

template <int F> struct Layout {
    static constexpr int kStage = kTileBytes + kBlockN * FmtTraits<F>::bRow;
    static constexpr int kEpi = 2 * kStage;                      // epilogue staging
    static constexpr int kEpiBytes = 8 * 8 * 68 * 4;              // 8 waves x 8 rows x 68 floats
    static constexpr bool kG128 = (F == FMT_G128A8 || F == FMT_G128A16);
    static constexpr int kGsz = kEpi + kEpiBytes;                  // g128 (scale, zero) table
    static constexpr int kBytes = kGsz + (kG128 ? kMaxG128Groups * kBlockN * 4 : 0);
};

template <int F, int E>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs p) {
    using T = FmtTraits<F>;
    using L = Layout<F>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBlockN - 1) / kBlockN;
    const int ntiles = ((p.m + kBlockM - 1) / kBlockM) * tiles_n;
    const int G = gridDim.x;
    const int slot = tile_slot(G);
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;  // bytes per A row
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;          // bytes per B row
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    const uint8_t* __restrict__ pa = p.a;
    const uint8_t* __restrict__ pb = p.b;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    uint32_t* gsz = (uint32_t*)(lds + L::kGsz);

    // Direct-to-LDS operand loads (global_load_lds_dwordx4): one wave
    // instruction fills 1 KiB of LDS, lane l writing bytes [16l, 16l+16), so
    // each lane loads the global chunk the swizzled layout puts there.
    constexpr int kBLoadsPerWave = (kBlockN * T::bRow) / 1024 / 8;
    uint32_t a_off[4], b_off[kBLoadsPerWave];
    auto set_tile = [&](int t, int& m0, int& n0) {
        const int tm = t / tiles_n;
        m0 = tm * kBlockM;
        n0 = (t - tm * tiles_n) * kBlockN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (wave * 4 + i) * 1024 + lane * 16;
            const int row = o >> 7, c = ((o >> 4) & 7) ^ (row & 7);
            a_off[i] = (uint32_t)((size_t)min(m0 + row, p.m - 1) * lda + c * 16);
        }
#pragma unroll
        for (int i = 0; i < kBLoadsPerWave; ++i) {
            const int o = (wave * kBLoadsPerWave + i) * 1024 + lane * 16;
            int row, c;
            if constexpr (T::bRow == 128) {
                row = o >> 7;
                c = ((o >> 4) & 7) ^ (row & 7);
            } else {
                row = o / T::bRow;
                c = (o % T::bRow) / 16;
            }
            b_off[i] = (uint32_t)((size_t)min(n0 + row, p.n - 1) * ldb + c * 16);
        }
    };
    // The loads are issued from inline asm so that the compiler does not order
    // every later LDS read behind them (it cannot tell the DMA target from the
    // buffer being read); the step loop waits for them explicitly.
    auto issue = [&](int step, int buf) {
        const uint32_t base = lds_base + buf * L::kStage;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(pa + a_off[i] + (size_t)step * kRowBytes, base + (wave * 4 + i) * 1024);
#pragma unroll
        for (int i = 0; i < kBLoadsPerWave; ++i)
            dma16(pb + b_off[i] + (size_t)step * T::bRow, base + kTileBytes + (wave * kBLoadsPerWave + i) * 1024);
    };

    int t = slot;
    if (t >= ntiles) return;
    int m0, n0;
    set_tile(t, m0, n0);
    issue(0, 0);
    int buf = 0;

    v4f accf[8][4];
    v4i acci[8][4];
    float* stage = (float*)(lds + L::kEpi + wave * (8 * 68 * 4));

    while (true) {
        const int t_next = t + G;
        const int cur_m0 = m0, cur_n0 = n0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                accf[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
                acci[i][j] = v4i{0, 0, 0, 0};
            }

        for (int step = 0; step < steps; ++step) {
            // This wave's loads for `step` have landed in LDS; the barrier makes
            // every wave's loads visible and retires all reads of the other
            // buffer before it is refilled.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if constexpr (L::kG128) {
                if (step == 0) {
                    for (int idx = tid; idx < kBlockN * groups; idx += kThreads) {
                        const int col = idx / groups, grp = idx - col * groups;
                        const size_t gi = (size_t)min(cur_n0 + col, p.n - 1) * groups + grp;
                        gsz[idx] = (uint32_t)p.g_scales[gi] | ((uint32_t)p.g_zeros[gi] << 16);
                    }
                    __syncthreads();
                }
            }
            if (step + 1 < steps) {
                issue(step + 1, buf ^ 1);
            } else if (t_next < ntiles) {
                set_tile(t_next, m0, n0);
                issue(0, buf ^ 1);
            }
            const uint8_t* As = lds + buf * L::kStage;
            const uint8_t* Bs = As + kTileBytes;
            const int n0 = cur_n0;
            (void)n0;

            // Decode this wave's four B fragments.
            uint4 b0[4], b1[4];
            float gs[4] = {1.f, 1.f, 1.f, 1.f};
    #pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int row = wn * 64 + bj * 16 + l16;
                if constexpr (T::bRow == 128) {
                    b0[bj] = *(const uint4*)(Bs + swz(row, g));
                    b1[bj] = *(const uint4*)(Bs + swz(row, 4 + g));
                } else {
                    const int kg = (step * T::kStep) >> 7;
                    const uint32_t sz = gsz[row * groups + kg];
                    const float z = h2f((uint16_t)(sz >> 16));
                    if constexpr (F == FMT_G128A8) {
                        gs[bj] = h2f((uint16_t)(sz & 0xffff));
                        const uint32_t zz = (uint32_t)(int)z * 0x01010101u;
                        const uint2 w0 = *(const uint2*)(Bs + row * 64 + 8 * g);
                        const uint2 w1 = *(const uint2*)(Bs + row * 64 + 32 + 8 * g);
                        u4x8_minus_z(w0.x, zz, b0[bj].x, b0[bj].y);
                        u4x8_minus_z(w0.y, zz, b0[bj].z, b0[bj].w);
                        u4x8_minus_z(w1.x, zz, b1[bj].x, b1[bj].y);
                        u4x8_minus_z(w1.y, zz, b1[bj].z, b1[bj].w);
                    } else {  // G128A16
                        const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(sz & 0xffff));
                        const _Float16 zh = (_Float16)(1024.0f + z);
                        const v2h ss = {s, s}, zz = {zh, zh};
                        const uint32_t w0 = *(const uint32_t*)(Bs + row * 32 + 4 * g);
                        const uint32_t w1 = *(const uint32_t*)(Bs + row * 32 + 16 + 4 * g);
                        b0[bj] = __builtin_bit_cast(uint4, u4x8_to_h(w0, zz, ss));
                        b1[bj] = __builtin_bit_cast(uint4, u4x8_to_h(w1, zz, ss));
                    }
                }
            }
#pragma unroll
            for (int ai = 0; ai < 8; ++ai) {
                const int row = wm * 128 + ai * 16 + l16;
                const uint4 a0 = *(const uint4*)(As + swz(row, g));
                const uint4 a1 = *(const uint4*)(As + swz(row, 4 + g));
#pragma unroll
                for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[ai][bj], acci[ai][bj], a0, a1, b0[bj], b1[bj], gs[bj]);
            }
            buf ^= 1;
        }

        epilogue<F, E>(p, accf, acci, stage, cur_m0, cur_n0, wm, wn, lane);
        if (t_next >= ntiles) break;
        t = t_next;
    }
}

}  // namespace pk
