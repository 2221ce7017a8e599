// Byte-tile GEMM engine for the quantized linears (gfx950 / CDNA4).
//
// A persistent workgroup per CU (8 wave64s) walks 256x256 output tiles; wave
// w owns output rows 128*(w/4) .. +128 and columns 64*(w%4) .. +64.  Every
// K-step moves 128 bytes of each of the tile's 256 activation rows and up to
// 128 bytes of each of its 256 weight rows global -> LDS with direct-to-LDS
// loads (double buffered, one barrier per step, the next tile's first step
// prefetched while the current tile finishes).  The 16-byte chunks of each
// 128-byte LDS row are XOR-swizzled (swz_key) so that the 16 lanes reading one
// chunk column hit distinct banks.
//
// The weights are the MFMA's first operand and the activations its second,
// so accumulator register r of lane l holds output column 4*(l/16)+r of row
// l%16.  Weight rows are assigned to the four 16-row MFMA blocks of a wave
// (bj) as n = 16*(i/4) + 4*bj + i%4 (i = MFMA row), which makes the 16
// accumulators a lane holds for one 16-row block of activations exactly the
// 16 consecutive output columns [16*(l/16), +16) of one row: the epilogue
// scales, converts and stores them straight from registers.
//
// The operand format only changes how a lane's two 16-byte chunks (K slots
// [16g, 16g+16) and [64+16g, 64+16g+16) of the step, g = lane/16) are decoded
// and which MFMA consumes them:
//   FP8     e4m3 x e4m3   v_mfma_f32_16x16x128_f8f6f4      K/step 128
//   I8      s8 x s8       2 x v_mfma_i32_16x16x64_i8       K/step 128 (exact)
//   S4      s4 x s4       nibbles -> s8, 4 x i8 MFMA       K/step 256 (exact)
//   G128A8  (q-z) x s8    group-wise INT4 weights, i8 MFMA per 128-K group,
//                         fp32 fma of each group sum with its fp16 scale
//   F16     f16 x f16     2 x v_mfma_f32_16x16x32_f16      K/step 64
//   G128A16 f16((q-z)*s) x f16, INT4 weights dequantized in registers
//   Q4K     f16(d*sc*q - dmin*mn) x f16, GGUF Q4_K superblocks (144 bytes
//           per 256 K) dequantized in registers, K/step 64 = one group pair
//   G128F8  e4m3 activations x group-wise INT4 weights given as e4m3 (q - z)
//           bytes (exact: |q - z| <= 15), one f8f6f4 MFMA per 128-K group
//           (fp32 group sum), fp32 fma of each group sum with its fp16 scale
#pragma once

#include "pk_common.hpp"

namespace pk {

// FMT_S4F6: INT4 codes as FP6 e3m2 (exact for -8..8), 16 codes a 16-byte
// chunk (12 bytes of 6-bit fields, code j at bits 6j.., then 4 zero bytes):
// rows have the int8 codes' size and layout of 16-byte chunks, so the engine
// moves them as FP8 bytes; the f8f6f4 MFMA multiplies them at the FP6 rate
// and its fp32 sums of at most 2^24 are the exact int32 accumulators.
enum Fmt { FMT_FP8 = 0, FMT_I8 = 1, FMT_S4 = 2, FMT_G128A8 = 3, FMT_F16 = 4, FMT_G128A16 = 5, FMT_I8_SKIP = 6, FMT_Q4K = 7, FMT_G128F8 = 8,
           FMT_S4F6 = 9 };

enum Epi {
    EPI_F16 = 0,     // fp16 out: act(scale(acc) [+bias]) * out_scale [+ res_scale * residual]
    EPI_F8 = 1,      // e4m3 out: e4m3(fp16(silu(scale(acc))) * 16)
    EPI_F8_24 = 2,   // as EPI_F8, then 2:4 compressed data + 4-bit metadata
    EPI_F32 = 3,     // fp32 out: scale(acc) [+bias]
    EPI_I32 = 4,     // raw int32 accumulators (integer formats only)
    EPI_F16_RES = 5, // EPI_F16 with a residual (chosen by the launcher when one is given)
    EPI_GLU = 6,     // fp16 out [M x N/2]: fp16(v) / (1 + exp(-fp16(g))), v = column c, g = column c + N/2
    EPI_I8S = 7,     // int8 out: rne(clamp(fp16(silu(scale(acc))) * 16, +-127)) (static INT8 at the x16 hidden scale)
};

struct GemmArgs {
    const uint8_t* a;           // [M x K] activations, row-major
    const uint8_t* b;           // [N x K] weights (weight_oi), row-major, format-specific bytes
    int m, n, k;                // logical sizes, k in elements
    const float* w_scales;      // [N] per output channel, or null (1.0)
    const float* row_scales;    // [M] per-row activation scales, or null (in_scale)
    float in_scale;
    int fused_scale;            // 1: v = fma(acc, in_scale * w_scale, bias) (linear.cu:362-365)
                                // 0: v = fma(acc * row_scale, w_scale, bias) (encoder.cu:975-995)
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
    int valid_rows;
    uint32_t* skip_count;       // FMT_I8_SKIP: {skipped, total} 16x128 activation blocks, or null
};

constexpr int kBlockM = 256;
constexpr int kBlockN = 256;
constexpr int kThreads = 512;
constexpr int kRowBytes = 128;
constexpr int kTileBytes = kBlockM * kRowBytes;  // the activation tile of one stage
constexpr int kMaxG128Groups = 32;               // K <= 4096 for the group-wise INT4 formats

template <int F> struct FmtTraits;
template <> struct FmtTraits<FMT_FP8> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_I8_SKIP> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = true; };
template <> struct FmtTraits<FMT_I8> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = true; };
template <> struct FmtTraits<FMT_S4> { static constexpr int kStep = 256, bRow = 128, aElemNum = 1, aElemDen = 2, bNum = 1, bDen = 2; static constexpr bool kInt = true; };
template <> struct FmtTraits<FMT_G128A8> { static constexpr int kStep = 128, bRow = 64, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 2; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_F16> { static constexpr int kStep = 64, bRow = 128, aElemNum = 2, aElemDen = 1, bNum = 2, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_G128A16> { static constexpr int kStep = 64, bRow = 32, aElemNum = 2, aElemDen = 1, bNum = 1, bDen = 2; static constexpr bool kInt = false; };
// Q4_K: per column and 64-K step the superblock's 16-byte header (d, dmin,
// 12 bytes of 6-bit scales/mins) and the step's 32 quant bytes.
template <> struct FmtTraits<FMT_S4F6> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_G128F8> { static constexpr int kStep = 128, bRow = 128, aElemNum = 1, aElemDen = 1, bNum = 1, bDen = 1; static constexpr bool kInt = false; };
template <> struct FmtTraits<FMT_Q4K> { static constexpr int kStep = 64, bRow = 48, aElemNum = 2, aElemDen = 1, bNum = 9, bDen = 16; static constexpr bool kInt = false; };

// LDS of one workgroup.  A stage holds one K-step of the activation and
// weight tiles.  The staged epilogue writes up to 64 KiB (256 rows x 256 fp8,
// or 128 rows x 256 fp16) starting at the stage the last K-step released
// (offset kStage * that buffer) while the next tile's first step is loading
// into the other buffer, so the 64 KiB from either start must miss the other
// buffer: stages are padded to 64 KiB, except for the G128 formats, whose
// per-tile group tables (fp32 scales [group][256 columns], u8 zero-points
// [group][256 columns]; refilled at each tile's first step) sit between the
// two stages and are free during the epilogue.
template <int F> struct Layout {
    static constexpr bool kG128 = (F == FMT_G128A8 || F == FMT_G128A16);
    static constexpr int kNatural = kTileBytes + kBlockN * FmtTraits<F>::bRow;
    static constexpr int kTables = kG128 ? kMaxG128Groups * kBlockN * 5 : 0;
    static constexpr int kStage = kG128 ? kNatural : (kNatural > 65536 ? kNatural : 65536);
    static constexpr int kBufStride = kStage + kTables;  // buffer b starts at b * kBufStride
    static constexpr int kScales = kStage;
    static constexpr int kZeros = kScales + kMaxG128Groups * kBlockN * 4;
    static constexpr int kBytes = 2 * kStage + kTables;
    static_assert(kStage + kTables >= 65536, "staged epilogue window");
};

// XOR key of a 128-byte LDS row's 16-byte chunks (bits: k0 = r1, k1 = r2^r4,
// k2 = r0^r3^r5).  One chunk column read by 8 (or 16) lanes then touches
// distinct banks both for 8 (16) consecutive rows and for the weight rows
// wrow(0..7 (15), bj), with 32 banks per 128 bytes as with 64 per 256 bytes.
__device__ __forceinline__ int swz_key(int row) {
    return ((row >> 1) & 1) | (((row >> 2) ^ (row >> 4)) & 1) << 1 | ((row ^ (row >> 3) ^ (row >> 5)) & 1) << 2;
}
__device__ __forceinline__ int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ swz_key(row)) << 4); }

// Weight row (within the wave's 64 columns) held by MFMA row i of block bj.
__device__ __forceinline__ int wrow(int i, int bj) { return ((i >> 2) << 4) + (bj << 2) + (i & 3); }

// XOR key of a 64-byte G128A8 weight row's 16-byte chunks: the 16 rows one
// fragment read covers, wrow(0..15, bj) = {0-3, 16-19, 32-35, 48-51} + 4 bj,
// would put rows 16 apart on the same banks; keyed by (row >> 4) & 3 their
// 8-byte reads fall on distinct banks (64 banks; at most 2 lanes a bank with 32).
__device__ __forceinline__ int g128a8_key(int row) { return (row >> 4) & 3; }

// G128A16 weight tile: per column and 64-K step 32 bytes (two 16-byte
// chunks).  A fragment read covers rows wrow(0..15, bj) = {0-3, 16-19, 32-35,
// 48-51} + 4 bj at one chunk position; stored at row * 32 + 16 c, rows 16
// apart fall on the same banks (four LDS cycles a read).  Row pairs share a
// 64-byte unit whose four chunk slots are XOR-keyed by (row >> 4) & 3, which
// spreads a read's sixteen chunks over every 16-byte bank group twice.
__device__ __forceinline__ int a16_slot(int row, int c) { return (row >> 1) * 4 + ((((row & 1) << 1) | c) ^ ((row >> 4) & 3)); }
// the (row, chunk) that 16-byte slot s of the tile holds (inverse of a16_slot)
__device__ __forceinline__ void a16_chunk_of_slot(int s, int& row, int& c) {
    const int u = s >> 2, y = (s & 3) ^ ((u >> 3) & 3);
    row = 2 * u + (y >> 1);
    c = y & 1;
}

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

__device__ __forceinline__ v4i as_v4i(const uint4& u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// One K-step of one 16x16 output block: w0/w1 are the weight chunks (first
// MFMA operand), x0/x1 the activation chunks (second operand).
template <int F>
__device__ __forceinline__ void mfma_step(v4f& accf, v4i& acci, const uint4& w0, const uint4& w1, const uint4& x0,
                                          const uint4& x1, const v4f& gscale) {
    if constexpr (F == FMT_FP8) {
        const v8i W = {(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
        const v8i X = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        accf = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(W, X, accf, 0, 0, 0, 0, 0, 0);
    } else if constexpr (F == FMT_S4F6) {
        // 32 FP6 codes a lane: the 12 data bytes of chunk g, then of chunk 4 + g
        const v8i W = {(int)w0.x, (int)w0.y, (int)w0.z, (int)w1.x, (int)w1.y, (int)w1.z, 0, 0};
        const v8i X = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x1.x, (int)x1.y, (int)x1.z, 0, 0};
        // both operands e3m2; block scales 127 (E8M0 2^0) select the scaled encoding
        accf = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(W, X, accf, 3, 3, 0, 127, 0, 127);
    } else if constexpr (F == FMT_I8 || F == FMT_I8_SKIP) {
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w0), as_v4i(x0), acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w1), as_v4i(x1), acci, 0, 0, 0);
    } else if constexpr (F == FMT_S4) {
        uint4 wl, wh, xl, xh;
        s4x8_to_s8(w0.x, wl.x, wh.x); s4x8_to_s8(w0.y, wl.y, wh.y); s4x8_to_s8(w0.z, wl.z, wh.z); s4x8_to_s8(w0.w, wl.w, wh.w);
        s4x8_to_s8(x0.x, xl.x, xh.x); s4x8_to_s8(x0.y, xl.y, xh.y); s4x8_to_s8(x0.z, xl.z, xh.z); s4x8_to_s8(x0.w, xl.w, xh.w);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(wl), as_v4i(xl), acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(wh), as_v4i(xh), acci, 0, 0, 0);
        s4x8_to_s8(w1.x, wl.x, wh.x); s4x8_to_s8(w1.y, wl.y, wh.y); s4x8_to_s8(w1.z, wl.z, wh.z); s4x8_to_s8(w1.w, wl.w, wh.w);
        s4x8_to_s8(x1.x, xl.x, xh.x); s4x8_to_s8(x1.y, xl.y, xh.y); s4x8_to_s8(x1.z, xl.z, xh.z); s4x8_to_s8(x1.w, xl.w, xh.w);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(wl), as_v4i(xl), acci, 0, 0, 0);
        acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(wh), as_v4i(xh), acci, 0, 0, 0);
    } else if constexpr (F == FMT_G128A8) {
        // w0/w1 already hold (q - z) as int8 (decoded once per step); each
        // 128-K group's exact int32 sum is scaled by its column's fp16 scale.
        v4i g = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w0), as_v4i(x0), v4i{0, 0, 0, 0}, 0, 0, 0);
        g = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w1), as_v4i(x1), g, 0, 0, 0);
        accf[0] = __builtin_fmaf((float)g[0], gscale[0], accf[0]);
        accf[1] = __builtin_fmaf((float)g[1], gscale[1], accf[1]);
        accf[2] = __builtin_fmaf((float)g[2], gscale[2], accf[2]);
        accf[3] = __builtin_fmaf((float)g[3], gscale[3], accf[3]);
    } else if constexpr (F == FMT_G128F8) {
        const v8i W = {(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
        const v8i X = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        const v4f g = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(W, X, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
        accf[0] = __builtin_fmaf(g[0], gscale[0], accf[0]);
        accf[1] = __builtin_fmaf(g[1], gscale[1], accf[1]);
        accf[2] = __builtin_fmaf(g[2], gscale[2], accf[2]);
        accf[3] = __builtin_fmaf(g[3], gscale[3], accf[3]);
    } else {  // F16, G128A16 and Q4K (weights already dequantized to halves)
        accf = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w0), __builtin_bit_cast(v8h, x0), accf, 0, 0, 0);
        accf = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w1), __builtin_bit_cast(v8h, x1), accf, 0, 0, 0);
    }
}

// 16 bytes global -> LDS per lane (global_load_lds_dwordx4): lane l writes
// LDS bytes [lds_addr + 16 l, + 16).  lds_addr must be wave-uniform.  Issued
// from inline asm so that the compiler does not order every later LDS read
// behind the load (it cannot tell the DMA target from the buffer being read);
// the step loop waits for these loads explicitly.  An LDS DMA reading M0
// needs one wait state after the SALU write of M0 (the compiler inserts it
// for the builtin, not inside inline asm), hence the s_nop.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory", "m0");
}
// Same with a wave-uniform 64-bit base (SGPR pair) and a 32-bit lane offset.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory", "m0");
}

// Persistent tile schedule.  The grid is one workgroup per CU (G of them);
// iteration i of workgroup b computes logical tile i*G + slot(b).  Workgroups
// are dispatched round-robin over the 8 XCDs, so slot() gives each XCD a
// contiguous run of G/8 logical tiles per iteration.  Logical tiles are
// ordered by groups of GW weight column-tiles, then by activation row-strip,
// then by column-tile within the group, so one XCD's run covers G/8/GW row
// strips of one column group, and its next runs keep the same weight columns
// (L2-resident) while sweeping new rows.
__device__ __forceinline__ int tile_slot(int G) {
    const int b = blockIdx.x;
    return (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
}

__device__ __forceinline__ int group_width(int tiles_n) {
    return (tiles_n & 7) == 0 ? 8 : ((tiles_n & 3) == 0 ? 4 : ((tiles_n & 1) == 0 ? 2 : 1));
}

// e4m3 of 16 * fp16(SiLU(v)) for four values packed in a dword (the FF
// expand epilogue, encoder.cu:1010-1025).  SiLU is >= -0.279, so clamping at
// 28 (= 448 / 16) before the fp16 rounding is the reference's saturation;
// v_cvt_scalef32_pk_fp8_f16 converts two fp16 values divided by its scale
// operand (1/16 here) with round-to-nearest-even.
__device__ __forceinline__ uint32_t silu_fp8x4(float a, float b, float c, float d) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    const v2h h01 = {(_Float16)__builtin_fminf(silu(a), 28.0f), (_Float16)__builtin_fminf(silu(b), 28.0f)};
    const v2h h23 = {(_Float16)__builtin_fminf(silu(c), 28.0f), (_Float16)__builtin_fminf(silu(d), 28.0f)};
    v2s o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(v2s{0, 0}, h01, 0.0625f, false);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, h23, 0.0625f, true);
    return __builtin_bit_cast(uint32_t, o);
}

// int8 of 16 * fp16(SiLU(v)) for four values packed in a dword: the
// reference's static INT8 quantizer (linear.cu:549-560, rne(clamp(x * s,
// +-127))) at the FF hidden scale 16 of the e4m3 epilogue above.  The fp16
// value times 16 is exact in fp32; adding 1.5 * 2^23 leaves rne(q) in the low
// mantissa bits (|q| <= 127).
__device__ __forceinline__ uint32_t silu_i8x4(float a, float b, float c, float d) {
    const float x[4] = {a, b, c, d};
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float h = round_f16(silu(x[i])) * 16.0f;
        q[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_fmed3f(h, -127.0f, 127.0f) + 12582912.0f);
    }
    const uint32_t ab = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(q[3], q[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// encoder.cu:685-704: of one quartet of e4m3 bytes keep the two largest
// magnitudes (bits & 127, ties to the lower index) in index order.  Returns
// the two kept bytes in bits 0-15 and idx0 | idx1 << 2 in bits 16-19.
// Branch-free: key i = magnitude << 2 | (3 - i) orders the elements by
// magnitude, then lower index, with distinct keys; the two largest keys of
// the four come from one max / min exchange per pair and a merge.
__device__ __forceinline__ uint32_t compress_quartet(uint32_t packed) {
    const uint32_t k0 = ((packed << 2) & 0x1fcu) | 3u, k1 = ((packed >> 6) & 0x1fcu) | 2u;
    const uint32_t k2 = ((packed >> 14) & 0x1fcu) | 1u, k3 = (packed >> 22) & 0x1fcu;
    const uint32_t a = max(k0, k1), b = min(k0, k1), c = max(k2, k3), d = min(k2, k3);
    const uint32_t i1 = 3u - (max(a, c) & 3u), i2 = 3u - (max(min(a, c), max(b, d)) & 3u);
    const uint32_t lo = min(i1, i2), hi = max(i1, i2);
    // v_perm selector: byte lo, byte hi, then two zero bytes (selector 0x0c)
    const uint32_t data = __builtin_amdgcn_perm(0u, packed, lo | (hi << 8) | 0x0c0c0000u);
    return data | ((lo | (hi << 2)) << 16);
}

// fp16 row-block stores that write whole cache lines.  A lane holds 16
// consecutive fp16 outputs (two 16-byte halves) of row r = 16-row block + l16,
// so the four lanes of a row cover the wave's 128-byte row segment and each
// plain 16-byte store instruction writes half of every line it touches.  The
// lanes holding rows r (l16 even) and r + 1 trade halves (one DPP quad_perm
// [1, 0, 3, 2] per dword): the first store then writes row r from both lanes,
// the second row r + 1, each instruction 8 rows x whole 128-byte segments.
__device__ __forceinline__ void store_f16_rowpair(uint16_t* out, size_t ldo, int grow, int gcol, int m, bool col_live, int l16,
                                                  const uint32_t (&h)[8]) {
    const bool odd = (l16 & 1) != 0;
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = (uint32_t)dpp_mov<0xB1>((int)(odd ? h[i] : h[4 + i]));
    const int r0 = grow - (odd ? 1 : 0);
    const int col = gcol + (odd ? 8 : 0);
    const uint4 s1 = odd ? uint4{y[0], y[1], y[2], y[3]} : uint4{h[0], h[1], h[2], h[3]};
    const uint4 s2 = odd ? uint4{h[4], h[5], h[6], h[7]} : uint4{y[0], y[1], y[2], y[3]};
    if (col_live && r0 < m) *(uint4*)(out + (size_t)r0 * ldo + col) = s1;
    if (col_live && r0 + 1 < m) *(uint4*)(out + (size_t)(r0 + 1) * ldo + col) = s2;
}

// Epilogue straight from the accumulators: for each of its 8 row blocks a
// lane finishes columns [gcol, gcol + 16) of one row (16 contiguous outputs,
// one to four 16-byte stores).  Column scales / bias and the 8 row scales are
// loaded once per tile; a residual row (kRes) is loaded one block ahead.
// With `stage` (4 KiB of LDS private to the wave, free), fp32 outputs of a
// row block pass through it so that every store instruction writes 8 rows x
// 128 contiguous bytes (whole cache lines): the direct stores put a row's
// 16-byte pieces 64 bytes apart per instruction, and a burst of such stores
// drains at about 60 % of the whole-line rate (C1, 192 tiles of 128 x 128
// fp32: 12.8 -> 11.1 us).  Measured no faster for fp16 outputs.
template <int F, int E, bool kRes = true, int kAI = 8>
__device__ __forceinline__ void epilogue(const GemmArgs& p, v4f (&accf)[kAI][4], v4i (&acci)[kAI][4], int m0, int n0, int wm,
                                         int wn, int lane, uint8_t* stage = nullptr) {
    using T = FmtTraits<F>;
    const int g = lane >> 4, l16 = lane & 15;
    const int gcol = n0 + wn * 64 + g * 16;
    const int ccol = min(gcol, p.n - 16);
    const bool col_live = gcol < p.n;
    float wsv[16], bsv[16], rsv[kAI];
    if constexpr (E != EPI_I32) {
#pragma unroll
        for (int j = 0; j < 16; j += 4) {
            const float4 w4 = p.w_scales ? *(const float4*)(p.w_scales + ccol + j) : float4{1.f, 1.f, 1.f, 1.f};
            const float4 b4 = p.bias ? *(const float4*)(p.bias + ccol + j) : float4{0.f, 0.f, 0.f, 0.f};
            wsv[j] = w4.x; wsv[j + 1] = w4.y; wsv[j + 2] = w4.z; wsv[j + 3] = w4.w;
            bsv[j] = b4.x; bsv[j + 1] = b4.y; bsv[j + 2] = b4.z; bsv[j + 3] = b4.w;
        }
#pragma unroll
        for (int ai = 0; ai < kAI; ++ai) {
            const int row = min(m0 + wm * 16 * kAI + ai * 16 + l16, p.m - 1);
            rsv[ai] = p.row_scales ? p.row_scales[row] : p.in_scale;
        }
    }
    // Retire the scale loads once here; a wait for them inside the block loop
    // would also wait for the previous block's stores.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    auto row_of = [&](int ai) { return min(m0 + wm * 16 * kAI + ai * 16 + l16, p.m - 1); };
    // Without a residual the loads read the (same-shaped) output instead and
    // a select discards them, keeping the block loop free of branches.
    const uint16_t* res_src = p.residual ? p.residual : (const uint16_t*)p.out;
    const bool has_res = kRes && p.residual != nullptr;
    uint4 rn0 = {0, 0, 0, 0}, rn1 = {0, 0, 0, 0};
    if constexpr (E == EPI_F16 && kRes) {
        const uint4* rp = (const uint4*)(res_src + (size_t)row_of(0) * p.ldo + ccol);
        rn0 = rp[0];
        rn1 = rp[1];
    }
#pragma unroll
    for (int ai = 0; ai < kAI; ++ai) {
        const int grow = m0 + wm * 16 * kAI + ai * 16 + l16;
        const bool live = grow < p.m && col_live;
        float v[16];
        if constexpr (E == EPI_I32) {
            if (live) {
                int4* o = (int4*)((int32_t*)p.out + (size_t)grow * p.ldo + gcol);
#pragma unroll
                for (int bj = 0; bj < 4; ++bj) o[bj] = int4{acci[ai][bj][0], acci[ai][bj][1], acci[ai][bj][2], acci[ai][bj][3]};
            }
            continue;
        } else {
#pragma unroll
            for (int bj = 0; bj < 4; ++bj)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[bj * 4 + r] = T::kInt ? (float)acci[ai][bj][r] : accf[ai][bj][r];
        }
        const float rs = rsv[ai];
        if (p.fused_scale) {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j], rs * wsv[j], bsv[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j] * rs, wsv[j], bsv[j]);
        }
        if constexpr (E == EPI_F32) {
            if (stage != nullptr) {
                // row l16 of the block, 16-byte chunk q = 4 g + j of its 256-byte
                // slab at slot q ^ l16 (8 consecutive lanes: distinct banks)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *(float4*)(stage + l16 * 256 + (((4 * g + j) ^ l16) << 4)) = float4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = (j & 1) * 8 + (lane >> 3), q = (j >> 1) * 8 + (lane & 7);
                    const float4 x = *(const float4*)(stage + r * 256 + ((q ^ r) << 4));
                    const int orow = m0 + wm * 16 * kAI + ai * 16 + r, ocol = n0 + wn * 64 + 4 * q;
                    if (orow < p.m && ocol < p.n) *(float4*)((float*)p.out + (size_t)orow * p.ldo + ocol) = x;
                }
            } else if (live) {
                float4* o = (float4*)((float*)p.out + (size_t)grow * p.ldo + gcol);
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = float4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
            }
        } else if constexpr (E == EPI_F16) {
            const uint4 r0 = rn0, r1 = rn1;
            if (kRes && ai + 1 < kAI) {
                const uint4* rp = (const uint4*)(res_src + (size_t)row_of(ai + 1) * p.ldo + ccol);
                rn0 = rp[0];
                rn1 = rp[1];
            }
            const uint32_t rw[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
            uint32_t h[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float y0 = v[2 * j] * p.out_scale, y1 = v[2 * j + 1] * p.out_scale;
                float x0 = has_res ? __builtin_fmaf(p.res_scale, h2f((uint16_t)(rw[j] & 0xffff)), y0) : y0;
                float x1 = has_res ? __builtin_fmaf(p.res_scale, h2f((uint16_t)(rw[j] >> 16)), y1) : y1;
                x0 = p.act == 1 ? silu(x0) : (p.act == 2 ? __builtin_fmaxf(x0, 0.0f) : x0);
                x1 = p.act == 1 ? silu(x1) : (p.act == 2 ? __builtin_fmaxf(x1, 0.0f) : x1);
                h[j] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
            }
            if constexpr (kRes) {
                // residual epilogues (read-modify-write of the output rows): whole-line stores
                // measured 2-11 % faster; plain fp16 outputs keep the direct stores
                (void)live;
                store_f16_rowpair((uint16_t*)p.out, (size_t)p.ldo, grow, gcol, p.m, col_live, l16, h);
            } else if (live) {
                uint4* o = (uint4*)((uint16_t*)p.out + (size_t)grow * p.ldo + gcol);
                o[0] = uint4{h[0], h[1], h[2], h[3]};
                o[1] = uint4{h[4], h[5], h[6], h[7]};
            }
        } else if constexpr (E == EPI_I8S) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = silu_i8x4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            if (live) *(uint4*)((uint8_t*)p.out + (size_t)grow * p.ldo + gcol) = uint4{w[0], w[1], w[2], w[3]};
        } else {  // EPI_F8, EPI_F8_24
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = silu_fp8x4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            if constexpr (E == EPI_F8) {
                if (live) *(uint4*)((uint8_t*)p.out + (size_t)grow * p.ldo + gcol) = uint4{w[0], w[1], w[2], w[3]};
            } else {
                uint32_t c[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) c[j] = compress_quartet(w[j]);
                if (live) {
                    const uint32_t d0 = (c[0] & 0xffff) | (c[1] << 16), d1 = (c[2] & 0xffff) | (c[3] << 16);
                    const uint32_t meta = (c[0] >> 16) | ((c[1] >> 16) << 4) | ((c[2] >> 16) << 8) | ((c[3] >> 16) << 12);
                    *(uint2*)((uint8_t*)p.out + (size_t)grow * (p.ldo / 2) + gcol / 2) = uint2{d0, d1};
                    *(uint16_t*)(p.out_meta + (size_t)grow * (p.ldo / 8) + gcol / 8) = (uint16_t)meta;
                }
            }
        }
    }
}


// Weight fragment of tile-local weight row `row` for one K-step: the lane's
// two 16-byte operand chunks (lane group g), decoded to the MFMA input type.
// sc / zr are the step's 128-K group scales / zero-points indexed by
// tile-local column (G128 formats); gs returns the group scales of the 4
// columns block bj's accumulators hold (G128A8: 16g + 4bj + r of the wave's 64).
template <int F>
__device__ __forceinline__ void weight_frag(const uint8_t* Bs, int row, int g, int bj, int wn, int step, const float* sc,
                                            const uint8_t* zr, uint4& w0, uint4& w1, v4f& gs) {
    using T = FmtTraits<F>;
    gs = v4f{1.f, 1.f, 1.f, 1.f};
    if constexpr (T::bRow == 128) {
        w0 = *(const uint4*)(Bs + swz(row, g));
        w1 = *(const uint4*)(Bs + swz(row, 4 + g));
    } else if constexpr (F == FMT_Q4K) {
        // K slots 8g..8g+7 are the low nibbles of quant bytes 8g..8g+7 (group
        // 2*(step&3)), K slots 32+8g.. the high nibbles (group 2*(step&3)+1).
        const uint4 h = *(const uint4*)(Bs + row * 48);
        const uint2 q = *(const uint2*)(Bs + row * 48 + 16 + 8 * g);
        float al, bl, ah, bh;
        q4k_coeffs(h, 2 * (step & 3), al, bl);
        q4k_coeffs(h, 2 * (step & 3) + 1, ah, bh);
        w0 = q4k_decode8(q.x & 0x0f0f0f0fu, q.y & 0x0f0f0f0fu, al, bl);
        w1 = q4k_decode8((q.x >> 4) & 0x0f0f0f0fu, (q.y >> 4) & 0x0f0f0f0fu, ah, bh);
    } else {
        const int z = zr[row];
        if constexpr (F == FMT_G128A8) {
            gs = *(const v4f*)(sc + wn * 64 + g * 16 + bj * 4);
            const uint32_t zz = (uint32_t)z * 0x01010101u;
            // logical bytes 8g and 32 + 8g of the row, its 16-byte chunks stored XOR-keyed
            const int key = g128a8_key(row), half = (g & 1) << 3;
            const uint2 q0 = *(const uint2*)(Bs + row * 64 + ((((g >> 1)) ^ key) << 4) + half);
            const uint2 q1 = *(const uint2*)(Bs + row * 64 + (((2 + (g >> 1)) ^ key) << 4) + half);
            u4x8_minus_z(q0.x, zz, w0.x, w0.y);
            u4x8_minus_z(q0.y, zz, w0.z, w0.w);
            u4x8_minus_z(q1.x, zz, w1.x, w1.y);
            u4x8_minus_z(q1.y, zz, w1.z, w1.w);
        } else {  // G128A16
            const _Float16 s = (_Float16)sc[row];
            const _Float16 zh = (_Float16)(1024 + z);
            const v2h ss = {s, s}, zz = {zh, zh};
            const uint32_t q0 = *(const uint32_t*)(Bs + a16_slot(row, 0) * 16 + 4 * g);
            const uint32_t q1 = *(const uint32_t*)(Bs + a16_slot(row, 1) * 16 + 4 * g);
            w0 = __builtin_bit_cast(uint4, u4x8_to_h(q0, zz, ss));
            w1 = __builtin_bit_cast(uint4, u4x8_to_h(q1, zz, ss));
        }
    }
}

// Output bytes per element of an epilogue.
template <int E> struct EpiBytes { static constexpr int v = (E == EPI_F8 || E == EPI_F8_24 || E == EPI_I8S) ? 1 : (E == EPI_F16 ? 2 : 4); };

// Epilogue through LDS for outputs without a residual: the waves convert
// their accumulators to output bytes and place them in the stage buffer the
// last K-step has just released (64 KiB: the whole 256x256 tile of fp8, half
// of fp16, a quarter of fp32 per pass); then all 512 threads store whole row
// segments, so one wave instruction writes four rows x 256 bytes of fp8.  16-
// byte chunks of a staged row are XOR-swizzled by (row & 15).
template <int F, int E>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& p, v4f (&accf)[8][4], v4i (&acci)[8][4], uint8_t* sbuf, int m0,
                                                int n0, int wm, int wn, int lane, int tid) {
    using T = FmtTraits<F>;
    constexpr int eb = EpiBytes<E>::v;
    static_assert(eb <= 2, "fp32 / int32 outputs use the register epilogue");
    constexpr int kRows = 256 / eb;          // rows staged per pass
    constexpr int kChunks = 16 * eb;         // 16-byte chunks per staged row (full width)
    const int g = lane >> 4, l16 = lane & 15;
    const int lcol = wn * 64 + g * 16;       // first of the lane's 16 columns within the tile
    const int gcol = n0 + lcol;
    const int ccol = min(gcol, p.n - 16);
    float wsv[16], bsv[16], rsv[8];
    if constexpr (E != EPI_I32) {
#pragma unroll
        for (int j = 0; j < 16; j += 4) {
            const float4 w4 = p.w_scales ? *(const float4*)(p.w_scales + ccol + j) : float4{1.f, 1.f, 1.f, 1.f};
            const float4 b4 = p.bias ? *(const float4*)(p.bias + ccol + j) : float4{0.f, 0.f, 0.f, 0.f};
            wsv[j] = w4.x; wsv[j + 1] = w4.y; wsv[j + 2] = w4.z; wsv[j + 3] = w4.w;
            bsv[j] = b4.x; bsv[j + 1] = b4.y; bsv[j + 2] = b4.z; bsv[j + 3] = b4.w;
        }
#pragma unroll
        for (int ai = 0; ai < 8; ++ai) {
            const int row = min(m0 + wm * 128 + ai * 16 + l16, p.m - 1);
            rsv[ai] = p.row_scales ? p.row_scales[row] : p.in_scale;
        }
    }
    const int ntile_cols = min(256, p.n - n0);  // multiple of 16
#pragma unroll
    for (int pass = 0; pass < eb; ++pass) {
        __syncthreads();  // the previous pass's stores have read the staging area
        // fp8: one pass, every wave; fp16: pass 0 = waves 0-3, pass 1 = 4-7
        if (eb == 2 && wm != pass) goto staged_store;
#pragma unroll
        for (int ai = 0; ai < 8; ++ai) {
            const int srow = (eb == 2 ? 0 : wm * 128) + ai * 16 + l16;
            uint8_t* dst = sbuf + srow * (kChunks * 16);
            auto put = [&](int chunk, uint4 val) { *(uint4*)(dst + ((chunk ^ (srow & 15)) << 4)) = val; };
            if constexpr (E == EPI_I32) {
#pragma unroll
                for (int bj = 0; bj < 4; ++bj)
                    put(lcol / 4 + bj, uint4{(uint32_t)acci[ai][bj][0], (uint32_t)acci[ai][bj][1], (uint32_t)acci[ai][bj][2], (uint32_t)acci[ai][bj][3]});
                continue;
            } else {
                float v[16];
#pragma unroll
                for (int bj = 0; bj < 4; ++bj)
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[bj * 4 + r] = T::kInt ? (float)acci[ai][bj][r] : accf[ai][bj][r];
                const float rs = rsv[ai];
                if (p.fused_scale) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j], rs * wsv[j], bsv[j]);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j] * rs, wsv[j], bsv[j]);
                }
                if constexpr (E == EPI_F32) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        put(lcol / 4 + j, __builtin_bit_cast(uint4, float4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]}));
                } else if constexpr (E == EPI_F16) {
                    uint32_t h[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        float x0 = v[2 * j] * p.out_scale, x1 = v[2 * j + 1] * p.out_scale;
                        x0 = p.act == 1 ? silu(x0) : (p.act == 2 ? __builtin_fmaxf(x0, 0.0f) : x0);
                        x1 = p.act == 1 ? silu(x1) : (p.act == 2 ? __builtin_fmaxf(x1, 0.0f) : x1);
                        h[j] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
                    }
                    put(lcol / 8, uint4{h[0], h[1], h[2], h[3]});
                    put(lcol / 8 + 1, uint4{h[4], h[5], h[6], h[7]});
                } else {
                    uint32_t w[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) w[j] = silu_fp8x4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
                    if constexpr (E == EPI_F8) {
                        put(lcol / 16, uint4{w[0], w[1], w[2], w[3]});
                    } else {
                        // 2:4 compressed: 8 data bytes at lcol/2 of a 128-byte
                        // data row, 2 metadata bytes at lcol/8 of a 32-byte row
                        // placed after the 32 KiB of data rows.
                        uint32_t c[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) c[j] = compress_quartet(w[j]);
                        const uint32_t d0 = (c[0] & 0xffff) | (c[1] << 16), d1 = (c[2] & 0xffff) | (c[3] << 16);
                        const uint32_t meta = (c[0] >> 16) | ((c[1] >> 16) << 4) | ((c[2] >> 16) << 8) | ((c[3] >> 16) << 12);
                        uint8_t* drow = sbuf + srow * 128;
                        const int dchunk = lcol >> 5, dhalf = (lcol >> 4) & 1;
                        *(uint2*)(drow + ((dchunk ^ (srow & 7)) << 4) + dhalf * 8) = uint2{d0, d1};
                        *(uint16_t*)(sbuf + 32768 + srow * 32 + lcol / 8) = (uint16_t)meta;
                    }
                }
            }
        }
    staged_store:
        __syncthreads();
        // Store phase: chunk q of the pass is row q / row_chunks, 16-byte
        // column chunk q % row_chunks; rows past M and columns past N drop.
        if constexpr (E == EPI_F8_24) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = i * kThreads + tid, row = q >> 3, c = q & 7;
                const int grow = m0 + row;
                if (grow < p.m && c * 32 < ntile_cols)
                    *(uint4*)((uint8_t*)p.out + (size_t)grow * (p.ldo / 2) + n0 / 2 + c * 16) =
                        *(const uint4*)(sbuf + row * 128 + ((c ^ (row & 7)) << 4));
            }
            {
                const int row = tid >> 1, c = tid & 1;
                const int grow = m0 + row;
                if (grow < p.m && c * 128 < ntile_cols) {
                    const uint4 mv = *(const uint4*)(sbuf + 32768 + row * 32 + c * 16);
                    uint8_t* md = p.out_meta + (size_t)grow * (p.ldo / 8) + n0 / 8 + c * 16;
                    if (ntile_cols - c * 128 >= 128) *(uint4*)md = mv;
                    else {
                        const uint8_t* mb = (const uint8_t*)&mv;
                        for (int j = 0; j < (ntile_cols - c * 128) / 8; ++j) md[j] = mb[j];
                    }
                }
            }
        } else {
            constexpr int kIters = kRows * kChunks / kThreads;
#pragma unroll
            for (int i = 0; i < kIters; ++i) {
                const int q = i * kThreads + tid, row = q / kChunks, c = q % kChunks;
                const int grow = m0 + pass * kRows + row;
                if (grow < p.m && c * (16 / eb) < ntile_cols)
                    *(uint4*)((uint8_t*)p.out + ((size_t)grow * p.ldo + n0) * eb + c * 16) =
                        *(const uint4*)(sbuf + row * (kChunks * 16) + ((c ^ (row & 15)) << 4));
            }
        }
    }
}

// GLU tiles (pointwise1 + GLU, encoder.cu:911-947): a 256-row weight tile
// starting at n0 serves output columns [n0/2, n0/2 + 128).  Tile row L holds
// value row c + (L & 7) for L % 16 < 8 and the matching gate row (+ N/2) for
// L % 16 >= 8, c = n0/2 + 8 (L / 16), so each lane's 16 accumulators are 8
// values and their 8 gates.
__device__ __forceinline__ int glu_row(int n0, int L, int n) {
    const int half = n >> 1;
    const int col = min((n0 >> 1) + ((L >> 4) << 3) + (L & 7), half - 1);
    return col + ((L & 8) ? half : 0);
}

// GLU epilogue: out[row, c + j] = fp16(fp16(v_j) / (1 + exp(-fp16(g_j)))),
// rows >= valid_rows written as zero (encoder.cu:936-947).
__device__ __forceinline__ void epilogue_glu(const GemmArgs& p, v4f (&accf)[8][4], int m0, int n0, int wm, int wn, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    const int half = p.n >> 1;
    const int oc = (n0 >> 1) + ((wn * 4 + g) << 3);  // first of the lane's 8 output columns
    const bool col_live = oc < half;
    const int cc = min(oc, half - 8);
    float wv[8], wg[8], rsv[8];
#pragma unroll
    for (int j = 0; j < 8; j += 4) {
        const float4 a = *(const float4*)(p.w_scales + cc + j);
        const float4 b = *(const float4*)(p.w_scales + half + cc + j);
        wv[j] = a.x; wv[j + 1] = a.y; wv[j + 2] = a.z; wv[j + 3] = a.w;
        wg[j] = b.x; wg[j + 1] = b.y; wg[j + 2] = b.z; wg[j + 3] = b.w;
    }
#pragma unroll
    for (int ai = 0; ai < 8; ++ai) {
        const int row = min(m0 + wm * 128 + ai * 16 + l16, p.m - 1);
        rsv[ai] = p.row_scales ? p.row_scales[row] : p.in_scale;
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
#pragma unroll
    for (int ai = 0; ai < 8; ++ai) {
        const int grow = m0 + wm * 128 + ai * 16 + l16;
        const float rs = rsv[ai];
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            float o[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int jj = j + u;
                const float val = round_f16(accf[ai][jj >> 2][jj & 3] * rs * wv[jj]);
                const float gate = round_f16(accf[ai][(jj + 8) >> 2][(jj + 8) & 3] * rs * wg[jj]);
                o[u] = grow < p.valid_rows ? val * __builtin_amdgcn_rcpf(1.0f + __expf(-gate)) : 0.0f;
            }
            h[j >> 1] = (uint32_t)f2h(o[0]) | ((uint32_t)f2h(o[1]) << 16);
        }
        if (grow < p.m && col_live) *(uint4*)((uint16_t*)p.out + (size_t)grow * p.ldo + oc) = uint4{h[0], h[1], h[2], h[3]};
    }
}

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
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;  // bytes per activation row
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;          // bytes per weight row
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    const uint8_t* __restrict__ pa = p.a;
    const uint8_t* __restrict__ pb = p.b;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    float* g_scale = (float*)(lds + L::kScales);
    uint8_t* g_zero = lds + L::kZeros;

    // Direct-to-LDS loads: one wave instruction fills 1 KiB of LDS, lane l
    // writing bytes [16l, 16l+16), so each lane loads the global chunk the
    // swizzled layout puts there.
    // Weight loads: wave w issues instructions bj(w, i) of the stage's kBLoads
    // (a contiguous run per wave; interleaved when kBLoads is not a multiple of 8).
    constexpr int kBLoads = (kBlockN * T::bRow) / 1024;
    constexpr int kBLoadsPerWave = (kBLoads + 7) / 8;
    auto bj_index = [&](int i) { return kBLoads % 8 == 0 ? wave * kBLoadsPerWave + i : i * 8 + wave; };
    uint32_t b_q4k = 0;  // Q4K: bit i set when load i carries quant bytes
    uint32_t a_off[4], b_off[kBLoadsPerWave];
    const int tiles_m = (p.m + kBlockM - 1) / kBlockM;
    const int gw = group_width(tiles_n);
    auto set_tile = [&](int t, int& m0, int& n0) {
        const int ng = t / (tiles_m * gw);
        const int r = t - ng * tiles_m * gw;
        const int tm = r / gw;
        m0 = tm * kBlockM;
        n0 = (ng * gw + (r - tm * gw)) * kBlockN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (wave * 4 + i) * 1024 + lane * 16;
            const int row = o >> 7, c = ((o >> 4) & 7) ^ swz_key(row);
            a_off[i] = (uint32_t)((size_t)min(m0 + row, p.m - 1) * lda + c * 16);
        }
#pragma unroll
        for (int i = 0; i < kBLoadsPerWave; ++i) {
            const int o = bj_index(i) * 1024 + lane * 16;
            int row, c;
            if constexpr (T::bRow == 128) {
                row = o >> 7;
                c = ((o >> 4) & 7) ^ swz_key(row);
            } else if constexpr (F == FMT_G128A16) {
                a16_chunk_of_slot(o >> 4, row, c);
            } else {
                row = o / T::bRow;
                c = (o % T::bRow) / 16;
            }
            int wr;
            if constexpr (E == EPI_GLU) wr = glu_row(n0, row, p.n);
            else wr = min(n0 + row, p.n - 1);
            b_off[i] = (uint32_t)((size_t)wr * ldb + c * 16);
            if constexpr (F == FMT_Q4K) b_q4k = c > 0 ? b_q4k | (1u << i) : b_q4k & ~(1u << i);
        }
    };
    auto issue = [&](int step, int buf) {
        const uint32_t base = lds_base + buf * L::kBufStride;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(pa + (size_t)step * kRowBytes, a_off[i], base + (wave * 4 + i) * 1024);
#pragma unroll
        for (int i = 0; i < kBLoadsPerWave; ++i) {
            if (kBLoads % 8 != 0 && bj_index(i) >= kBLoads) continue;
            if constexpr (F == FMT_Q4K) {
                // superblock step >> 2; quant chunks advance 32 bytes per step
                const uint32_t qa = (b_q4k >> i) & 1u ? (uint32_t)(step & 3) * 32u : 0u;
                dma16(pb + (size_t)(step >> 2) * 144, b_off[i] + qa, base + kTileBytes + bj_index(i) * 1024);
            } else {
                dma16(pb + (size_t)step * T::bRow, b_off[i], base + kTileBytes + bj_index(i) * 1024);
            }
        }
    };

    int t = tile_slot(G);
    if (t >= ntiles) return;
    int m0, n0;
    set_tile(t, m0, n0);
    issue(0, 0);
    int buf = 0;

    v4f accf[8][4];
    v4i acci[8][4];
    uint32_t skipped = 0, blocks = 0;

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
                        const int grp = idx >> 8, col = idx & 255;
                        const size_t gi = (size_t)min(cur_n0 + col, p.n - 1) * groups + grp;
                        g_scale[idx] = h2f(p.g_scales[gi]);
                        g_zero[idx] = (uint8_t)(int)h2f(p.g_zeros[gi]);
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
            const uint8_t* As = lds + buf * L::kBufStride;
            const uint8_t* Bs = As + kTileBytes;

            // This wave's four weight fragments for the step.
            uint4 w0[4], w1[4];
            v4f gs[4];
            const int kg = (step * T::kStep) >> 7;
#pragma unroll
            for (int bj = 0; bj < 4; ++bj)
                weight_frag<F>(Bs, wn * 64 + wrow(l16, bj), g, bj, wn, step, g_scale + kg * kBlockN, g_zero + kg * kBlockN, w0[bj],
                               w1[bj], gs[bj]);
            // Activation fragments are read one 16-row block ahead of the
            // MFMAs that consume them where the step's weight decode leaves the
            // registers for it (FP8, INT8, FP16).
            constexpr bool kAhead = F == FMT_FP8 || F == FMT_I8 || F == FMT_I8_SKIP || F == FMT_F16;
            uint4 x0, x1, y0, y1;
            if constexpr (kAhead) {
                const int row = wm * 128 + l16;
                x0 = *(const uint4*)(As + swz(row, g));
                x1 = *(const uint4*)(As + swz(row, 4 + g));
            }
#pragma unroll
            for (int ai = 0; ai < 8; ++ai) {
                if (!kAhead || ai + 1 < 8) {
                    const int row = wm * 128 + (kAhead ? ai + 1 : ai) * 16 + l16;
                    y0 = *(const uint4*)(As + swz(row, g));
                    y1 = *(const uint4*)(As + swz(row, 4 + g));
                }
                if constexpr (!kAhead) {
                    x0 = y0;
                    x1 = y1;
                }
                bool live = true;
                if constexpr (F == FMT_I8_SKIP) {
                    // Activation-sparse FF2: the wave's 64 lanes hold this
                    // 16-row x 128-K activation block; when every byte is zero
                    // its products are exactly zero and the MFMAs are skipped.
                    const bool nz = (x0.x | x0.y | x0.z | x0.w | x1.x | x1.y | x1.z | x1.w) != 0u;
                    live = __builtin_amdgcn_ballot_w64(nz) != 0;
                    skipped += live ? 0u : 1u;
                }
                if (live) {
#pragma unroll
                    for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[ai][bj], acci[ai][bj], w0[bj], w1[bj], x0, x1, gs[bj]);
                }
                if constexpr (kAhead) {
                    x0 = y0;
                    x1 = y1;
                }
            }
            if constexpr (F == FMT_FP8 || F == FMT_I8) {
                // Scheduling order: the 8 weight reads and the first block's 2
                // activation reads, then per block the next block's 2 reads
                // ahead of this block's MFMAs.
                constexpr int kMfma = F == FMT_FP8 ? 4 : 8;
                __builtin_amdgcn_sched_group_barrier(0x100, 10, 0);
#pragma unroll
                for (int ai = 0; ai < 8; ++ai) {
                    if (ai + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
                }
            }
            buf ^= 1;
        }
        blocks += 8 * steps;

        // Outputs without a residual go through the stage buffer the last
        // K-step has released (buf ^ 1 after the final flip); the next tile's
        // first step is already loading into the other buffer.
        if constexpr (E == EPI_GLU) epilogue_glu(p, accf, cur_m0, cur_n0, wm, wn, lane);
        else if constexpr (E == EPI_F16_RES) epilogue<F, EPI_F16>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
        else if constexpr (E == EPI_F32 || E == EPI_I32) epilogue<F, E>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
        else epilogue_staged<F, E>(p, accf, acci, lds + (buf ^ 1) * L::kStage, cur_m0, cur_n0, wm, wn, lane, tid);
        if (t_next >= ntiles) break;
        t = t_next;
    }
    if constexpr (F == FMT_I8_SKIP) {
        if (p.skip_count && lane == 0) {
            atomicAdd(p.skip_count, skipped);
            atomicAdd(p.skip_count + 1, blocks);
        }
    }
}

}  // namespace pk
