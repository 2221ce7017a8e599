// Occupancy-2 GEMM engine (gfx950) for every format but the GLU epilogue.
//
// Two independent workgroups share each CU, so one workgroup's epilogue
// (VALU: scaling, SiLU, conversions, stores) and its barrier waits run while
// the other issues MFMAs.  A workgroup is 4 wave64s (one per SIMD) walking
// 256x128 output tiles persistently; wave w owns rows 128*(w/2) .. +128 and
// columns 64*(w%2) .. +64, with the fragment layout, MFMAs and register
// epilogue of the 256x256 engine (16x16x128 blocks, weights as the first
// operand, a lane's 16 accumulators of one row = 16 consecutive columns).
//
// LDS per workgroup (80 KiB, two per CU): the activation tile (256 rows x 128
// bytes) double buffered, the weight tile (128 rows x 128 bytes) single
// buffered.  Each K-step: wait for this wave's loads, barrier (the step's
// tiles are complete); every wave copies its four weight fragments into
// registers and the next activation tile starts loading; a second barrier
// (all weight fragments copied) lets the next weight tile load into the same
// buffer while the MFMAs run.  Loads are direct-to-LDS.  The G128 formats
// stream each step's group scales / zero-points (tile columns) through a
// two-slot LDS table written alongside the next weight tile.
#pragma once

#include "pk_gemm.hpp"

namespace pk {
namespace g3 {

constexpr int kBN = 128, kThreads = 256;

// Group tables of one 128-column tile for all K groups, laid out
// [group][column] in LDS: scales (fp32, or the fp16 bits when S is
// uint16_t) and u8 zero points.  The tile's rows of the [N x groups] fp16
// tables are one contiguous run of 128 * groups halves; when groups % 8 == 0
// (<= 32), every column is in range and the tables are 16-byte aligned, it is
// read with 16-byte loads, all issued before the first LDS write (one load
// latency instead of one per element the threads loop over).
template <typename S, int kT = kThreads>
__device__ __forceinline__ void load_group_tables(const GemmArgs& p, int n0, int groups, S* tab_s, uint8_t* tab_z, int tid) {
    const bool vec = (groups & 7) == 0 && n0 + kBN <= p.n &&
                     ((((uintptr_t)p.g_scales) | ((uintptr_t)p.g_zeros)) & 15) == 0;
    if (vec) {
        const int chunks = kBN * groups / 8;  // <= 512 for groups <= 32
        const uint4* gs = (const uint4*)(p.g_scales + (size_t)n0 * groups);
        const uint4* gz = (const uint4*)(p.g_zeros + (size_t)n0 * groups);
        uint4 vs[2], vz[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kT;
            vs[i] = c < chunks ? gs[c] : uint4{0, 0, 0, 0};
            vz[i] = c < chunks ? gz[c] : uint4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kT;
            if (c >= chunks) continue;
            const int e = c * 8, col = e / groups, grp = e % groups;
            const uint32_t sw[4] = {vs[i].x, vs[i].y, vs[i].z, vs[i].w};
            const uint32_t zw[4] = {vz[i].x, vz[i].y, vz[i].z, vz[i].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint16_t sh = (uint16_t)(sw[j >> 1] >> ((j & 1) * 16));
                const uint16_t zh = (uint16_t)(zw[j >> 1] >> ((j & 1) * 16));
                if constexpr (sizeof(S) == 4) tab_s[(grp + j) * kBN + col] = h2f(sh);
                else tab_s[(grp + j) * kBN + col] = sh;
                tab_z[(grp + j) * kBN + col] = (uint8_t)(int)h2f(zh);
            }
        }
        return;
    }
    for (int e = tid; e < kBN * groups; e += kT) {
        const int col = e % kBN, grp = e / kBN;
        const size_t gi = (size_t)min(n0 + col, p.n - 1) * groups + grp;
        if constexpr (sizeof(S) == 4) tab_s[grp * kBN + col] = h2f(p.g_scales[gi]);
        else tab_s[grp * kBN + col] = p.g_scales[gi];
        tab_z[grp * kBN + col] = (uint8_t)(int)h2f(p.g_zeros[gi]);
    }
}

// Loads issued from inline asm are invisible to the compiler's wait
// insertion: the code waits for them with an explicit s_waitcnt and then
// passes the destinations through an empty asm (launder), so that no use is
// scheduled before the wait.
__device__ __forceinline__ uint4 asm_load4(const void* ptr) {
    v4i r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(ptr) : "memory");
    return __builtin_bit_cast(uint4, r);
}
__device__ __forceinline__ uint32_t asm_load1(const void* ptr) {
    uint32_t r;
    asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(ptr) : "memory");
    return r;
}
// A 16-byte global store issued from inline asm: the deferred epilogue below
// waits for the next tile's loads with vmcnt(its store count), which is exact
// only if every store it makes is one instruction the compiler cannot split,
// merge, predicate away or move past that wait.  A store of more than 8 bytes
// reads its data registers after issue: on this GPU a VALU write to them
// needs two wait states after the store (one was measured not to suffice:
// the compiler reused a store's data registers for the next address).  The
// compiler inserts them for the stores it can see, not for inline asm, hence
// the s_nop 1.
__device__ __forceinline__ void asm_store4(void* ptr, uint4 v) {
    const v4i x = __builtin_bit_cast(v4i, v);
    asm volatile("global_store_dwordx4 %0, %1, off\n\ts_nop 1" ::"v"(ptr), "v"(x) : "memory");
}
__device__ __forceinline__ uint32_t launder(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ uint4 launder(uint4 x) {
    v4i y = __builtin_bit_cast(v4i, x);
    asm volatile("" : "+v"(y));
    return __builtin_bit_cast(uint4, y);
}

// Epilogue whose scale loads are issued (as inline asm, invisible to the
// compiler's wait insertion) before `issue` (the next tile's first direct-to-
// LDS loads, kIssue per wave), then waited for with vmcnt(kIssue): the wait
// never covers the next tile's loads.  Non-residual epilogues only.
template <int F, int E, int kAI, int kIssue, typename Issue>
__device__ __forceinline__ void epilogue_defer(const GemmArgs& p, v4f (&accf)[kAI][4], v4i (&acci)[kAI][4], int m0, int n0, int wm,
                                               int wn, int lane, bool has_next, Issue&& issue) {
    using T = FmtTraits<F>;
    const int g = lane >> 4, l16 = lane & 15;
    const int gcol = n0 + wn * 64 + g * 16;
    const int ccol = min(gcol, p.n - 16);
    const bool col_live = gcol < p.n;
    const float* wsp = p.w_scales ? p.w_scales + ccol : (const float*)p.a;
    const float* bp = p.bias ? p.bias + ccol : wsp;
    uint4 wq[4], bq[4];
    uint32_t rq[kAI];
#pragma unroll
    for (int j = 0; j < 4; ++j) wq[j] = asm_load4(wsp + 4 * j);
#pragma unroll
    for (int j = 0; j < 4; ++j) bq[j] = asm_load4(bp + 4 * j);
#pragma unroll
    for (int ai = 0; ai < kAI; ++ai) {
        const int row = min(m0 + wm * 16 * kAI + ai * 16 + l16, p.m - 1);
        const float* rp = p.row_scales ? p.row_scales + row : (const float*)p.a;
        rq[ai] = asm_load1(rp);
    }
    if (has_next) {
        issue();
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kIssue) : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    // the loads above have landed: pass every destination through an empty
    // asm so that no use can be scheduled before the wait
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wq[j] = launder(wq[j]);
        bq[j] = launder(bq[j]);
    }
#pragma unroll
    for (int ai = 0; ai < kAI; ++ai) rq[ai] = launder(rq[ai]);
    float wsv[16], bsv[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 w4 = __builtin_bit_cast(float4, wq[j]);
        const float4 b4 = __builtin_bit_cast(float4, bq[j]);
        wsv[4 * j] = p.w_scales ? w4.x : 1.f; wsv[4 * j + 1] = p.w_scales ? w4.y : 1.f;
        wsv[4 * j + 2] = p.w_scales ? w4.z : 1.f; wsv[4 * j + 3] = p.w_scales ? w4.w : 1.f;
        bsv[4 * j] = p.bias ? b4.x : 0.f; bsv[4 * j + 1] = p.bias ? b4.y : 0.f;
        bsv[4 * j + 2] = p.bias ? b4.z : 0.f; bsv[4 * j + 3] = p.bias ? b4.w : 0.f;
    }
#pragma unroll
    for (int ai = 0; ai < kAI; ++ai) {
        const int grow = m0 + wm * 16 * kAI + ai * 16 + l16;
        const bool live = grow < p.m && col_live;
        const float rs = p.row_scales ? __builtin_bit_cast(float, rq[ai]) : p.in_scale;
        float v[16];
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[bj * 4 + r] = T::kInt ? (float)acci[ai][bj][r] : accf[ai][bj][r];
        if (p.fused_scale) {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j], rs * wsv[j], bsv[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(v[j] * rs, wsv[j], bsv[j]);
        }
        if constexpr (E == EPI_F32) {
            if (live) {
                float* o = (float*)p.out + (size_t)grow * p.ldo + gcol;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    asm_store4(o + 4 * j, __builtin_bit_cast(uint4, float4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]}));
            }
        } else if constexpr (E == EPI_F16) {
            uint32_t h[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float x0 = v[2 * j] * p.out_scale, x1 = v[2 * j + 1] * p.out_scale;
                x0 = p.act == 1 ? silu(x0) : (p.act == 2 ? __builtin_fmaxf(x0, 0.0f) : x0);
                x1 = p.act == 1 ? silu(x1) : (p.act == 2 ? __builtin_fmaxf(x1, 0.0f) : x1);
                h[j] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
            }
            if (live) {
                uint16_t* o = (uint16_t*)p.out + (size_t)grow * p.ldo + gcol;
                asm_store4(o, uint4{h[0], h[1], h[2], h[3]});
                asm_store4(o + 8, uint4{h[4], h[5], h[6], h[7]});
            }
        } else {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = silu_fp8x4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            if (live) *(uint4*)((uint8_t*)p.out + (size_t)grow * p.ldo + gcol) = uint4{w[0], w[1], w[2], w[3]};
        }
    }
}



// Tile rows: 32 * kAI (kAI = 16-row MFMA blocks per wave: 8 for 256-row tiles,
// 4 for 128-row tiles, which double the tile count of small grids).  Weight
// tile bytes of one step, and the LDS of one workgroup: two activation tiles,
// one weight tile and (G128 formats) a 2-entry ring of the step's group scales
// (fp32) and zero-points (u8) for the tile's 128 columns.
template <int F, int kAI> struct L3 {
    static constexpr int kBM = 32 * kAI;
    static constexpr int kATile = kBM * kRowBytes;
    static constexpr int kB = 2 * kATile;  // weight buffer offset
    static constexpr bool kG128 = (F == FMT_G128A8 || F == FMT_G128A16);
    static constexpr int kBTile = kBN * FmtTraits<F>::bRow;
    static constexpr int kTab = kB + kBTile;
    static constexpr int kBytes = kTab + (kG128 ? 2 * kBN * 5 : 0);
    static constexpr int kBLoads = kBTile / 1024;  // direct-to-LDS weight loads per step
    static constexpr int kBPerWave = (kBLoads + 3) / 4;
};

template <int F, int E, int kAI>
__global__ __launch_bounds__(kThreads, 2) void gemm3_kernel(GemmArgs p) {
    using T = FmtTraits<F>;
    using L = L3<F, kAI>;
    constexpr int kBM = L::kBM, kATile = L::kATile, kB = L::kB;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBN - 1) / kBN;
    const int tiles_m = (p.m + kBM - 1) / kBM;
    const int ntiles = tiles_m * tiles_n;
    const int G = gridDim.x;
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;  // bytes per activation row
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;          // bytes per weight row
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    const uint8_t* __restrict__ pa = p.a;
    const uint8_t* __restrict__ pb = p.b;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const int gw = group_width(tiles_n);
    float* tab_s = (float*)(lds + L::kTab);                  // [2][128] group scales
    uint8_t* tab_z = lds + L::kTab + 2 * kBN * 4;            // [2][128] zero-points

    // Activation load i of this wave covers tile rows wave*8kAI + 8i + q,
    // q = lane / 8, 16-byte chunk position lane % 8.  swz_key of that row is
    // kq(q) ^ ki((wave*kAI + i) & 7), so a lane keeps only its first row and
    // (lane % 8) ^ kq.
    const int q = lane >> 3;
    const uint32_t a_cq = (uint32_t)((lane & 7) ^ ((q >> 1) & 1) ^ (((q >> 2) & 1) << 1) ^ ((q & 1) << 2));
    int a_row = 0;  // m0 + wave*64 + q of the issue tile
    // FP8 / INT8 read activation fragments two row blocks ahead (three in
    // registers), the others one ahead; the formats with registers to spare
    // keep the 8 load offsets instead of deriving them at issue time.
    constexpr bool kAhead2 = F == FMT_FP8 || F == FMT_I8 || F == FMT_S4F6;
    constexpr bool kPreOff = F == FMT_I8_SKIP || F == FMT_F16;
    uint32_t a_off[kPreOff ? kAI : 1];
    uint32_t b_off[L::kBPerWave];
    uint32_t b_q4k = 0;  // Q4K: bit i set when weight load i carries quant bytes
    auto tile_origin = [&](int tt, int& m0, int& n0) {
        const int ng = tt / (tiles_m * gw);
        const int r = tt - ng * tiles_m * gw;
        const int tm = r / gw;
        m0 = tm * kBM;
        n0 = (ng * gw + (r - tm * gw)) * kBN;
    };
    auto set_tile = [&](int tt, int& m0, int& n0) {
        tile_origin(tt, m0, n0);
        a_row = m0 + wave * 8 * kAI + q;
        if constexpr (kPreOff) {
#pragma unroll
            for (int i = 0; i < kAI; ++i) {
                const int x = (wave * kAI + i) & 7;
                const uint32_t ki = (uint32_t)((((x >> 1) & 1) << 1) | (((x ^ (x >> 2)) & 1) << 2));
                a_off[i] = (uint32_t)min(a_row + 8 * i, p.m - 1) * (uint32_t)lda + ((a_cq ^ ki) << 4);
            }
        }
#pragma unroll
        for (int i = 0; i < L::kBPerWave; ++i) {
            const int o = (i * 4 + wave) * 1024 + lane * 16;
            int row, c;
            if constexpr (T::bRow == 128) {
                row = o >> 7;
                c = ((o >> 4) & 7) ^ swz_key(row);
            } else if constexpr (F == FMT_G128A8) {
                row = o >> 6;
                c = ((o >> 4) & 3) ^ g128a8_key(row);
            } else if constexpr (F == FMT_G128A16) {
                a16_chunk_of_slot(o >> 4, row, c);
            } else {
                row = o / T::bRow;
                c = (o % T::bRow) / 16;
            }
            b_off[i] = (uint32_t)min(n0 + row, p.n - 1) * (uint32_t)ldb + (uint32_t)(c * 16);
            if constexpr (F == FMT_Q4K) b_q4k = c > 0 ? b_q4k | (1u << i) : b_q4k & ~(1u << i);
        }
    };
    auto issue_a = [&](int step, int buf) {
        const uint32_t base = lds_base + buf * kATile;
#pragma unroll
        for (int i = 0; i < kAI; ++i) {
            uint32_t off;
            if constexpr (kPreOff) {
                off = a_off[i];
            } else {
                const int x = (wave * kAI + i) & 7;
                const uint32_t ki = (uint32_t)((((x >> 1) & 1) << 1) | (((x ^ (x >> 2)) & 1) << 2));
                off = (uint32_t)min(a_row + 8 * i, p.m - 1) * (uint32_t)lda + ((a_cq ^ ki) << 4);
            }
            dma16(pa + (size_t)step * kRowBytes, off, base + (wave * kAI + i) * 1024);
        }
    };
    auto issue_b = [&](int step) {
#pragma unroll
        for (int i = 0; i < L::kBPerWave; ++i) {
            if (L::kBLoads % 4 != 0 && i * 4 + wave >= L::kBLoads) continue;
            const uint32_t dst = lds_base + kB + (i * 4 + wave) * 1024;
            if constexpr (F == FMT_Q4K) {
                // superblock step >> 2; quant chunks advance 32 bytes per step
                const uint32_t qa = (b_q4k >> i) & 1u ? (uint32_t)(step & 3) * 32u : 0u;
                dma16(pb + (size_t)(step >> 2) * 144, b_off[i] + qa, dst);
            } else {
                dma16(pb + (size_t)step * T::bRow, b_off[i], dst);
            }
        }
    };
    // G128: the scale and zero-point of a step's 128-K group for the tile's
    // columns are fetched two steps ahead (a cursor over this workgroup's
    // (tile, step) sequence) and written into table slot `step & 1` at the
    // step before their use.
    float tv_s = 0.0f;
    uint32_t tv_z = 0;
    int f_t = 0, f_step = 0, f_n0 = 0;
    auto fetch_tab = [&]() {
        if constexpr (L::kG128) {
            if (tid < kBN && f_t < ntiles) {
                const size_t gi = (size_t)min(f_n0 + tid, p.n - 1) * groups + ((f_step * T::kStep) >> 7);
                tv_s = h2f(p.g_scales[gi]);
                tv_z = (uint32_t)(int)h2f(p.g_zeros[gi]);
            }
            if (++f_step == steps) {
                f_step = 0;
                f_t += G;
                int fm0;
                if (f_t < ntiles) tile_origin(f_t, fm0, f_n0);
            }
        }
    };
    auto store_tab = [&](int step) {
        if constexpr (L::kG128) {
            if (tid < kBN) {
                tab_s[(step & 1) * kBN + tid] = tv_s;
                tab_z[(step & 1) * kBN + tid] = (uint8_t)tv_z;
            }
        }
    };

    // G128F8 keeps no LDS table (its 80 KiB of tiles leave no room at two
    // workgroups per CU): its scales are group-major ([K/128][N] fp16), so a
    // lane's 16 accumulator columns n0 + 64 wn + 16 g .. + 15 of a step's
    // group are 32 contiguous bytes, loaded a step ahead (sc_nxt) with two
    // 16-byte loads.  N % 16 == 0 (checked by the host): a 16-column run is in
    // range or wholly past N, then read from the last run and unused.
    uint4 sc_cur[2] = {}, sc_nxt[2] = {};
    auto load_sc = [&](int cn0, int st) {
        const int col = min(cn0 + wn * 64 + g * 16, p.n - 16);
        const uint4* src = (const uint4*)(p.g_scales + (size_t)st * p.n + col);
        sc_nxt[0] = src[0];
        sc_nxt[1] = src[1];
    };

    int t = tile_slot(G);
    if (t >= ntiles) return;
    int m0, n0;
    set_tile(t, m0, n0);
    if constexpr (F == FMT_G128F8) load_sc(n0, 0);
    issue_a(0, 0);
    issue_b(0);
    if constexpr (L::kG128) {
        f_t = t;
        f_n0 = n0;
        fetch_tab();  // step 0
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        store_tab(0);
        fetch_tab();  // the second step
    }
    int buf = 0;
    // fp16 / fp32 epilogues without a residual (FP8, INT8): the next tile's
    // first loads are issued inside the epilogue, after its scale loads, so
    // that its wait for the scales does not also wait for them; the first
    // step of the next tile then waits for them with vmcnt(stores issued
    // since), not for the epilogue's stores (QKV at T = 45000: 174 -> 162 us).
    constexpr bool kDefer = kAhead2 && (E == EPI_F16 || E == EPI_F32);
    // stores of one deferred epilogue: asm_store4 instructions, 2 (fp16) or 4
    // (fp32) per row block of a wave, every one issued when the tile is full
    constexpr int kStores = kAI * (E == EPI_F16 ? 2 : 4);
    bool prev_full = false;  // the last epilogue issued all kStores stores

    v4f accf[kAI][4];
    v4i acci[kAI][4];
    uint32_t skipped = 0, blocks = 0;

    while (true) {
        const int t_next = t + G;
        const int cur_m0 = m0, cur_n0 = n0;
#pragma unroll
        for (int i = 0; i < kAI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                accf[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
                acci[i][j] = v4i{0, 0, 0, 0};
            }

        // The two workgroups of a CU alternate between K-loop and epilogue.
        // Wave priorities order their instruction issue: highest (3) from a
        // K-step's first barrier to its second (waits, loads, fragment reads:
        // the step's latency chain), 1 during its MFMA burst, 0 in the
        // epilogue, so that the other workgroup's VALU-heavy epilogue fills
        // the gaps instead of delaying the K-loop (stack at T = 45000: 3 %
        // faster than without priorities).
        for (int step = 0; step < steps; ++step) {
            __builtin_amdgcn_s_setprio(3);
            if (kDefer && step == 0 && prev_full) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStores) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            // The next step's (or next tile's first step's) activations load
            // into the other buffer, which every wave finished with last step.
            int nstep = -1;
            if (step + 1 < steps) nstep = step + 1;
            else if (t_next < ntiles && !kDefer) {
                set_tile(t_next, m0, n0);
                nstep = 0;
            }
            if constexpr (F == FMT_G128F8) {
                sc_cur[0] = sc_nxt[0];
                sc_cur[1] = sc_nxt[1];
                if (nstep >= 0) load_sc(n0, nstep);
            }
            if (nstep >= 0) issue_a(nstep, buf ^ 1);
            const uint8_t* As = lds + buf * kATile;
            const uint8_t* Bs = lds + kB;
            uint4 w0[4], w1[4];
            v4f gs[4];
#pragma unroll
            for (int bj = 0; bj < 4; ++bj)
                weight_frag<F>(Bs, wn * 64 + wrow(l16, bj), g, bj, wn, step, tab_s + (step & 1) * kBN, tab_z + (step & 1) * kBN,
                               w0[bj], w1[bj], gs[bj]);
            if constexpr (F == FMT_G128F8) {
                const uint32_t sw[8] = {sc_cur[0].x, sc_cur[0].y, sc_cur[0].z, sc_cur[0].w,
                                        sc_cur[1].x, sc_cur[1].y, sc_cur[1].z, sc_cur[1].w};
#pragma unroll
                for (int bj = 0; bj < 4; ++bj)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        gs[bj][r] = h2f((uint16_t)(sw[(4 * bj + r) >> 1] >> (((4 * bj + r) & 1) * 16)));
            }
            uint4 x0, x1, y0, y1;
            uint4 xr0[3], xr1[3];  // kAhead2: row blocks ai, ai + 1, ai + 2 in slots ai % 3 ...
            if constexpr (kAhead2) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int row = wm * 16 * kAI + i * 16 + l16;
                    xr0[i] = *(const uint4*)(As + swz(row, g));
                    xr1[i] = *(const uint4*)(As + swz(row, 4 + g));
                }
            } else {
                const int row = wm * 16 * kAI + l16;
                x0 = *(const uint4*)(As + swz(row, g));
                x1 = *(const uint4*)(As + swz(row, 4 + g));
            }
            // every wave holds its weight fragments: the weight buffer (and the
            // group table slot of the step before) are free
            __syncthreads();
            __builtin_amdgcn_s_setprio(1);
            if (nstep >= 0) {
                issue_b(nstep);
                store_tab(nstep);  // fetched a step ago
                fetch_tab();       // for the step after nstep
            }
            if constexpr (F == FMT_G128A8) {
                // Software-pipelined over the wave's 4 kAI blocks (row block ai,
                // column block bj): block b's exact int32 group sum goes to one
                // of three rotating registers while block b - 2's is converted
                // and scaled, so the MFMAs overlap the VALU work instead of
                // waiting on it (and the next block's MFMAs on the register).
                v4i gi[3];
#pragma unroll
                for (int b = 0; b < 4 * kAI + 2; ++b) {
                    const int ai = b >> 2, bj = b & 3;
                    if (b < 4 * kAI) {
                        if (bj == 0 && ai + 1 < kAI) {
                            const int row = wm * 16 * kAI + (ai + 1) * 16 + l16;
                            y0 = *(const uint4*)(As + swz(row, g));
                            y1 = *(const uint4*)(As + swz(row, 4 + g));
                        }
                        gi[b % 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w0[bj]), as_v4i(x0), v4i{0, 0, 0, 0}, 0, 0, 0);
                        gi[b % 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(w1[bj]), as_v4i(x1), gi[b % 3], 0, 0, 0);
                        if (bj == 3) {
                            x0 = y0;
                            x1 = y1;
                        }
                    }
                    if (b >= 2) {
                        const int pa = (b - 2) >> 2, pj = (b - 2) & 3;
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            accf[pa][pj][r] = __builtin_fmaf((float)gi[(b - 2) % 3][r], gs[pj][r], accf[pa][pj][r]);
                    }
                }
                // Issue order per block: its activation reads (every fourth
                // block), its two MFMAs, then the eight conversions / FMAs of
                // block b - 2, so the VALU work interleaves with the MFMAs
                // (INT4-g128 x INT8 linears at T = 45000: 4-7 % faster; the
                // residual variant, short of registers, ran 5-7 % slower with it).
                if constexpr (E != EPI_F16_RES)
#pragma unroll
                for (int b = 0; b < 4 * kAI + 2; ++b) {
                    if (b < 4 * kAI) {
                        if ((b & 3) == 0 && (b >> 2) + 1 < kAI) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    }
                    if (b >= 2) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                }
            } else if constexpr (F == FMT_G128F8) {
                // One MFMA per block and 128-K group: its fp32 group sum goes
                // to one of two rotating registers while block b - 1's is
                // scaled into the accumulators (one fma per value).  Issue
                // order left to the compiler: at a distance of one block and
                // without sched_group_barrier pinning the contract runs
                // 255.6 us against 279.5 us at a distance of two with the
                // MFMA / VALU interleave pinned (T = 45000, N = 1024, K = 4096).
                v4f gf[2];
#pragma unroll
                for (int b = 0; b < 4 * kAI + 1; ++b) {
                    const int ai = b >> 2, bj = b & 3;
                    if (b < 4 * kAI) {
                        if (bj == 0 && ai + 1 < kAI) {
                            const int row = wm * 16 * kAI + (ai + 1) * 16 + l16;
                            y0 = *(const uint4*)(As + swz(row, g));
                            y1 = *(const uint4*)(As + swz(row, 4 + g));
                        }
                        const v8i W = {(int)w0[bj].x, (int)w0[bj].y, (int)w0[bj].z, (int)w0[bj].w,
                                       (int)w1[bj].x, (int)w1[bj].y, (int)w1[bj].z, (int)w1[bj].w};
                        const v8i X = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
                        gf[b & 1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(W, X, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
                        if (bj == 3) {
                            x0 = y0;
                            x1 = y1;
                        }
                    }
                    if (b >= 1) {
                        const int pa = (b - 1) >> 2, pj = (b - 1) & 3;
#pragma unroll
                        for (int r = 0; r < 4; ++r) accf[pa][pj][r] = __builtin_fmaf(gf[(b - 1) & 1][r], gs[pj][r], accf[pa][pj][r]);
                    }
                }
            } else if constexpr (kAhead2) {
#pragma unroll
                for (int ai = 0; ai < kAI; ++ai) {
                    if (ai + 2 < kAI) {
                        const int row = wm * 16 * kAI + (ai + 2) * 16 + l16;
                        xr0[(ai + 2) % 3] = *(const uint4*)(As + swz(row, g));
                        xr1[(ai + 2) % 3] = *(const uint4*)(As + swz(row, 4 + g));
                    }
#pragma unroll
                    for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[ai][bj], acci[ai][bj], w0[bj], w1[bj], xr0[ai % 3], xr1[ai % 3], gs[bj]);
                }
                constexpr int kMfma = F == FMT_I8 ? 8 : 4;
#pragma unroll
                for (int ai = 0; ai < kAI; ++ai) {
                    if (ai + 2 < kAI) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
                }
            } else
#pragma unroll
            for (int ai = 0; ai < kAI; ++ai) {
                if (ai + 1 < kAI) {
                    const int row = wm * 16 * kAI + (ai + 1) * 16 + l16;
                    y0 = *(const uint4*)(As + swz(row, g));
                    y1 = *(const uint4*)(As + swz(row, 4 + g));
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
                x0 = y0;
                x1 = y1;
            }
            buf ^= 1;
        }
        blocks += kAI * steps;
        __builtin_amdgcn_s_setprio(0);

        if constexpr (E == EPI_F16_RES) {
            epilogue<F, EPI_F16, true, kAI>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
        } else if constexpr (kDefer) {
            const bool has_next = t_next < ntiles;
            if (has_next) set_tile(t_next, m0, n0);
            static_assert(L::kBLoads % 4 == 0, "every wave issues the same number of weight loads");
            epilogue_defer<F, E, kAI, kAI + L::kBPerWave>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane, has_next, [&] {
                issue_a(0, buf);
                issue_b(0);
            });
            prev_full = cur_m0 + kBM <= p.m && cur_n0 + kBN <= p.n;
        } else {
            epilogue<F, E, false, kAI>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
        }
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


// ---- small grids: one tile per workgroup, an S-stage ring -----------------
//
// When a launch has no more tiles than CUs (INT4-g128 at
// T = 750), every workgroup computes exactly one tile and the K-loop is the
// whole latency chain: with the engine's one-step prefetch each K-step waits
// for a memory round trip.  This variant gives the one workgroup of a CU an
// S-stage LDS ring of (activation + weight) stages, so that a stage's loads
// have S - 1 steps to land, and one barrier per step: at step s the wave
// waits for stage s (vmcnt counts only the younger stages), the barrier
// makes it visible and frees the slot of step s - 1, stage s + S - 1 starts
// loading into that slot, and the fragments of stage s are read and
// multiplied.  The INT4-g128 group tables of the tile's columns (all K groups)
// are loaded once into [group][column] fp32 scales and u8 zero points and
// indexed by the step's group.  Arithmetic, fragment layouts and
// epilogues are those of gemm3_kernel, so results are identical.  kOcc = 2
// sizes the ring for two workgroups per CU (80 KiB each) instead of one.
template <int F, int kAI, int kOcc = 1> struct LS {
    static constexpr int kBM = 32 * kAI;
    static constexpr int kATile = kBM * kRowBytes;
    static constexpr int kBTile = kBN * FmtTraits<F>::bRow;
    static constexpr int kStageBytes = kATile + kBTile;
    static constexpr bool kG128 = (F == FMT_G128A8 || F == FMT_G128A16);
    static constexpr int kTabBytes = kG128 ? kMaxG128Groups * kBN * 5 : 0;   // fp32 scales + u8 zeros [group][column]
    static constexpr int kFit = ((kOcc == 1 ? 150 : 80) * 1024 - kTabBytes) / kStageBytes;
    static constexpr int kS = kFit > 8 ? 8 : kFit;
    static constexpr int kTab = kS * kStageBytes;
    static constexpr int kBytes = kTab + kTabBytes;
    static constexpr int kBLoads = kBTile / 1024;
    static constexpr int kBPerWave = kBLoads / 4;
    static constexpr int kOps = kAI + kBPerWave;  // direct-to-LDS loads per wave and stage
    static_assert(kBLoads % 4 == 0 && kS >= 3 && kBytes <= 160 * 1024, "ring layout");
};

template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// vmcnt(kOps * younger) for a runtime count of younger stages (0 .. 7).
template <int kOps> __device__ __forceinline__ void wait_stages(int younger) {
    switch (younger) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<kOps>(); break;
    case 2: wait_vm<2 * kOps>(); break;
    case 3: wait_vm<3 * kOps>(); break;
    case 4: wait_vm<4 * kOps>(); break;
    case 5: wait_vm<5 * kOps>(); break;
    case 6: wait_vm<6 * kOps>(); break;
    default: wait_vm<7 * kOps>(); break;
    }
}

template <int F, int E, int kAI, int kOcc = 1>
__global__ __launch_bounds__(kThreads, kOcc) void gemm3_ring_kernel(GemmArgs p) {
    using T = FmtTraits<F>;
    using L = LS<F, kAI, kOcc>;
    constexpr int kS = L::kS, kBM = L::kBM;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBN - 1) / kBN;
    const int tiles_m = (p.m + kBM - 1) / kBM;
    const int tile = blockIdx.x;
    if (tile >= tiles_m * tiles_n) return;
    // tiles of one column strip are consecutive blocks, which the dispatcher
    // deals out over the 8 XCDs; placing each strip on one XCD (its weights
    // fetched into one L2) measured slower (C1: 13.2 -> 14.6 us)
    const int m0 = (tile % tiles_m) * kBM, n0 = (tile / tiles_m) * kBN;
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    float* tab_s = (float*)(lds + L::kTab);
    uint8_t* tab_z = lds + L::kTab + kMaxG128Groups * kBN * 4;

    const int q = lane >> 3;
    const uint32_t a_cq = (uint32_t)((lane & 7) ^ ((q >> 1) & 1) ^ (((q >> 2) & 1) << 1) ^ ((q & 1) << 2));
    const int a_row = m0 + wave * 8 * kAI + q;
    uint32_t a_off[kAI], b_off[L::kBPerWave];
#pragma unroll
    for (int i = 0; i < kAI; ++i) {
        const int x = (wave * kAI + i) & 7;
        const uint32_t ki = (uint32_t)((((x >> 1) & 1) << 1) | (((x ^ (x >> 2)) & 1) << 2));
        a_off[i] = (uint32_t)min(a_row + 8 * i, p.m - 1) * (uint32_t)lda + ((a_cq ^ ki) << 4);
    }
#pragma unroll
    for (int i = 0; i < L::kBPerWave; ++i) {
        const int o = (i * 4 + wave) * 1024 + lane * 16;
        int row, c;
        if constexpr (T::bRow == 128) {
            row = o >> 7;
            c = ((o >> 4) & 7) ^ swz_key(row);
        } else if constexpr (F == FMT_G128A8) {
            row = o >> 6;
            c = ((o >> 4) & 3) ^ g128a8_key(row);
        } else if constexpr (F == FMT_G128A16) {
            a16_chunk_of_slot(o >> 4, row, c);
        } else {
            row = o / T::bRow;
            c = (o % T::bRow) / 16;
        }
        b_off[i] = (uint32_t)min(n0 + row, p.n - 1) * (uint32_t)ldb + (uint32_t)(c * 16);
    }
    auto issue = [&](int step) {
        const uint32_t sbase = lds_base + (uint32_t)((step % kS) * L::kStageBytes);
#pragma unroll
        for (int i = 0; i < kAI; ++i) dma16(p.a + (size_t)step * kRowBytes, a_off[i], sbase + (wave * kAI + i) * 1024);
#pragma unroll
        for (int i = 0; i < L::kBPerWave; ++i)
            dma16(p.b + (size_t)step * T::bRow, b_off[i], sbase + L::kATile + (i * 4 + wave) * 1024);
    };

    const int pre = min(kS - 1, steps);
    for (int s = 0; s < pre; ++s) issue(s);
    // Group tables of the tile's columns, all K groups, loaded after the
    // first stages (whose latency they share): [group][column] fp32 scales
    // and u8 zero points.
    if constexpr (L::kG128) load_group_tables(p, n0, groups, tab_s, tab_z, tid);

    v4f accf[kAI][4];
    v4i acci[kAI][4];
#pragma unroll
    for (int i = 0; i < kAI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            accf[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
            acci[i][j] = v4i{0, 0, 0, 0};
        }

    for (int step = 0; step < steps; ++step) {
        wait_stages<L::kOps>(min(step + kS - 2, steps - 1) - step);
        __syncthreads();
        if (step + kS - 1 < steps) issue(step + kS - 1);
        const uint8_t* As = lds + (step % kS) * L::kStageBytes;
        const uint8_t* Bs = As + L::kATile;
        const int grp = (step * T::kStep) >> 7;
        uint4 w0[4], w1[4];
        v4f gs[4];
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            weight_frag<F>(Bs, wn * 64 + wrow(l16, bj), g, bj, wn, step, tab_s + grp * kBN, tab_z + grp * kBN, w0[bj], w1[bj], gs[bj]);
        uint4 xr0[3], xr1[3];
#pragma unroll
        for (int i = 0; i < 2 && i < kAI; ++i) {
            const int row = wm * 16 * kAI + i * 16 + l16;
            xr0[i] = *(const uint4*)(As + swz(row, g));
            xr1[i] = *(const uint4*)(As + swz(row, 4 + g));
        }
#pragma unroll
        for (int ai = 0; ai < kAI; ++ai) {
            if (ai + 2 < kAI) {
                const int row = wm * 16 * kAI + (ai + 2) * 16 + l16;
                xr0[(ai + 2) % 3] = *(const uint4*)(As + swz(row, g));
                xr1[(ai + 2) % 3] = *(const uint4*)(As + swz(row, 4 + g));
            }
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[ai][bj], acci[ai][bj], w0[bj], w1[bj], xr0[ai % 3], xr1[ai % 3], gs[bj]);
        }
    }
    if constexpr (E == EPI_F16_RES) {
        epilogue<F, EPI_F16, true, kAI>(p, accf, acci, m0, n0, wm, wn, lane);
    } else if constexpr (E == EPI_F32) {
        __syncthreads();  // every wave is done with the ring: 4 KiB of it per wave stage the output rows
        epilogue<F, E, false, kAI>(p, accf, acci, m0, n0, wm, wn, lane, lds + wave * 4096);
    } else {
        epilogue<F, E, false, kAI>(p, accf, acci, m0, n0, wm, wn, lane);
    }
}


// ---- small grids, long K: one 32 x 128 tile per workgroup, K split over its 4 waves ----
//
// The ring kernel with two waves per SIMD: waves w and w + 4 share quadrant
// w % 4 of the tile (its 64 columns and 16 kAI rows) and take its first
// ceil(kAI / 2) / remaining row blocks, so each SIMD runs two independent
// fragment-read / decode / MFMA chains of a K-step.  A stage's direct-to-LDS
// loads (4 kAI activation row groups, then the weight chunks, L in all, a
// multiple of 8) are dealt out as load j to wave j % 8.  Stages, swizzles,
// group tables and epilogue as gemm3_ring_kernel.
template <int F> constexpr int ring8_loads(int kAI) { return 4 * kAI + LS<F, 1, 1>::kBLoads; }
template <int F, int E, int kAI>
__global__ __launch_bounds__(2 * kThreads, 1) void gemm3_ring8_kernel(GemmArgs p) {
    using T = FmtTraits<F>;
    using L = LS<F, kAI, 1>;
    constexpr int kS = L::kS, kBM = L::kBM;
    constexpr int kH0 = (kAI + 1) / 2, kH1 = kAI - kH0;  // row blocks of the first / second wave of a quadrant
    constexpr int kL = ring8_loads<F>(kAI), kOps = kL / 8;
    static_assert(kH1 >= 1 && kL % 8 == 0 && kOps <= 4, "8-wave ring layout");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qd = wave & 3, half = wave >> 2;
    const int wm = qd >> 1, wn = qd & 1;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBN - 1) / kBN;
    const int tiles_m = (p.m + kBM - 1) / kBM;
    const int tile = blockIdx.x;
    if (tile >= tiles_m * tiles_n) return;
    const int m0 = (tile % tiles_m) * kBM, n0 = (tile / tiles_m) * kBN;
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    float* tab_s = (float*)(lds + L::kTab);
    uint8_t* tab_z = lds + L::kTab + kMaxG128Groups * kBN * 4;

    // load slot i of this wave: j = wave + 8 i; activation row group j (rows
    // 8 j + q) for j < 4 kAI, else weight chunk j - 4 kAI
    const int q = lane >> 3;
    const uint32_t a_cq = (uint32_t)((lane & 7) ^ ((q >> 1) & 1) ^ (((q >> 2) & 1) << 1) ^ ((q & 1) << 2));
    uint32_t off[kOps], dst[kOps];
#pragma unroll
    for (int i = 0; i < kOps; ++i) {
        const int j = wave + 8 * i;
        if (j < 4 * kAI) {
            const int xs = j & 7;
            const uint32_t ki = (uint32_t)((((xs >> 1) & 1) << 1) | (((xs ^ (xs >> 2)) & 1) << 2));
            off[i] = (uint32_t)min(m0 + 8 * j + q, p.m - 1) * (uint32_t)lda + ((a_cq ^ ki) << 4);
            dst[i] = (uint32_t)(j * 1024);
        } else {
            const int c = j - 4 * kAI;
            const int o = c * 1024 + lane * 16;
            int row, ch;
            if constexpr (T::bRow == 128) {
                row = o >> 7;
                ch = ((o >> 4) & 7) ^ swz_key(row);
            } else if constexpr (F == FMT_G128A8) {
                row = o >> 6;
                ch = ((o >> 4) & 3) ^ g128a8_key(row);
            } else {
                a16_chunk_of_slot(o >> 4, row, ch);
            }
            off[i] = (uint32_t)min(n0 + row, p.n - 1) * (uint32_t)ldb + (uint32_t)(ch * 16);
            dst[i] = (uint32_t)(L::kATile + c * 1024);
        }
    }
    auto issue = [&](int step) {
        const uint32_t sbase = lds_base + (uint32_t)((step % kS) * L::kStageBytes);
#pragma unroll
        for (int i = 0; i < kOps; ++i) {
            if (wave + 8 * i < 4 * kAI) dma16(p.a + (size_t)step * kRowBytes, off[i], sbase + dst[i]);
            else dma16(p.b + (size_t)step * T::bRow, off[i], sbase + dst[i]);
        }
    };

    const int pre = min(kS - 1, steps);
    for (int s = 0; s < pre; ++s) issue(s);
    if constexpr (L::kG128) load_group_tables<float, 2 * kThreads>(p, n0, groups, tab_s, tab_z, tid);

    v4f accf[kH0][4];
    v4i acci[kH0][4];
#pragma unroll
    for (int i = 0; i < kH0; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            accf[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
            acci[i][j] = v4i{0, 0, 0, 0};
        }
    const int nb = half ? kH1 : kH0;            // this wave's row blocks (wave-uniform)
    const int rb0 = wm * kAI + half * kH0;      // its first 16-row block of the tile
    for (int step = 0; step < steps; ++step) {
        wait_stages<kOps>(min(step + kS - 2, steps - 1) - step);
        __syncthreads();
        if (step + kS - 1 < steps) issue(step + kS - 1);
        const uint8_t* As = lds + (step % kS) * L::kStageBytes;
        const uint8_t* Bs = As + L::kATile;
        const int grp = (step * T::kStep) >> 7;
        uint4 w0[4], w1[4];
        v4f gs[4];
#pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            weight_frag<F>(Bs, wn * 64 + wrow(l16, bj), g, bj, wn, step, tab_s + grp * kBN, tab_z + grp * kBN, w0[bj], w1[bj], gs[bj]);
#pragma unroll
        for (int i = 0; i < kH0; ++i) {
            if (i < nb) {
                const int row = (rb0 + i) * 16 + l16;
                const uint4 x0 = *(const uint4*)(As + swz(row, g));
                const uint4 x1 = *(const uint4*)(As + swz(row, 4 + g));
#pragma unroll
                for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[i][bj], acci[i][bj], w0[bj], w1[bj], x0, x1, gs[bj]);
            }
        }
    }
    // rows of this wave: m0 + 16 rb0 + 16 a + l16 (a < nb), as the register
    // epilogue's wave 0 of a kH0-block tile at m0 + 16 rb0 whose rows end
    // after nb blocks (the accumulators past them hold zeros and are not stored)
    GemmArgs pe = p;
    pe.m = min(p.m, m0 + 16 * (rb0 + nb));
    if constexpr (E == EPI_F16_RES) {
        epilogue<F, EPI_F16, true, kH0>(pe, accf, acci, m0 + 16 * rb0, n0, 0, wn, lane);
    } else if constexpr (E == EPI_F32) {
        __syncthreads();  // every wave is done with the ring: 4 KiB of it per wave stage the output rows
        epilogue<F, E, false, kH0>(pe, accf, acci, m0 + 16 * rb0, n0, 0, wn, lane, lds + wave * 4096);
    } else {
        epilogue<F, E, false, kH0>(pe, accf, acci, m0 + 16 * rb0, n0, 0, wn, lane);
    }
}

// For the group-wise INT4 formats at small T (FF2 at T = 750: 192 tiles of
// 32 rows, K = 4096) the ring kernel above is a chain of K-steps whose every
// link is an LDS read, the INT4 decode and the MFMAs; the tile count cannot
// grow.  Here the workgroup has 4 kCH waves: K-part kp = wave % 4 takes a
// quarter of the K-steps through a private LDS ring, and the part's kCH
// waves (column slice ch = wave / 4) share that ring, each computing 32 rows
// x 128 / kCH columns (2 x 4 / (kCH / 2) blocks of 16 x 16) over it: kCH
// waves per SIMD hide each other's LDS and decode latency, and the chain is a
// quarter as long.  Each wave of a part issues its share of the stage's
// direct-to-LDS loads and waits for its own (vmcnt); one barrier per K-step
// makes the whole stage visible and frees the slot refilled after it.  The group tables of the tile's columns
// (fp16 scales, u8 zero points, all groups) are loaded once.  Then the four
// parts meet in LDS and wave q < 4 adds the partials of quarter q (rows
// 16 (q / 2), columns 64 (q % 2)) in K order, ((p0 + p1) + p2) + p3, and runs
// the ring kernel's epilogue of its wave q on them.  Within a part the
// arithmetic is the ring kernel's (INT4-g128 x INT8: exact int32 group sums,
// each scaled and added in group order), so the result is the ring kernel's
// with the fp32 sum over groups associated by parts.
template <int F, int kCH> struct LK {
    static constexpr int kBM = 32;
    static constexpr int kATile = kBM * kRowBytes;
    static constexpr int kBTile = kBN * FmtTraits<F>::bRow;
    static constexpr int kStage = kATile + kBTile;
    static constexpr int kTabBytes = kMaxG128Groups * kBN * 3;  // fp16 scales + u8 zero points [group][column]
    static constexpr int kFit = (160 * 1024 - kTabBytes) / (4 * kStage);
    static constexpr int kS = kFit > 4 ? 4 : kFit;
    static constexpr int kPart = kS * kStage;  // one K-part's ring
    static constexpr int kTab = 4 * kPart;
    static constexpr int kBytes = kTab + kTabBytes;
    static constexpr int kBLoads = kBTile / 1024;
    static constexpr int kThreads = 256 * kCH;
    static constexpr int kAW = 4 / kCH, kBW = kBLoads / kCH;  // a wave's share of a stage's loads
    static constexpr int kOps = kAW + kBW;                    // direct-to-LDS loads per wave and stage
    static constexpr int kRed = 16 * 64 * 64;     // partials [quarter][part][block][lane] x 4 floats
    static_assert(kS >= 2 && kS <= 4 && kBytes <= 160 * 1024 && kRed <= kTab && kBLoads % kCH == 0, "split-K layout");
};

template <int F, int E, int kCH>
__global__ __launch_bounds__(256 * kCH, 1) void gemm3_splitk_kernel(GemmArgs p) {
    static_assert(F == FMT_G128A8 || F == FMT_G128A16, "group-wise INT4 formats");
    using T = FmtTraits<F>;
    using L = LK<F, kCH>;
    constexpr int kNB = 4 / (kCH / 2);  // 16-column blocks per wave (64 or 32 columns)
    constexpr int kS = L::kS;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kp = wave & 3, ch = wave >> 2;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBN - 1) / kBN;
    const int tiles_m = (p.m + L::kBM - 1) / L::kBM;
    const int tile = blockIdx.x;
    if (tile >= tiles_m * tiles_n) return;
    const int m0 = (tile % tiles_m) * L::kBM, n0 = (tile / tiles_m) * kBN;
    const size_t lda = (size_t)p.k * T::aElemNum / T::aElemDen;
    const size_t ldb = (size_t)p.k * T::bNum / T::bDen;
    const int steps = p.k / T::kStep;
    const int groups = p.k >> 7;
    // this part's K-steps (wave-uniform: the loads' global base is a scalar
    // operand); part sizes differ by at most one, and every wave runs the
    // longest part's iteration count so that all 8 meet at every barrier
    const int s0 = __builtin_amdgcn_readfirstlane(steps * kp / 4);
    const int ns = __builtin_amdgcn_readfirstlane(steps * (kp + 1) / 4) - s0;
    const int nmax = (steps + 3) / 4;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const uint32_t ring = lds_base + (uint32_t)(kp * L::kPart);
    uint16_t* tab_s = (uint16_t*)(lds + L::kTab);
    uint8_t* tab_z = lds + L::kTab + kMaxG128Groups * kBN * 2;

    // this wave's half of a stage: activation loads 2 half + i (tile rows
    // 8 (2 half + i) + lane / 8, 16-byte chunk position lane % 8 holding source
    // chunk position ^ swz_key(row)); weight loads kBLoads / 2 * half + i as
    // the ring kernel's
    constexpr int kAW = L::kAW, kHB = L::kBW;
    uint32_t a_off[kAW], b_off[kHB];
#pragma unroll
    for (int i = 0; i < kAW; ++i) {
        const int r = 8 * (kAW * ch + i) + (lane >> 3);
        a_off[i] = (uint32_t)min(m0 + r, p.m - 1) * (uint32_t)lda + (uint32_t)((((lane & 7) ^ swz_key(r))) << 4);
    }
#pragma unroll
    for (int i = 0; i < kHB; ++i) {
        const int o = (kHB * ch + i) * 1024 + lane * 16;
        int row, c;
        if constexpr (F == FMT_G128A8) {
            row = o >> 6;
            c = ((o >> 4) & 3) ^ g128a8_key(row);
        } else if constexpr (F == FMT_G128A16) {
            a16_chunk_of_slot(o >> 4, row, c);
        } else {
            row = o / T::bRow;
            c = (o % T::bRow) / 16;
        }
        b_off[i] = (uint32_t)min(n0 + row, p.n - 1) * (uint32_t)ldb + (uint32_t)(c * 16);
    }
    auto issue = [&](int j) {
        const int step = s0 + j;
        const uint32_t base = ring + (uint32_t)((j % kS) * L::kStage);
#pragma unroll
        for (int i = 0; i < kAW; ++i) dma16(p.a + (size_t)step * kRowBytes, a_off[i], base + (kAW * ch + i) * 1024);
#pragma unroll
        for (int i = 0; i < kHB; ++i)
            dma16(p.b + (size_t)step * T::bRow, b_off[i], base + L::kATile + (kHB * ch + i) * 1024);
    };
    const int pre = min(kS - 1, ns);
    for (int j = 0; j < pre; ++j) issue(j);
    load_group_tables<uint16_t, L::kThreads>(p, n0, groups, tab_s, tab_z, tid);

    // this wave's columns: 64-column half cw, blocks bj0 .. bj0 + kNB - 1 of it
    const int cw = kCH == 2 ? ch : ch >> 1, bj0 = kCH == 2 ? 0 : (ch & 1) * 2;
    v4f accf[2][kNB];
    v4i acci[2][kNB];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < kNB; ++c) {
            accf[i][c] = v4f{0.f, 0.f, 0.f, 0.f};
            acci[i][c] = v4i{0, 0, 0, 0};
        }
    for (int j = 0; j < nmax; ++j) {
        if (j < ns) {
            switch (min(j + kS - 2, ns - 1) - j) {  // younger stages still loading: 0 .. kS - 2 <= 2
            case 0: wait_vm<0>(); break;
            case 1: wait_vm<L::kOps>(); break;
            default: wait_vm<2 * L::kOps>(); break;
            }
        }
        __syncthreads();  // the partner's half of stage j has landed; slot j - 1 is free (and, at j = 0, the tables)
        if (j >= ns) continue;
        if (j + kS - 1 < ns) issue(j + kS - 1);
        const uint8_t* As = lds + kp * L::kPart + (j % kS) * L::kStage;
        const uint8_t* Bs = As + L::kATile;
        const int grp = ((s0 + j) * T::kStep) >> 7;
        const uint16_t* ts = tab_s + grp * kBN;
        const uint8_t* tz = tab_z + grp * kBN;
        uint4 x0[2], x1[2];
#pragma unroll
        for (int rw = 0; rw < 2; ++rw) {
            x0[rw] = *(const uint4*)(As + swz(rw * 16 + l16, g));
            x1[rw] = *(const uint4*)(As + swz(rw * 16 + l16, 4 + g));
        }
#pragma unroll
        for (int b = 0; b < kNB; ++b) {
            const int bj = bj0 + b;
            const int row = cw * 64 + wrow(l16, bj);
            const uint32_t z = tz[row];
            uint4 w0, w1;
            v4f gs = v4f{1.f, 1.f, 1.f, 1.f};
            if constexpr (F == FMT_G128A8) {
                const uint2 sc = *(const uint2*)(ts + cw * 64 + g * 16 + bj * 4);  // 4 fp16 scales, one read
                gs = v4f{h2f((uint16_t)(sc.x & 0xffffu)), h2f((uint16_t)(sc.x >> 16)), h2f((uint16_t)(sc.y & 0xffffu)),
                         h2f((uint16_t)(sc.y >> 16))};
                const uint32_t zz = z * 0x01010101u;
                const int key = g128a8_key(row), hb = (g & 1) << 3;
                const uint2 q0 = *(const uint2*)(Bs + row * 64 + ((((g >> 1)) ^ key) << 4) + hb);
                const uint2 q1 = *(const uint2*)(Bs + row * 64 + (((2 + (g >> 1)) ^ key) << 4) + hb);
                u4x8_minus_z(q0.x, zz, w0.x, w0.y);
                u4x8_minus_z(q0.y, zz, w0.z, w0.w);
                u4x8_minus_z(q1.x, zz, w1.x, w1.y);
                u4x8_minus_z(q1.y, zz, w1.z, w1.w);
            } else {
                const _Float16 sh = __builtin_bit_cast(_Float16, ts[row]);
                const _Float16 zh = (_Float16)(1024 + (int)z);
                const v2h ss = {sh, sh}, zzh = {zh, zh};
                const uint32_t q0 = *(const uint32_t*)(Bs + a16_slot(row, 0) * 16 + 4 * g);
                const uint32_t q1 = *(const uint32_t*)(Bs + a16_slot(row, 1) * 16 + 4 * g);
                w0 = __builtin_bit_cast(uint4, u4x8_to_h(q0, zzh, ss));
                w1 = __builtin_bit_cast(uint4, u4x8_to_h(q1, zzh, ss));
            }
#pragma unroll
            for (int rw = 0; rw < 2; ++rw) mfma_step<F>(accf[rw][b], acci[rw][b], w0, w1, x0[rw], x1[rw], gs);
        }
    }

    __syncthreads();  // every wave is done with its ring
    // [quarter][part][block][lane] float4: consecutive lanes write consecutive 16 bytes
    float4* red = (float4*)lds;
#pragma unroll
    for (int rw = 0; rw < 2; ++rw)
#pragma unroll
        for (int b = 0; b < kNB; ++b) {
            const v4f v = accf[rw][b];
            red[(((rw * 2 + cw) * 4 + kp) * 4 + bj0 + b) * 64 + lane] = float4{v[0], v[1], v[2], v[3]};
        }
    __syncthreads();
    if (wave >= 4) return;
    v4f sum[1][4];
    v4i isum[1][4];
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
        const float4 a0 = red[((wave * 4 + 0) * 4 + bj) * 64 + lane];
        const float4 a1 = red[((wave * 4 + 1) * 4 + bj) * 64 + lane];
        const float4 a2 = red[((wave * 4 + 2) * 4 + bj) * 64 + lane];
        const float4 a3 = red[((wave * 4 + 3) * 4 + bj) * 64 + lane];
        sum[0][bj] = v4f{((a0.x + a1.x) + a2.x) + a3.x, ((a0.y + a1.y) + a2.y) + a3.y, ((a0.z + a1.z) + a2.z) + a3.z,
                         ((a0.w + a1.w) + a2.w) + a3.w};
        isum[0][bj] = v4i{0, 0, 0, 0};
    }
    if constexpr (E == EPI_F16_RES) epilogue<F, EPI_F16, true, 1>(p, sum, isum, m0, n0, wave >> 1, wave & 1, lane);
    else epilogue<F, E, false, 1>(p, sum, isum, m0, n0, wave >> 1, wave & 1, lane);
}

}  // namespace g3
}  // namespace pk
