// Occupancy-2 GEMM engine for the 128-byte-row formats (FP8, INT8) on gfx950.
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
// buffer while the MFMAs run.  Loads are direct-to-LDS, whole 128-byte rows.
#pragma once

#include "pk_gemm.hpp"

namespace pk {
namespace g3 {

constexpr int kBM = 256, kBN = 128, kThreads = 256;
constexpr int kATile = kBM * kRowBytes;  // 32 KiB
constexpr int kBTile = kBN * kRowBytes;  // 16 KiB
constexpr int kB = 2 * kATile;           // weight buffer offset
constexpr int kLds = 2 * kATile + kBTile;  // 80 KiB

template <int F, int E>
__global__ __launch_bounds__(kThreads, 2) void gemm3_kernel(GemmArgs p) {
    using T = FmtTraits<F>;
    static_assert(T::bRow == 128 && T::kStep == 128, "128-byte rows, one MFMA K per step");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBN - 1) / kBN;
    const int tiles_m = (p.m + kBM - 1) / kBM;
    const int ntiles = tiles_m * tiles_n;
    const int G = gridDim.x;
    const size_t ld = (size_t)p.k;  // bytes per row (1-byte elements)
    const int steps = p.k / T::kStep;
    const uint8_t* __restrict__ pa = p.a;
    const uint8_t* __restrict__ pb = p.b;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const int gw = group_width(tiles_n);

    uint32_t a_off[8], b_off[4];
    auto set_tile = [&](int tt, int& m0, int& n0) {
        const int ng = tt / (tiles_m * gw);
        const int r = tt - ng * tiles_m * gw;
        const int tm = r / gw;
        m0 = tm * kBM;
        n0 = (ng * gw + (r - tm * gw)) * kBN;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int o = (wave * 8 + i) * 1024 + lane * 16;
            const int row = o >> 7, c = ((o >> 4) & 7) ^ swz_key(row);
            a_off[i] = (uint32_t)((size_t)min(m0 + row, p.m - 1) * ld + c * 16);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (wave * 4 + i) * 1024 + lane * 16;
            const int row = o >> 7, c = ((o >> 4) & 7) ^ swz_key(row);
            b_off[i] = (uint32_t)((size_t)min(n0 + row, p.n - 1) * ld + c * 16);
        }
    };
    auto issue_a = [&](int step, int buf) {
        const uint32_t base = lds_base + buf * kATile;
#pragma unroll
        for (int i = 0; i < 8; ++i) dma16(pa + (size_t)step * kRowBytes, a_off[i], base + (wave * 8 + i) * 1024);
    };
    auto issue_b = [&](int step) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(pb + (size_t)step * kRowBytes, b_off[i], lds_base + kB + (wave * 4 + i) * 1024);
    };

    int t = tile_slot(G);
    if (t >= ntiles) return;
    int m0, n0;
    set_tile(t, m0, n0);
    issue_a(0, 0);
    issue_b(0);
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
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            // The next step's (or next tile's first step's) activations load
            // into the other buffer, which every wave finished with last step.
            int nstep = -1;
            if (step + 1 < steps) nstep = step + 1;
            else if (t_next < ntiles) {
                set_tile(t_next, m0, n0);
                nstep = 0;
            }
            if (nstep >= 0) issue_a(nstep, buf ^ 1);
            const uint8_t* As = lds + buf * kATile;
            const uint8_t* Bs = lds + kB;
            uint4 w0[4], w1[4];
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int row = wn * 64 + wrow(l16, bj);
                w0[bj] = *(const uint4*)(Bs + swz(row, g));
                w1[bj] = *(const uint4*)(Bs + swz(row, 4 + g));
            }
            uint4 x0, x1, y0, y1;
            {
                const int row = wm * 128 + l16;
                x0 = *(const uint4*)(As + swz(row, g));
                x1 = *(const uint4*)(As + swz(row, 4 + g));
            }
            // every wave holds its weight fragments: the weight buffer is free
            __syncthreads();
            if (nstep >= 0) issue_b(nstep);
#pragma unroll
            for (int ai = 0; ai < 8; ++ai) {
                if (ai + 1 < 8) {
                    const int row = wm * 128 + (ai + 1) * 16 + l16;
                    y0 = *(const uint4*)(As + swz(row, g));
                    y1 = *(const uint4*)(As + swz(row, 4 + g));
                }
                bool live = true;
                if constexpr (F == FMT_I8_SKIP) {
                    const bool nz = (x0.x | x0.y | x0.z | x0.w | x1.x | x1.y | x1.z | x1.w) != 0u;
                    live = __builtin_amdgcn_ballot_w64(nz) != 0;
                    skipped += live ? 0u : 1u;
                }
                if (live) {
#pragma unroll
                    for (int bj = 0; bj < 4; ++bj) mfma_step<F>(accf[ai][bj], acci[ai][bj], w0[bj], w1[bj], x0, x1, v4f{1.f, 1.f, 1.f, 1.f});
                }
                x0 = y0;
                x1 = y1;
            }
            if constexpr (F == FMT_FP8 || F == FMT_I8) {
                constexpr int kMfma = F == FMT_FP8 ? 4 : 8;
#pragma unroll
                for (int ai = 0; ai < 8; ++ai) {
                    if (ai + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
                }
            }
            buf ^= 1;
        }
        blocks += 8 * steps;

        if constexpr (E == EPI_F16_RES) epilogue<F, EPI_F16, true>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
        else epilogue<F, E, false>(p, accf, acci, cur_m0, cur_n0, wm, wn, lane);
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

}  // namespace g3
}  // namespace pk
