// FF contract on 2:4-compressed FP8 activations (encoder.cu:1087-1095,
// epilogue 8): out (fp16, in place) = fp16(fma(0.5, acc * (1/16) * w_scale, out)).
//
// The activations are the sparse first operand of v_smfmac_f32_16x16x128_fp8_fp8
// (16 compressed bytes + one 32-bit index word per lane), the FP8 weights the
// dense second operand.  With the dense operand laid out as in the GEMM engine
// (lane group g holds weight bytes [16g, 16g+16) and [64+16g, +16) of the
// 128-K step), lane group g of the sparse operand covers the logical K range
// [32g, 32g+32): exactly the reference's compressed bytes [16g, 16g+16) of the
// step and its metadata word g (quartet j's idx0 | idx1 << 2 at bits 4j), so
// the reference's 2:4 rows are consumed as they are stored.
//
// Workgroup tile 256 x 256 (8 waves, 128 x 64 each), persistent over tiles,
// direct-to-LDS loads, double-buffered stages of 16 KiB compressed data +
// 4 KiB metadata + 32 KiB weights.  Weight row n(j, bj) = 4j + bj feeds MFMA
// column j of block bj, so each lane's accumulators for one 16-row block are
// 4 rows x 4 contiguous output columns.
#include "pk_kernels.hpp"

namespace pk {

constexpr int kSpData = 256 * 64;     // compressed activation bytes per stage
constexpr int kSpMeta = 256 * 16;     // metadata bytes per stage
constexpr int kSpW = 256 * 128;       // weight bytes per stage
constexpr int kSpStage = kSpData + kSpMeta + kSpW;

// XOR key of a 64-byte compressed row's 16-byte chunks: 8 (16) consecutive
// rows reading one chunk column touch distinct banks of 128 (256) bytes.
__device__ __forceinline__ int sp_key(int row) { return ((row >> 1) & 2) | (((row >> 1) ^ (row >> 3)) & 1); }
// XOR key of a 128-byte weight row's chunks for the rows 4i + bj that lanes
// i = 0..15 read: distinct for every 8 lanes (16 lanes share each bank pair).
__device__ __forceinline__ int spw_key(int row) { return (row >> 2) & 7; }
__device__ __forceinline__ int spw(int row, int chunk) { return row * 128 + ((chunk ^ spw_key(row)) << 4); }

struct SparseArgs {
    const uint8_t* data;    // [M x K/2]
    const uint8_t* meta;    // [M x K/8]
    const uint8_t* w;       // [N x K] e4m3
    const float* w_scales;  // [N]
    float in_scale;
    uint16_t* out;          // [M x N] fp16, residual in place
    int m, n, k;
};

__global__ __launch_bounds__(kThreads, 1) void sparse24_contract_kernel(SparseArgs p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = (p.n + kBlockN - 1) / kBlockN;
    const int tiles_m = (p.m + kBlockM - 1) / kBlockM;
    const int ntiles = tiles_m * tiles_n;
    const int G = gridDim.x;
    const int steps = p.k >> 7;
    const size_t ld_data = (size_t)p.k >> 1, ld_meta = (size_t)p.k >> 3, ld_w = (size_t)p.k;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;

    // Per-lane source offsets of this wave's direct-to-LDS loads: compressed
    // data (2 KiB per wave, 64-byte rows, 16-byte chunks swizzled by sp_key),
    // metadata (waves 0-3, 1 KiB each, 16-byte rows), weights (4 KiB per wave,
    // 128-byte rows swizzled by spw_key).
    uint32_t d_off[2], m_off = 0, w_off[4];
    const int gw = group_width(tiles_n);
    auto set_tile = [&](int t, int& m0, int& n0) {
        const int ng = t / (tiles_m * gw);
        const int r = t - ng * tiles_m * gw;
        const int tm = r / gw;
        m0 = tm * kBlockM;
        n0 = (ng * gw + (r - tm * gw)) * kBlockN;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int o = (wave * 2 + i) * 1024 + lane * 16;
            const int row = o >> 6, c = ((o >> 4) & 3) ^ sp_key(row);
            d_off[i] = (uint32_t)((size_t)min(m0 + row, p.m - 1) * ld_data + c * 16);
        }
        {
            const int o = (wave & 3) * 1024 + lane * 16;
            m_off = (uint32_t)((size_t)min(m0 + (o >> 4), p.m - 1) * ld_meta);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (wave * 4 + i) * 1024 + lane * 16;
            const int row = o >> 7, c = ((o >> 4) & 7) ^ spw_key(row);
            w_off[i] = (uint32_t)((size_t)min(n0 + row, p.n - 1) * ld_w + c * 16);
        }
    };
    auto issue = [&](int step, int buf) {
        const uint32_t base = lds_base + buf * kSpStage;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16(p.data + d_off[i] + (size_t)step * 64, base + (wave * 2 + i) * 1024);
        if (wave < 4) dma16(p.meta + m_off + (size_t)step * 16, base + kSpData + wave * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(p.w + w_off[i] + (size_t)step * 128, base + kSpData + kSpMeta + (wave * 4 + i) * 1024);
    };

    int t = tile_slot(G);
    if (t >= ntiles) return;
    int m0, n0;
    set_tile(t, m0, n0);
    issue(0, 0);
    int buf = 0;
    v4f acc[8][4];

    while (true) {
        const int t_next = t + G;
        const int cur_m0 = m0, cur_n0 = n0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

        for (int step = 0; step < steps; ++step) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (step + 1 < steps) {
                issue(step + 1, buf ^ 1);
            } else if (t_next < ntiles) {
                set_tile(t_next, m0, n0);
                issue(0, buf ^ 1);
            }
            const uint8_t* Ds = lds + buf * kSpStage;
            const uint8_t* Ms = Ds + kSpData;
            const uint8_t* Ws = Ms + kSpMeta;
            v8i wf[4];
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int row = wn * 64 + 4 * l16 + bj;
                const uint4 w0 = *(const uint4*)(Ws + spw(row, g));
                const uint4 w1 = *(const uint4*)(Ws + spw(row, 4 + g));
                wf[bj] = v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
            }
#pragma unroll
            for (int ai = 0; ai < 8; ++ai) {
                const int row = wm * 128 + ai * 16 + l16;
                const uint4 d = *(const uint4*)(Ds + row * 64 + ((g ^ sp_key(row)) << 4));
                const int idx = *(const int*)(Ms + row * 16 + g * 4);
                const v4i dv = {(int)d.x, (int)d.y, (int)d.z, (int)d.w};
#pragma unroll
                for (int bj = 0; bj < 4; ++bj) acc[ai][bj] = __builtin_amdgcn_smfmac_f32_16x16x128_fp8_fp8(dv, wf[bj], acc[ai][bj], idx, 0, 0);
            }
            buf ^= 1;
        }

        // Epilogue: lane holds rows 4g + r of each 16-row block and columns
        // [4 l16, 4 l16 + 4) of the wave's 64.
        const int gcol = cur_n0 + wn * 64 + 4 * l16;
        const bool col_live = gcol < p.n;
        const float4 ws = *(const float4*)(p.w_scales + min(gcol, p.n - 4));
        const float wsv[4] = {ws.x, ws.y, ws.z, ws.w};
#pragma unroll
        for (int ai = 0; ai < 8; ++ai) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int grow = cur_m0 + wm * 128 + ai * 16 + 4 * g + r;
                if (grow >= p.m || !col_live) continue;
                uint16_t* o = p.out + (size_t)grow * p.n + gcol;
                const uint2 res = *(const uint2*)o;
                const float r0 = h2f((uint16_t)(res.x & 0xffff)), r1 = h2f((uint16_t)(res.x >> 16));
                const float r2 = h2f((uint16_t)(res.y & 0xffff)), r3 = h2f((uint16_t)(res.y >> 16));
                const float v0 = acc[ai][0][r] * p.in_scale * wsv[0], v1 = acc[ai][1][r] * p.in_scale * wsv[1];
                const float v2 = acc[ai][2][r] * p.in_scale * wsv[2], v3 = acc[ai][3][r] * p.in_scale * wsv[3];
                *(uint2*)o = uint2{(uint32_t)f2h(__builtin_fmaf(0.5f, v0, r0)) | ((uint32_t)f2h(__builtin_fmaf(0.5f, v1, r1)) << 16),
                                   (uint32_t)f2h(__builtin_fmaf(0.5f, v2, r2)) | ((uint32_t)f2h(__builtin_fmaf(0.5f, v3, r3)) << 16)};
            }
        }
        if (t_next >= ntiles) break;
        t = t_next;
    }
}

int launch_sparse24_contract(const uint8_t* data, const uint8_t* meta, const uint8_t* w, const float* w_scales, float in_scale,
                             uint16_t* out, int m, int n, int k, hipStream_t s) {
    if (m == 0) return 0;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)sparse24_contract_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kSpStage);
    });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute failed: %s", hipGetErrorString(attr));
        return -3;
    }
    SparseArgs a{data, meta, w, w_scales, in_scale, out, m, n, k};
    const int tiles = ((m + kBlockM - 1) / kBlockM) * ((n + kBlockN - 1) / kBlockN);
    const int cus = cu_count();
    const int grid = tiles < cus ? tiles : cus - cus % 8;
    hipLaunchKernelGGL(sparse24_contract_kernel, dim3(grid), dim3(kThreads), 2 * kSpStage, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("sparse contract launch failed: %s", hipGetErrorString(e));
        return -3;
    }
    return 0;
}

}  // namespace pk
