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

// INT8 2:4 contract's weight tile: weight row r of the tile lives in LDS slot
// (r & 3) * 32 + r / 4 with its 16-byte chunks XOR-keyed by (slot >> 1) & 7, so
// the 16 lanes of a fragment read (rows 4 l16 + bj) hit 16 distinct 16-byte
// bank groups (alternating slot parity x 8 keys).
__device__ __forceinline__ int sp8w_slot(int row) { return ((row & 3) << 5) | (row >> 2); }
__device__ __forceinline__ int sp8w_row(int slot) { return ((slot & 31) << 2) | (slot >> 5); }
__device__ __forceinline__ int sp8w(int row, int chunk) {
    const int slot = sp8w_slot(row);
    return slot * 128 + ((chunk ^ ((slot >> 1) & 7)) << 4);
}

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

// ---- exact 2:4 INT8 FF contract (activation-sparse FF2) ------------------
//
// Activations arrive as the 2:4 form of their INT8 rows (data [M x K/2],
// metadata [M x K/8], the layout above) plus per-row overflow lists holding
// the nonzeros the 2:4 selection dropped (quantize_rows_sp24_kernel).  The
// contract runs v_smfmac_i32_16x16x128_i8 on the 2:4 part (activations sparse
// first operand, INT8 weights dense second operand, operand layouts as in the
// FP8 kernel above) and adds each overflow entry's products to the int32
// accumulators before the epilogue, so the accumulators are the exact dense
// INT8 dot products and the fp32 output, (acc * input_scale[r]) *
// weight_scale[n], equals the dense INT8 contract's bit for bit.
//
// Workgroup: 2 kWM waves (kWM along M x 2 along N), tile (16 kAI kWM) x 128,
// wave (16 kAI) x 64 = kAI x 4 blocks of 16 x 16.  The launcher runs kAI = 4:
// 256-row tiles of 8 waves (kWM = 4), one workgroup per CU, a 4-stage LDS ring
// of 36 KiB stages, where those tiles give at least half the CUs one, else
// 128-row tiles of 4 waves, two workgroups per CU, a 3-stage ring of 26 KiB
// stages (256-row tiles of 4 waves, 128 x 64 each, measured 15-20 % slower).  A stage holds one 128-K step: compressed data (64
// bytes a row), metadata (16 bytes a row) and the weight tile (128 rows x 128
// bytes); its direct-to-LDS loads have kS - 1 steps to land, and there is one
// barrier per step.  Blocks are laid out so that the column tiles of one row
// strip run on the same XCD (blocks b, b + 8, ... share b % 8) and share that
// strip's activations in L2.
//
// Overflow: after the K-loop the ring is free.  The tile's per-row counts are
// scanned into offsets; in chunks, the entries (value and tile row) and, for
// each, the 128 bytes of its weight column for the tile's columns (a row of
// the transposed weights W^T [K x N], direct-to-LDS) are staged in LDS; each
// lane then walks the entries of its rows and adds v * W[n, k] to the
// accumulators of its 4 columns.  When the producer also wrote the residual
// 2:4 form (the two positions of each quartet the selection did not keep),
// tiles with many entries run the K-loop a second time on it instead.
template <int kAI, int kWM = 2> struct Sp8 {
    static constexpr int kRows = 16 * kAI * kWM;   // tile rows: kWM waves along M, each kAI blocks of 16
    static constexpr int kWaves = 2 * kWM, kThreads = 64 * kWaves;
    static constexpr int kOcc = kRows <= 128 ? 2 : 1;  // workgroups per CU
    static constexpr int kData = kRows * 64, kMeta = kRows * 16, kW = 128 * 128;
    static constexpr int kStage = kData + kMeta + kW;
    static constexpr int kFit = (kOcc == 2 ? 80 : 150) * 1024 / kStage;
    static constexpr int kS = kFit > 4 ? 4 : kFit;
    static constexpr int kLds = kS * kStage;
    static constexpr int kWLoads = 16 / kWaves;     // 1 KiB weight loads per wave and stage
    static constexpr int kOps = kAI / 2 + 1 + kWLoads;  // direct-to-LDS loads per wave and stage
    static constexpr int kMetaLanes = 8 * kAI;     // metadata rows per wave
    // overflow staging inside the ring: counts, offsets (+ wave totals), entries
    // (tile row and byte; then k), weight rows
    static constexpr int kChunk = kOcc == 1 ? 1024 : 512;
    static constexpr int kCnt = 0, kOff = kRows * 4, kEnt = kOff + (kRows + 8) * 4, kWt = kEnt + 8 * kChunk;
    static_assert(kS >= 3 && kWt + kChunk * 128 <= kLds, "overflow staging fits the ring");
    static_assert(kLds * kOcc <= 160 * 1024 && kMetaLanes <= 64 && 16 % kWaves == 0, "layout");
};

struct Sparse8Args {
    const uint8_t* data;        // [M x K/2]
    const uint8_t* meta;        // [M x K/8]
    const float* in_scales;     // [M]
    const uint32_t* ovf_count;  // [M]
    const uint32_t* ovf;        // [M x K/2]
    const uint8_t* data2;       // [M x K/2] residual 2:4 form, or null
    const uint8_t* meta2;       // [M x K/8]
    const int8_t* w;            // [N x K]
    const int8_t* wt;           // [K x N]
    const float* w_scales;      // [N]
    float* out;                 // [M x N]
    int m, n, k;
};

template <int N> __device__ __forceinline__ void sp8_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
// vmcnt(kOps * younger) for younger = 0 .. 3 stages still loading
template <int kOps> __device__ __forceinline__ void sp8_wait_stages(int younger) {
    switch (younger) {
    case 0: sp8_wait<0>(); break;
    case 1: sp8_wait<kOps>(); break;
    case 2: sp8_wait<2 * kOps>(); break;
    default: sp8_wait<3 * kOps>(); break;
    }
}

constexpr int kResidualPerRow = 8;

template <int kAI, int kWM>
__global__ __launch_bounds__((Sp8<kAI, kWM>::kThreads), (Sp8<kAI, kWM>::kOcc)) void sparse24_i8_kernel(Sparse8Args p) {
    using L = Sp8<kAI, kWM>;
    constexpr int kS = L::kS;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, l16 = lane & 15;
    const int tiles_n = p.n >> 7;
    const int tiles_m = (p.m + L::kRows - 1) / L::kRows;
    // block b runs on XCD x = b % 8; that XCD's j-th block is column tile
    // j % tiles_n of row strip 8 (j / tiles_n) + x (measured: giving each XCD
    // a column group instead, so that its weight slice stays in L2, changed
    // the time by < 4 %)
    const int b = blockIdx.x, x = b & 7, j = b >> 3;
    const int tm = (j / tiles_n) * 8 + x, tn = j % tiles_n;
    if (tm >= tiles_m) return;
    const int m0 = tm * L::kRows, n0 = tn * 128;
    const int steps = p.k >> 7;
    const size_t ld_data = (size_t)p.k >> 1, ld_meta = (size_t)p.k >> 3;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;

    // direct-to-LDS sources: kAI / 2 data loads (16 rows x 64 bytes each), one
    // metadata load (8 kAI rows x 16 bytes), kWLoads weight loads (8 rows x 128 bytes)
    uint32_t d_off[kAI / 2], w_off[L::kWLoads];
#pragma unroll
    for (int i = 0; i < kAI / 2; ++i) {
        const int o = (wave * (kAI / 2) + i) * 1024 + lane * 16;
        const int row = o >> 6, c = ((o >> 4) & 3) ^ sp_key(row);
        d_off[i] = (uint32_t)((size_t)min(m0 + row, p.m - 1) * ld_data + c * 16);
    }
    const uint32_t m_off = (uint32_t)((size_t)min(m0 + wave * L::kMetaLanes + (lane % L::kMetaLanes), p.m - 1) * ld_meta);
#pragma unroll
    for (int i = 0; i < L::kWLoads; ++i) {
        const int o = (wave * L::kWLoads + i) * 1024 + lane * 16;
        const int slot = o >> 7, c = ((o >> 4) & 7) ^ ((slot >> 1) & 7);
        w_off[i] = (uint32_t)((size_t)(n0 + sp8w_row(slot)) * p.k + c * 16);
    }
    const uint8_t* src_d = p.data;  // the 2:4 form the K-loop reads: the kept pairs, then (residual pass) the rest
    const uint8_t* src_m = p.meta;
    auto issue = [&](int step) {
        const uint32_t base = lds_base + (uint32_t)((step % kS) * L::kStage);
#pragma unroll
        for (int i = 0; i < kAI / 2; ++i) dma16(src_d + d_off[i] + (size_t)step * 64, base + (wave * (kAI / 2) + i) * 1024);
        if (lane < L::kMetaLanes) dma16(src_m + m_off + (size_t)step * 16, base + L::kData + wave * L::kMetaLanes * 16);
#pragma unroll
        for (int i = 0; i < L::kWLoads; ++i)
            dma16(p.w + w_off[i] + (size_t)step * 128, base + L::kData + L::kMeta + (wave * L::kWLoads + i) * 1024);
    };

    v4i acc[kAI][4];
#pragma unroll
    for (int i = 0; i < kAI; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = v4i{0, 0, 0, 0};

    auto kloop = [&]() {
        const int pre = min(kS - 1, steps);
        for (int st = 0; st < pre; ++st) issue(st);
        for (int step = 0; step < steps; ++step) {
            // stage `step` has landed once only the younger stages' loads are pending
            sp8_wait_stages<L::kOps>(min(step + kS - 2, steps - 1) - step);
            __syncthreads();
            if (step + kS - 1 < steps) issue(step + kS - 1);
            const uint8_t* Ds = lds + (step % kS) * L::kStage;
            const uint8_t* Ms = Ds + L::kData;
            const uint8_t* Ws = Ms + L::kMeta;
            v8i wf[4];
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                const int row = wn * 64 + 4 * l16 + bj;
                const uint4 w0 = *(const uint4*)(Ws + sp8w(row, g));
                const uint4 w1 = *(const uint4*)(Ws + sp8w(row, 4 + g));
                wf[bj] = v8i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
            }
#pragma unroll
            for (int ai = 0; ai < kAI; ++ai) {
                const int row = wm * 16 * kAI + ai * 16 + l16;
                const uint4 d = *(const uint4*)(Ds + row * 64 + ((g ^ sp_key(row)) << 4));
                const int idx = *(const int*)(Ms + row * 16 + g * 4);
                const v4i dv = {(int)d.x, (int)d.y, (int)d.z, (int)d.w};
#pragma unroll
                for (int bj = 0; bj < 4; ++bj) acc[ai][bj] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(dv, wf[bj], acc[ai][bj], idx, 0, 0);
            }
        }
        __syncthreads();  // every wave is done with the ring
    };
    kloop();

    // ---- overflow entries of the tile's rows ----
    uint32_t* cnt_s = (uint32_t*)(lds + L::kCnt);
    uint32_t* off_s = (uint32_t*)(lds + L::kOff);
    uint32_t* ent_s = (uint32_t*)(lds + L::kEnt);
    const size_t cap = (size_t)p.k >> 1;
    uint32_t incl = 0;  // inclusive scan of the counts within each wave (thread = tile row)
    if (tid < L::kRows) {
        const uint32_t c = m0 + tid < p.m ? p.ovf_count[m0 + tid] : 0u;
        cnt_s[tid] = c;
        incl = c;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t u = (uint32_t)__shfl_up((int)incl, d, 64);
            if (lane >= d) incl += u;
        }
        if (lane == 63) off_s[L::kRows + 1 + wave] = incl;  // wave totals
    }
    __syncthreads();
    if (tid < L::kRows) {
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += off_s[L::kRows + 1 + w];
        off_s[tid + 1] = before + incl;
        if (tid == 0) off_s[0] = 0;
    }
    __syncthreads();
    const uint32_t total = off_s[L::kRows];
    // Tiles with more than kResidualPerRow overflow entries per row take the
    // residual 2:4 form through a second K-loop instead of the entry lists:
    // its cost is one more pass over K, the lists' grows with every entry
    // (T = 7500: the lists add about 2.6 us per entry per row, the second pass
    // about 21 us, so they meet near 8 entries per row).
    const bool residual = p.data2 != nullptr && total > (uint32_t)(kResidualPerRow * L::kRows);
    if (residual) {
        src_d = p.data2;
        src_m = p.meta2;
        __syncthreads();  // every thread has read the offsets before the ring is reused
        kloop();
    }
    for (uint32_t c0 = 0; !residual && c0 < total; c0 += L::kChunk) {
        const int len = (int)min((uint32_t)L::kChunk, total - c0);
        // stage entries as (tile row << 8) | byte; issue the weight-row loads
        // straight from the global entries (k = entry >> 8)
        for (int e = tid; e < len; e += L::kThreads) {
            const uint32_t gi = c0 + (uint32_t)e;
            int lo = 0, hi = L::kRows - 1;  // last row r with off[r] <= gi
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (off_s[mid] <= gi) lo = mid;
                else hi = mid - 1;
            }
            const uint32_t en = p.ovf[(size_t)(m0 + lo) * cap + (gi - off_s[lo])];
            ent_s[e] = (uint32_t)lo << 8 | (en & 255u);
            ent_s[L::kChunk + e] = en >> 8;  // k, read back by the weight-row loads below
        }
        __syncthreads();
        for (int blk = wave; blk * 8 < len; blk += L::kWaves) {
            const int e = min(blk * 8 + (lane >> 3), len - 1);
            const uint32_t kk = ent_s[L::kChunk + e];
            dma16(p.wt + (size_t)kk * p.n + n0 + (lane & 7) * 16, lds_base + L::kWt + blk * 1024);
        }
        sp8_wait<0>();
        __syncthreads();
#pragma unroll
        for (int ai = 0; ai < kAI; ++ai)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wm * 16 * kAI + ai * 16 + 4 * g + r;
                const int beg = (int)(max(off_s[row], c0) - c0);
                const int end = (int)(min(off_s[row + 1], c0 + (uint32_t)len) - c0);
                for (int e = beg; e < end; ++e) {
                    const int v = (int)(int8_t)(ent_s[e] & 255u);
                    const uint32_t w4 = *(const uint32_t*)(lds + L::kWt + e * 128 + wn * 64 + 4 * l16);
#pragma unroll
                    for (int bj = 0; bj < 4; ++bj) acc[ai][bj][r] += v * (int)(int8_t)(w4 >> (8 * bj));
                }
            }
        __syncthreads();
    }

    // ---- epilogue: rows 4g + r of each block, columns 4 l16 .. + 3 ----
    const int gcol = n0 + wn * 64 + 4 * l16;
    const float4 ws = *(const float4*)(p.w_scales + gcol);
#pragma unroll
    for (int ai = 0; ai < kAI; ++ai)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int grow = m0 + wm * 16 * kAI + ai * 16 + 4 * g + r;
            if (grow >= p.m) continue;
            const float rs = p.in_scales[grow];
            *(float4*)(p.out + (size_t)grow * p.n + gcol) =
                float4{__builtin_fmaf((float)acc[ai][0][r] * rs, ws.x, 0.0f), __builtin_fmaf((float)acc[ai][1][r] * rs, ws.y, 0.0f),
                       __builtin_fmaf((float)acc[ai][2][r] * rs, ws.z, 0.0f), __builtin_fmaf((float)acc[ai][3][r] * rs, ws.w, 0.0f)};
        }
}

template <int kAI, int kWM>
static int launch_sp8(const Sparse8Args& a, hipStream_t s) {
    using L = Sp8<kAI, kWM>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] { attr = hipFuncSetAttribute((const void*)sparse24_i8_kernel<kAI, kWM>, hipFuncAttributeMaxDynamicSharedMemorySize, L::kLds); });
    if (attr != hipSuccess) {
        set_error("hipFuncSetAttribute failed: %s", hipGetErrorString(attr));
        return -3;
    }
    const int tiles_m = (a.m + L::kRows - 1) / L::kRows, tiles_n = a.n / 128;
    const int grid = 8 * ((tiles_m + 7) / 8) * tiles_n;
    hipLaunchKernelGGL((sparse24_i8_kernel<kAI, kWM>), dim3(grid), dim3(L::kThreads), L::kLds, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("sparse INT8 contract launch failed: %s", hipGetErrorString(e));
        return -3;
    }
    return 0;
}

int launch_sparse24_i8_contract(const uint8_t* data, const uint8_t* meta, const float* in_scales, const uint32_t* ovf_count,
                                const uint32_t* ovf, const uint8_t* data2, const uint8_t* meta2, const int8_t* w, const int8_t* wt,
                                const float* w_scales, float* out, int m, int n, int k, hipStream_t s) {
    if (m == 0) return 0;
    if (n <= 0 || k <= 0 || n % 128 != 0 || k % 128 != 0 || k > (1 << 24)) {
        set_error("sparse INT8 contract: n and k must be positive multiples of 128 (k <= 2^24), got n=%d k=%d", n, k);
        return -1;
    }
    if (((uintptr_t)data | (uintptr_t)meta | (uintptr_t)data2 | (uintptr_t)meta2 | (uintptr_t)w | (uintptr_t)wt | (uintptr_t)w_scales |
         (uintptr_t)out) & 15) {
        set_error("sparse INT8 contract: data, meta, residual data / meta, weight, weight_t, weight_scales and output must be 16-byte aligned");
        return -2;
    }
    if ((data2 == nullptr) != (meta2 == nullptr)) {
        set_error("sparse INT8 contract: residual data and metadata go together");
        return -1;
    }
    if (((size_t)m * (size_t)(k / 2)) >> 32 || ((size_t)n * (size_t)k) >> 32) {
        set_error("sparse INT8 contract: operands past 4 GiB are not supported");
        return -1;
    }
    const Sparse8Args a{data, meta, in_scales, ovf_count, ovf, data2, meta2, w, wt, w_scales, out, m, n, k};
    // 256-row tiles of 8 waves, one workgroup per CU and a 4-stage ring, where
    // they give at least half the CUs a tile (T = 7500: 41.5 -> 39.4 us at 95 %
    // sparsity); smaller grids keep 128-row tiles two per CU
    const long tiles256 = (long)((m + 255) / 256) * (n / 128);
    return 2 * tiles256 >= cu_count() ? launch_sp8<4, 4>(a, s) : launch_sp8<4, 2>(a, s);
}

// W [n x k] int8 -> W^T [k x n] (load-time derivation for the overflow pass).
__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ w, int8_t* __restrict__ wt, int n, int k) {
    __shared__ int8_t tile[64][65];
    const int k0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4)
        if (n0 + r < n && k0 + tx < k) tile[r][tx] = w[(size_t)(n0 + r) * k + k0 + tx];
    __syncthreads();
    for (int r = ty; r < 64; r += 4)
        if (k0 + r < k && n0 + tx < n) wt[(size_t)(k0 + r) * n + n0 + tx] = tile[tx][r];
}

int launch_transpose_i8(const int8_t* w, int8_t* wt, int n, int k, hipStream_t s) {
    if (n <= 0 || k <= 0) return 0;
    hipLaunchKernelGGL(transpose_i8_kernel, dim3((k + 63) / 64, (n + 63) / 64), dim3(256), 0, s, w, wt, n, k);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("transpose launch failed: %s", hipGetErrorString(e));
        return -3;
    }
    return 0;
}

}  // namespace pk
